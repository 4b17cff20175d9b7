"""Index files (jhq_save / jhq_load).  The reference has no serialization, so
parity is pinned by invariants: a reloaded index holds the same canonical
lists and trained state, searches bit-identically to the index it was saved
from, and keeps accepting appends that match the oracle's one-shot add."""
import numpy as np
import pytest

from datagen import queries_and_base
from test_gpu_parity import _bits, _stagewise
from test_gpu_streaming import _lists_equal, _pair

import jhq_gpu_amd as jg

pytestmark = pytest.mark.gpu


def _same_state(a, b):
    ca, cb = a.codebooks(), b.codebooks()
    for key in ca:
        assert np.array_equal(_bits(np.asarray(ca[key])), _bits(np.asarray(cb[key]))), key
    la, lb = a.lists(), b.lists()
    for key in la:
        assert np.array_equal(la[key], lb[key]), key
    assert a.ntotal == b.ntotal and a.params == b.params


@pytest.mark.parametrize("per_sub", [0, 1], ids=["shared_books", "per_subspace_books"])
def test_save_load_roundtrip(gpu, tmp_path, per_sub):
    d, M, nlist, nprobe, k = 64, 16, 16, 5, 10
    base, q = queries_and_base(6000, 24, d, 40, seed=611 + per_sub)
    g, o = _pair(d, M, nlist, nprobe, per_sub)
    g.train(base[:2000])
    o.train(base[:2000])
    g.add(base[:2500])
    g.append(base[2500:4000])  # lists moved: the pool has gaps
    path = tmp_path / "idx.jhq"
    g.save(path)
    h = jg.JHQGpuIndex.load(path)
    _same_state(g, h)
    used_g, _ = g.pool()
    used_h, cap_h = h.pool()
    assert used_h <= used_g and used_h <= cap_h
    d1, i1 = g.search(q, k)
    d2, i2 = h.search(q, k)
    assert np.array_equal(i1, i2) and np.array_equal(_bits(d1), _bits(d2))
    # a reloaded index keeps the one-shot add guard and accepts appends
    with pytest.raises(RuntimeError, match="one add"):
        h.add(base[:10])
    h.append(base[4000:])
    o.add(base)
    _lists_equal(h, o)
    _stagewise(h, o, q, k)
    # tunables as last set travel in the file
    h.set_nprobe(7)
    h.set_alpha(6.0)
    h.save(path)
    h2 = jg.JHQGpuIndex.load(path)
    assert h2.params.nprobe == 7 and h2.params.alpha == 6.0
    _same_state(h, h2)


def test_save_load_trained_only(gpu, tmp_path):
    """A trained, empty index reloads and then takes the one-shot add."""
    d, M, nlist, nprobe, k = 32, 8, 8, 3, 5
    base, q = queries_and_base(3000, 12, d, 16, seed=77)
    g, o = _pair(d, M, nlist, nprobe, 0)
    g.train(base[:1000])
    o.train(base[:1000])
    path = tmp_path / "trained.jhq"
    g.save(path)
    h = jg.JHQGpuIndex.load(path)
    assert h.ntotal == 0
    h.add(base)
    o.add(base)
    _lists_equal(h, o)
    _stagewise(h, o, q, k)
