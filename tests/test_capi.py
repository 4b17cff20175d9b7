"""The C-ABI library without a GPU: it loads, exports every entry point that
include/jhq.h declares, and its host-side logic (parameter validation in the
reference's order, call-order errors, the host-built JL rotation) behaves like
the reference's JHQGpuIndex (jhq_v14_streaming_add/jhq_gpu_index.cu:103-131,
417-420, 535-537).  No compute call reaches the device here."""
import ctypes
import os
import re

import numpy as np
import pytest

import pyoracle as po

import jhq_gpu_amd as jg

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    src = open(os.path.join(ROOT, "include", "jhq.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(jhq_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    syms = _declared_symbols()
    assert len(syms) >= 20
    L = ctypes.CDLL(jg.lib_path())
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    # the Python mirror binds exactly the declared entry points
    assert set(jg._SIGS) == set(syms)


def test_params_default_match_reference():
    p = jg._Params()
    jg.lib().jhq_params_default(ctypes.byref(p))
    ref = jg.Params()
    assert (p.M, p.B, p.Br, p.alpha, p.nlist, p.nprobe, p.ivf_iters, p.batch_size, p.seed,
            p.add_batch) == (ref.M, ref.B, ref.Br, ref.alpha, ref.nlist, ref.nprobe,
                             ref.ivf_iters, ref.batch_size, ref.seed, ref.add_batch)
    assert (ref.M, ref.B, ref.Br, ref.alpha, ref.nlist, ref.nprobe, ref.ivf_iters,
            ref.batch_size, ref.seed, ref.add_batch) == (96, 8, 4, 4.0, 1024, 8, 8, 256, 42, 65536)


@pytest.mark.parametrize("d,kw,msg", [
    (10, dict(M=3), "divisible by M"),
    (16, dict(M=8, B=3), "divisible by Ds"),
    (16, dict(M=1, B=16), "<= 8"),
    (16, dict(M=2, B=4), "divisible by Ds"),
    (16, dict(M=16, B=16), "<= 8"),
    (16, dict(M=8, Br=2), "Br must be 4 or 8"),
    (16, dict(M=8, nlist=0), "nlist"),
    (16, dict(M=8, nprobe=0), "nprobe"),
    (16, dict(M=8, ivf_iters=0), "ivf_iters"),
    (16, dict(M=8, batch_size=0), "batch_size"),
    (16, dict(M=8, add_batch=0), "add_batch"),
    (16, dict(M=8, alpha=0.0), "alpha"),
    (0, dict(M=8), "d must be positive"),
    (16, dict(M=8, residual_per_subspace=2), "residual_per_subspace"),
    (64, dict(M=64, B=8, Br=8, residual_per_subspace=1), "per-subspace"),
])
def test_constructor_validation(d, kw, msg):
    with pytest.raises(ValueError, match=msg):
        jg.JHQGpuIndex(d, jg.Params(**kw))


def test_derived_sizes_and_nprobe_clamp():
    g = jg.JHQGpuIndex(100, jg.Params(M=25, B=8, Br=4, nlist=8, nprobe=50))
    assert g.dims() == dict(Ds=4, K1D=4, bpd=2, Kr=16, bpv=50)
    assert g.dim == 100 and g.ntotal == 0
    g2 = jg.JHQGpuIndex(33, jg.Params(M=33, B=8, Br=4, nlist=4))
    assert g2.dims()["bpv"] == 17 and g2.dims()["K1D"] == 256


@pytest.mark.parametrize("d", [8, 64, 100])
def test_host_rotation_matches_oracle(d):
    """The engine builds Pi on the host at construction (cpu/jl_transform.cpp:25-56);
    it must be bit-identical to the oracle's restatement."""
    g = jg.JHQGpuIndex(d, jg.Params(M=d // 4 if d % 4 == 0 else d, B=8 if d % 4 else 8, nlist=4,
                                    seed=42))
    P = g.rotation()
    assert np.array_equal(P.view(np.uint32), po.rotation_rowmajor(d, 42).view(np.uint32))


def test_call_order_errors_before_device():
    g = jg.JHQGpuIndex(16, jg.Params(M=8, nlist=4, nprobe=2))
    x = np.zeros((100, 16), np.float32)
    with pytest.raises(RuntimeError, match="train"):
        g.add(x)
    with pytest.raises(RuntimeError, match="empty"):
        g.search(x[:2], 3)
    with pytest.raises(ValueError, match="nlist"):
        g.train(x[:3])
    with pytest.raises(ValueError):
        g.train(np.zeros((10, 15), np.float32))
    with pytest.raises(ValueError):
        g.set_nprobe(0)
    with pytest.raises(ValueError):
        g.set_alpha(-1.0)
    with pytest.raises(RuntimeError, match="not trained"):
        g.codebooks()
    assert "not trained" in jg.lib().jhq_last_error().decode()


def test_append_and_typed_inputs_validate_before_device():
    g = jg.JHQGpuIndex(16, jg.Params(M=8, nlist=4, nprobe=2))
    x8 = np.zeros((100, 16), np.uint8)
    with pytest.raises(RuntimeError, match="train"):
        g.append(x8)
    with pytest.raises(ValueError):
        g.append(np.zeros((10, 15), np.float32))
    L = jg.lib()
    assert L.jhq_train_ex(g._h, x8.ctypes.data_as(jg._VP), 7, 100) == jg.JHQ_EINVAL
    assert L.jhq_append_ex(g._h, None, 0, 10) == jg.JHQ_EINVAL


def test_index_file_errors_before_device(tmp_path):
    g = jg.JHQGpuIndex(16, jg.Params(M=8, nlist=4, nprobe=2))
    with pytest.raises(RuntimeError, match="not trained"):
        g.save(tmp_path / "untrained.jhq")
    with pytest.raises(ValueError, match="cannot open"):
        jg.JHQGpuIndex.load(tmp_path / "missing.jhq")
    bad = tmp_path / "bad.jhq"
    bad.write_bytes(b"NOTANIDX" + bytes(64))
    with pytest.raises(ValueError, match="not a JHQ index file"):
        jg.JHQGpuIndex.load(bad)
    short = tmp_path / "short.jhq"
    short.write_bytes(b"JHQAMD01")
    with pytest.raises(ValueError, match="not a JHQ index file"):
        jg.JHQGpuIndex.load(short)
    p = jg.Params(M=8, nlist=4, nprobe=2)
    got = jg.Params(**{f: getattr(p, f) for f in ("M", "B", "Br")})
    cp = jg._Params()
    assert jg.lib().jhq_get_params(g._h, ctypes.byref(cp)) == jg.JHQ_OK
    assert (cp.M, cp.B, cp.Br, cp.nlist, cp.nprobe) == (got.M, got.B, got.Br, 4, 2)


def test_kernel_entry_points_reject_bad_arguments():
    L = jg.lib()
    assert L.jhq_k_rotate(None, None, 4, 8, None, None) == jg.JHQ_EINVAL
    assert L.jhq_k_primary_encode(None, None, None, 4, 8, 3, 2, 2, 1, None) == jg.JHQ_EINVAL
    assert L.jhq_k_assign(None, 4, 8, None, None, 0, None, None) == jg.JHQ_EINVAL
    assert L.jhq_destroy(None) == jg.JHQ_OK
    assert L.jhq_ntotal(None) == 0


def test_no_cpu_fallback_without_library(tmp_path, monkeypatch):
    """The product fails loudly when the HIP library is absent."""
    monkeypatch.setattr(jg, "_LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(jg, "_lib", None)
    with pytest.raises(jg.JHQNotBuiltError):
        jg.JHQGpuIndex(16, jg.Params(M=8))
