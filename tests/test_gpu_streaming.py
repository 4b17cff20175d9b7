"""GPU parity of the extensions config 5 needs:
streaming add into existing IVF lists and per-subspace residual codebooks,
plus uint8 / int8 ingestion.

The reference has none of these (one add() only, v14/jhq_gpu_index.cu:419-420;
one global residual codebook, :302-330; float32 input only), so parity is
pinned by invariants: a sequence of appends must leave exactly the list
storage that one add() of the same vectors in the same order leaves in the
oracle, and search stays bit-exact stage by stage after every append."""
import numpy as np
import pytest

import pyoracle as po
from datagen import queries_and_base
from test_gpu_parity import _bits, _stagewise

import jhq_gpu_amd as jg

pytestmark = pytest.mark.gpu


def _lists_equal(g, o):
    L = g.lists()
    assert np.array_equal(L["offsets"], o.list_offsets)
    assert np.array_equal(L["ids"], o.list_ids)
    assert np.array_equal(L["codes"], o.list_codes)
    assert np.array_equal(L["res"], o.list_res)
    assert np.array_equal(_bits(L["corr"]), _bits(o.list_corr))


def _pair(d, M, nlist, nprobe, per_sub, alpha=4.0, Br=4, batch=32):
    p = jg.Params(M=M, B=8, Br=Br, alpha=alpha, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                  batch_size=batch, seed=42, residual_per_subspace=per_sub)
    g = jg.JHQGpuIndex(d, p)
    o = po.OracleIndex(d, M=M, B=8, Br=Br, alpha=alpha, nlist=nlist, nprobe=nprobe,
                       ivf_iters=4, seed=42, residual_per_subspace=per_sub)
    return g, o


@pytest.mark.parametrize("per_sub", [0, 1], ids=["shared_books", "per_subspace_books"])
def test_streaming_append_equals_one_shot(gpu, per_sub):
    d, M, nlist, nprobe, k = 64, 16, 16, 5, 10
    base, q = queries_and_base(12800, 30, d, 40, seed=501 + per_sub)
    g, o = _pair(d, M, nlist, nprobe, per_sub)
    g.train(base[:2000])
    o.train(base[:2000])
    cb = g.codebooks()
    assert np.array_equal(_bits(cb["res_c1d"]), _bits(o.res_c1d))
    g.add(base[:1200])
    upto = 1200
    # ragged appends, one that fits in the existing blocks, some that move
    # lists, and a larger one (several encode workgroups' worth, as config 5)
    for n in (5, 1, 700, 2300, 40, 2754, 5800):
        g.append(base[upto:upto + n])
        upto += n
        o.add(base[:upto])
        assert g.ntotal == upto
        _lists_equal(g, o)
        _stagewise(g, o, q, k)
    used, cap = g.pool()
    assert used <= cap and used >= upto
    # re-packing bounds the pool: a quarter of headroom per list plus a
    # quarter for later moves, never the dead blocks of moved lists
    assert cap <= 1.6 * upto + 20 * nlist


@pytest.mark.parametrize("d,M", [(128, 32), (256, 64)], ids=["m32", "m64"])
def test_streaming_append_skewed_scan(gpu, d, M):
    """M a multiple of 32: the search takes the skewed scan, whose row copy
    of the codes is brought up to date before each search (appended rows,
    moved lists, a re-packed pool)."""
    nlist, nprobe, k = 16, 5, 10
    base, q = queries_and_base(6000, 24, d, 40, seed=733 + M)
    g, o = _pair(d, M, nlist, nprobe, 0)
    g.train(base[:2000])
    o.train(base[:2000])
    assert g.scan_plan(k)[0] == "scan_skew_kernel"
    g.add(base[:1000])
    upto = 1000
    o.add(base[:upto])
    _stagewise(g, o, q, k)
    for n in (3, 600, 1, 2500, 31, 1865):
        g.append(base[upto:upto + n])
        upto += n
        o.add(base[:upto])
        _lists_equal(g, o)
        _stagewise(g, o, q, k)
        d1, i1 = g.search(q, k)
        d2, i2 = g.search(q, k)  # no change between: the copy is current
        assert np.array_equal(i1, i2) and np.array_equal(_bits(d1), _bits(d2))


def test_append_from_empty_and_add_guard(gpu):
    d, M, nlist, nprobe, k = 32, 8, 8, 3, 5
    base, q = queries_and_base(3000, 12, d, 16, seed=77)
    g, o = _pair(d, M, nlist, nprobe, 0)
    g.train(base[:1000])
    o.train(base[:1000])
    for a, b in ((0, 900), (900, 2000), (2000, 3000)):
        g.append(base[a:b])
    o.add(base)
    _lists_equal(g, o)
    _stagewise(g, o, q, k)
    with pytest.raises(RuntimeError, match="one add"):
        g.add(base[:10])


@pytest.mark.parametrize("kind,scan", [(2, "mfma_scan_kernel"), (1, "scan_dump_kernel")],
                         ids=["pre_scan", "byte_lut_dump"])
def test_streaming_config5_shape(gpu, kind, scan):
    """Config 5's shape at small N: D=768, M=96, per-subspace codebooks
    (Kr=16 each), k=100 with alpha=4 (ck=400), batch 128, inserts in batches
    interleaved with searches.  Both scans config 5 can take: the pre-scan
    (what bench.py --config 5 runs; ck 400 > 128, so its short lists go to
    refine_topk_kernel) and the byte-LUT dump scan with per-query selection."""
    d, M, nlist, nprobe, k = 768, 96, 8, 4, 100
    base, q = queries_and_base(5000, 16, d, 24, seed=909)
    g, o = _pair(d, M, nlist, nprobe, 1, batch=128)
    g.set_scan_kind(kind)
    g.train(base[:1000])
    o.train(base[:1000])
    g.add(base[:3000])
    o.add(base[:3000])
    assert g.scan_plan(k) == (scan, 400)
    upto = 3000
    for n in (1000, 1000):
        _stagewise(g, o, q, k)
        g.append(base[upto:upto + n])
        upto += n
        o.add(base[:upto])
        _lists_equal(g, o)
        assert g.scan_plan(k) == (scan, 400)
    _stagewise(g, o, q, k)


@pytest.mark.parametrize("dtype", ["uint8", "int8"])
def test_byte_ingestion(gpu, dtype):
    """uint8 / int8 rows cross PCIe as bytes and become float32 on the device;
    results equal the float32 path on the converted data."""
    d, M, nlist, nprobe, k = 100, 25, 8, 3, 10
    rng = np.random.default_rng(31 if dtype == "uint8" else 32)
    cent = rng.normal(0, 30, (12, d))
    x = cent[rng.integers(0, 12, 9000)] + rng.normal(0, 20, (9000, d))
    if dtype == "uint8":
        xb = np.clip(np.rint(x + 128), 0, 255).astype(np.uint8)
    else:
        xb = np.clip(np.rint(x), -128, 127).astype(np.int8)
    xf = xb.astype(np.float32)
    g, o = _pair(d, M, nlist, nprobe, 0)
    g.train(xb[:1500])
    o.train(xf[:1500])
    g.add(xb[:3000])
    g.append(xb[3000:])
    o.add(xf)
    _lists_equal(g, o)
    qb, qf = xb[:20], xf[:20]
    d1, i1 = g.search(qb, k)
    d2, i2 = g.search(qf, k)
    assert np.array_equal(i1, i2) and np.array_equal(_bits(d1), _bits(d2))
    _stagewise(g, o, qf, k)
