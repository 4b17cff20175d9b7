"""GPU parity of the integer-MFMA pre-scan with exact re-check
(mfma_plan_kernel, mfma_scan_kernel, mfma_recheck_kernel), the scan that
one-bit-digit indexes (K1D = 2, Ds = 8) take by default.

The pre-scan only chooses which candidates are re-checked; the short list is
then selected from distances recomputed in the reference's order
(v14/search.cu:65-91,146-151) by (dist, stored position).  So every case must
give the oracle's short list bit for bit, and the same results as the
byte-LUT scans (scan kind 1) bit for bit.  Cases cover every M the kernel is
built for up to 128, ck from 10 to 400, lists whose capacity exceeds their
size (after appends), duplicates that overflow the re-check buffer (the
streamed fallback), every source of the re-check's first bound (tile minima
in LDS, in registers, from global memory) and of its exact ck-th value (in
registers, over the whole row), and pipelined device searches.  The cases force the
pre-scan (scan kind 2); test_default_choice checks when the default takes it."""
import sys
import zlib

import numpy as np
import pytest

import pyoracle as po
from datagen import queries_and_base
from test_gpu_parity import _bits, _stagewise

import jhq_gpu_amd as jg

pytestmark = pytest.mark.gpu

# (name, d, M, nlist, nprobe, alpha, n, nq, k, batch)
CASES = [
    ("m16_a10", 128, 16, 32, 8, 10.0, 6000, 40, 10, 32),
    ("m32_a4", 256, 32, 16, 5, 4.0, 4000, 24, 10, 16),
    ("m48_b7", 384, 48, 24, 7, 4.0, 3000, 21, 10, 7),
    ("m64_p12", 512, 64, 16, 12, 3.0, 3000, 20, 10, 20),
    ("m80_a10", 640, 80, 12, 4, 10.0, 2500, 16, 10, 16),
    ("m96_flat", 768, 96, 1, 1, 4.0, 2500, 9, 10, 1),
    ("m112_a4", 896, 112, 8, 3, 4.0, 2500, 12, 10, 12),
    ("m128_a10", 1024, 128, 32, 6, 10.0, 3000, 20, 10, 64),
    ("m32_ck400", 256, 32, 8, 4, 4.0, 6000, 12, 100, 16),
    # 80 K candidates per query: 5,000 tile minima, more than the re-check
    # holds in LDS (4,096), so they are ranked from registers
    ("m32_wide", 256, 32, 2, 2, 10.0, 80000, 8, 10, 8),
]
IDS = [c[0] for c in CASES]
_BUILT = {}


def _say(msg):
    print(f"[mfma] {msg}", file=sys.stderr, flush=True)


def _build(case):
    name, d, M, nlist, nprobe, alpha, n, nq, k, batch = case
    if name in _BUILT:
        return _BUILT[name]
    _say(f"build {name}")
    base, q = queries_and_base(n, nq, d, max(4, nlist * 2), seed=zlib.crc32(name.encode()) % 10000)
    p = jg.Params(M=M, B=8, Br=4, alpha=alpha, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                  batch_size=batch, seed=42)
    g = jg.JHQGpuIndex(d, p)
    o = po.OracleIndex(d, M=M, B=8, Br=4, alpha=alpha, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                       seed=42)
    ntrain = min(n, 1000) if nlist > 1 else n
    g.train(base[:ntrain])
    o.train(base[:ntrain])
    g.add(base)
    o.add(base)
    g.set_scan_kind(2)
    _BUILT[name] = (g, o, q, k)
    return _BUILT[name]


def _same(a, b):
    assert np.array_equal(a["topck_pos"], b["topck_pos"])
    assert np.array_equal(_bits(a["topck_dist"]), _bits(b["topck_dist"]))
    assert np.array_equal(a["ids"], b["ids"])
    assert np.array_equal(_bits(a["dists"]), _bits(b["dists"]))


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_mfma_scan_matches_oracle_and_lut_scans(gpu, case):
    g, o, q, k = _build(case)
    assert g.scan_plan(k)[0] == "mfma_scan_kernel"
    _say(f"{case[0]}: stage-wise")
    gr, _ = _stagewise(g, o, q, k)
    g.set_scan_kind(1)
    try:
        assert g.scan_plan(k)[0] != "mfma_scan_kernel"
        lr = g.search_debug(q, k)
    finally:
        g.set_scan_kind(2)
    _same(gr, lr)
    # repeated searches are bit-identical (the work list's order varies)
    _same(gr, g.search_debug(q, k))


def test_mfma_duplicates_overflow_recheck(gpu):
    """7000 copies of one vector tie in every distance: more survivors than
    the re-check buffer holds, so the streamed fallback selects the short
    list (ties broken by stored position)."""
    d, M, nlist, nprobe, k = 128, 16, 4, 2, 10
    base, q = queries_and_base(3000, 6, d, 8, seed=991)
    dup = np.repeat(q[:1] + np.float32(1e-3), 7000, axis=0)
    base = np.ascontiguousarray(np.concatenate([base[:1500], dup, base[1500:]]), np.float32)
    p = jg.Params(M=M, B=8, Br=4, alpha=4.0, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                  batch_size=8, seed=42)
    g = jg.JHQGpuIndex(d, p)
    o = po.OracleIndex(d, M=M, B=8, Br=4, alpha=4.0, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                       seed=42)
    g.train(base[:4000])
    o.train(base[:4000])
    g.add(base)
    o.add(base)
    g.set_scan_kind(2)
    assert g.scan_plan(k)[0] == "mfma_scan_kernel"
    gr, _ = _stagewise(g, o, q, k)
    g.set_scan_kind(1)
    try:
        lr = g.search_debug(q, k)
    finally:
        g.set_scan_kind(2)
    _same(gr, lr)


def test_mfma_after_appends(gpu):
    """Appends leave lists with more capacity than size (the code rows'
    stride differs from the candidate count)."""
    d, M, nlist, nprobe, k = 256, 32, 16, 5, 10
    base, q = queries_and_base(6000, 24, d, 40, seed=4242)
    p = jg.Params(M=M, B=8, Br=4, alpha=10.0, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                  batch_size=16, seed=42)
    g = jg.JHQGpuIndex(d, p)
    o = po.OracleIndex(d, M=M, B=8, Br=4, alpha=10.0, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                       seed=42)
    g.train(base[:2000])
    o.train(base[:2000])
    g.set_scan_kind(2)
    g.add(base[:1000])
    upto = 1000
    for n in (3, 600, 1, 2500, 31, 1865):
        g.append(base[upto:upto + n])
        upto += n
        o.add(base[:upto])
        assert g.scan_plan(k)[0] == "mfma_scan_kernel"
        gr, _ = _stagewise(g, o, q, k)
        g.set_scan_kind(1)
        try:
            lr = g.search_debug(q, k)
        finally:
            g.set_scan_kind(2)
        _same(gr, lr)


def test_mfma_device_search_pipelined(gpu):
    """Many batches of a device search (the search lanes, one workspace each;
    consecutive batch pairs of a lane share one query product, the last pair
    ragged) return what the host search returns."""
    import torch
    g, o, q, k = _build(CASES[IDS.index("m32_a4")])
    batch = CASES[IDS.index("m32_a4")][-1]
    g.reserve(k)
    qq = np.ascontiguousarray(np.tile(q, (1 + 5 * batch // q.shape[0], 1))[:5 * batch + 3])
    d1, i1 = g.search(qq, k)
    qt = torch.from_numpy(qq).to(gpu)
    od = torch.full((qq.shape[0], k), -1.0, dtype=torch.float32, device=gpu)
    oi = torch.full((qq.shape[0], k), -2, dtype=torch.int32, device=gpu)
    s = torch.cuda.current_stream()
    for rep in range(2):
        g.search_device(qt, k, od, oi, stream=s)
        assert np.array_equal(oi.cpu().numpy(), i1), rep
        assert np.array_equal(_bits(od.cpu().numpy()), _bits(d1)), rep


def test_default_choice(gpu):
    """Scan kind 0 takes the pre-scan when the queries of a batch share their
    lists (large batch, few lists) and the byte-LUT scan when each probed
    list serves about one query (one query per batch) or the short list is
    long."""
    g, o, q, k = _build(CASES[IDS.index("m128_a10")])
    g96, _, _, k96 = _build(CASES[IDS.index("m96_flat")])
    try:
        g.set_scan_kind(0)
        g96.set_scan_kind(0)
        assert g.scan_plan(k)[0] == "mfma_scan_kernel"
        assert g96.scan_plan(k96)[0] == "scan_skew_kernel"
        # short lists longer than 1024 (k = 110, alpha = 10: 1100) keep the
        # byte-LUT scan
        assert g.scan_plan(110)[0] != "mfma_scan_kernel"
    finally:
        g.set_scan_kind(2)
        g96.set_scan_kind(2)


def _from_gpu_lists(g, d):
    cb = g.codebooks()
    L = g.lists()
    o = po.OracleIndex.from_state(d, g.params, cb["P"], cb["c1d"], cb["res_c1d"],
                                  cb["centroids"], cb["cent_norms"], L["offsets"], L["ids"],
                                  L["codes"], L["res"], L["corr"])
    return o, L


def test_mfma_recheck_tile_minima_from_global(gpu):
    """One list of 600,000 vectors probed by every query: 37,500 tiles per
    query, more tile minima than the re-check ranks in registers (32 per
    thread x 1024 threads = 32,768), so the bound comes from the radix
    select over global memory (block_radix_kth_glob).  The short lists must
    equal the oracle's over the same lists and the byte-LUT scan's."""
    d, M, n, nq, k = 128, 16, 600_000, 8, 10
    base, q = queries_and_base(n, nq, d, 64, seed=6060)
    p = jg.Params(M=M, B=8, Br=4, alpha=10.0, nlist=1, nprobe=1, ivf_iters=4, batch_size=8,
                  seed=42)
    g = jg.JHQGpuIndex(d, p)
    g.train(base[:20_000])
    g.add(base)
    g.set_scan_kind(2)
    assert g.scan_plan(k)[0] == "mfma_scan_kernel"
    o, L = _from_gpu_lists(g, d)
    tiles = (np.diff(L["offsets"]) + 15) // 16
    assert tiles.sum() > 32 * 1024
    _say("600K flat: stage-wise")
    gr, _ = _stagewise(g, o, q, k)
    g.set_scan_kind(1)
    try:
        lr = g.search_debug(q, k)
    finally:
        g.set_scan_kind(2)
    _same(gr, lr)


def test_mfma_recheck_whole_row_select(gpu):
    """30,000 copies of the first query vector: for that query the ck
    smallest I values all tie at the copies' I (their codes minimise the
    ADC distance), so the ck-th smallest tile minimum is that value and
    1,875 tiles have a minimum at or below it.  The survivors (over 30,000)
    exceed the re-check buffer, the tiles exceed what the in-register select
    holds (1,536 listed tiles, 8 values per thread), so the exact ck-th I
    comes from the radix select over the whole row (block_radix_kth_row) and
    the short list from the streamed selection; ties break by stored
    position.  The other queries take the usual path."""
    d, M, nlist, nprobe, k = 128, 16, 4, 2, 10
    base, q = queries_and_base(20_000, 6, d, 8, seed=7070)
    dup = np.repeat(q[:1], 30_000, axis=0)
    base = np.ascontiguousarray(np.concatenate([base[:9000], dup, base[9000:]]), np.float32)
    p = jg.Params(M=M, B=8, Br=4, alpha=4.0, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                  batch_size=8, seed=42)
    g = jg.JHQGpuIndex(d, p)
    g.train(base[:12_000])
    g.add(base)
    g.set_scan_kind(2)
    assert g.scan_plan(k)[0] == "mfma_scan_kernel"
    o, L = _from_gpu_lists(g, d)
    # the copies sit in one list, next to each other
    pos = np.empty(base.shape[0], np.int64)
    pos[L["ids"]] = np.arange(base.shape[0])
    dp = pos[9000:39_000]
    assert dp.max() - dp.min() == 30_000 - 1
    _say("30K duplicates: stage-wise")
    gr, _ = _stagewise(g, o, q, k)
    g.set_scan_kind(1)
    try:
        lr = g.search_debug(q, k)
    finally:
        g.set_scan_kind(2)
    _same(gr, lr)
