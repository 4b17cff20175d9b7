"""GPU parity: the HIP product against the CPU oracle on identical seeded inputs.

Bar: codebooks, rotation, codes and list layout are
bit-exact.  Search is checked stage-wise: the query rotation and centroid
scores run on fp32 MFMA, so the oracle is fed the GPU's rotated queries (checked
against float64) and its probe lists (checked against the oracle's own
selection up to score near-ties); from there the top-ck short list is
bit-exact, final ids are exact wherever neighbouring distances differ by more
than 1e-5 relative, and final distances agree within 1e-4 relative.
"""
import zlib

import numpy as np
import pytest

import pyoracle as po
from datagen import queries_and_base

import jhq_gpu_amd as jg

pytestmark = pytest.mark.gpu

DIST_RTOL = 1e-4
TIE_RTOL = 1e-5
QROT_RTOL = 1e-6      # fp32 MFMA rotation vs float64, per sqrt(d)
SCORE_TIE_RTOL = 1e-5

# (name, d, M, B, Br, nlist, nprobe, alpha, n, nq, k, batch)
CASES = [
    ("ds8_k1d2", 64, 8, 8, 4, 16, 4, 4.0, 3000, 70, 10, 32),
    ("ds4_k1d4_d100", 100, 25, 8, 4, 8, 3, 4.0, 2000, 40, 10, 16),
    ("ds1_k1d256_br8", 32, 32, 8, 8, 8, 2, 2.0, 1500, 33, 5, 64),
    ("b4_ds4_k1d2", 48, 12, 4, 4, 8, 8, 3.0, 1200, 20, 7, 8),
    ("flat_nlist1", 64, 16, 8, 4, 1, 1, 4.0, 2500, 25, 10, 1),
    ("d1024_m128", 1024, 128, 8, 4, 32, 6, 4.0, 2000, 20, 10, 64),
    # one query per batch split into ~250 chunks: multi-round streaming merge
    ("flat_many_chunks", 32, 8, 8, 4, 1, 1, 4.0, 20000, 6, 10, 1),
    # k=100 with alpha=4: ck=400 short list
    ("k100_ck400", 64, 16, 8, 4, 8, 4, 4.0, 6000, 12, 100, 16),
    # M a multiple of 32: lanes skewed across subspaces (K1D=4; ck=100)
    ("m64_ds4_ck100", 256, 64, 8, 4, 16, 5, 10.0, 3000, 20, 10, 32),
    ("m96_d768", 768, 96, 8, 4, 8, 3, 4.0, 2500, 16, 10, 16),
    # k=100, alpha=4 with M=32: ck=400 takes the dump scan and per-query selection
    ("m32_ck400", 128, 32, 8, 4, 8, 4, 4.0, 6000, 12, 100, 16),
    # skewed scan with more probes than a wave has lanes (probe lookup through LDS)
    ("m32_p80", 64, 32, 8, 4, 96, 80, 4.0, 4000, 12, 10, 16),
    # skewed scan at M=128 (parity LUT) with exactly 64 probes (lookup in registers)
    ("m128_p64", 256, 128, 8, 4, 64, 64, 4.0, 3000, 10, 10, 16),
    # M=16 (config 3's code size): the wave scan with ck=100 (three 64-key wave
    # buffers) and many segments
    ("m16_ck100", 128, 16, 8, 4, 32, 8, 10.0, 6000, 40, 10, 32),
    # M=16 with Ds=4 (K1D=4) and more probes than a wave has lanes
    ("m16_p80", 64, 16, 8, 4, 96, 80, 4.0, 5000, 12, 10, 16),
    # M=24 (not a multiple of 16): the wave scan
    ("m24_wave", 96, 24, 8, 4, 16, 5, 4.0, 3000, 20, 10, 32),
    # query product with K split over 5 workgroups of one step per wave
    ("qprod_d320_split5", 320, 40, 8, 4, 24, 5, 4.0, 2500, 70, 10, 64),
    # query product over 3 row blocks (batch 130) with a 20-row last batch,
    # K split over 3 workgroups of three steps per wave
    ("qprod_d576_b130", 576, 72, 8, 4, 40, 6, 4.0, 3000, 150, 10, 130),
]
IDS = [c[0] for c in CASES]

_BUILT = {}


def _build(case):
    name, d, M, B, Br, nlist, nprobe, alpha, n, nq, k, batch = case
    if name in _BUILT:
        return _BUILT[name]
    base, q = queries_and_base(n, nq, d, max(4, nlist * 2), seed=zlib.crc32(name.encode()) % 10000)
    p = jg.Params(M=M, B=B, Br=Br, alpha=alpha, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                  batch_size=batch, seed=42)
    g = jg.JHQGpuIndex(d, p)
    o = po.OracleIndex(d, M=M, B=B, Br=Br, alpha=alpha, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                       seed=42)
    ntrain = min(n, 1000) if nlist > 1 else n
    g.train(base[:ntrain])
    o.train(base[:ntrain])
    g.add(base)
    o.add(base)
    _BUILT[name] = (g, o, base, q, k)
    return _BUILT[name]


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_codebooks_bit_exact(gpu, case):
    g, o, *_ = _build(case)
    cb = g.codebooks()
    assert np.array_equal(_bits(cb["P"]), _bits(o.P))
    assert np.float32(cb["sigma"]) == o.sigma
    assert np.array_equal(_bits(cb["c1d"]), _bits(o.c1d))
    assert np.array_equal(_bits(cb["centroids"]), _bits(o.cent))
    assert np.array_equal(_bits(cb["cent_norms"]), _bits(o.cent_norms))
    assert np.array_equal(_bits(cb["res_c1d"]), _bits(o.res_c1d))


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_lists_bit_exact(gpu, case):
    g, o, *_ = _build(case)
    L = g.lists()
    assert np.array_equal(L["offsets"], o.list_offsets)
    assert np.array_equal(L["ids"], o.list_ids)
    assert np.array_equal(L["codes"], o.list_codes)
    assert np.array_equal(L["res"], o.list_res)
    assert np.array_equal(_bits(L["corr"]), _bits(o.list_corr))


def _check_final(gd, gi, od, oi):
    fin = np.isfinite(od)
    assert np.array_equal(np.isfinite(gd), fin)
    assert np.array_equal(gi[~fin], oi[~fin])
    rel = np.abs(gd[fin].astype(np.float64) - od[fin]) / np.maximum(np.abs(od[fin]), 1e-30)
    assert rel.max(initial=0.0) <= DIST_RTOL, rel.max()
    tie = po.near_tie_mask(np.where(fin, od, np.float32(3e38)), TIE_RTOL)
    mism = (gi != oi) & ~tie
    assert not mism.any(), np.argwhere(mism)[:5]


def _check_qrot(q, P, q_rot):
    """fp32 MFMA rotation against the float64 product."""
    want = q.astype(np.float64) @ P.astype(np.float64).T
    err = np.abs(q_rot.astype(np.float64) - want).max(initial=0.0)
    scale = np.abs(want).max(initial=1.0)
    assert err <= QROT_RTOL * scale * np.sqrt(q.shape[1]), err


def _check_probes(gp, op, q_rot, o):
    """GPU probe lists against the oracle's selection from the same rotated
    queries; they may differ only where the nprobe-th and (nprobe+1)-th
    centroid scores are a near-tie (the GPU scores come from fp32 MFMA)."""
    P = gp.shape[1]
    s = o.cent_norms[None, :].astype(np.float64) - 2.0 * q_rot.astype(np.float64) @ \
        o.cent.astype(np.float64).T
    srt = np.sort(s, axis=1)
    for i in range(gp.shape[0]):
        if set(gp[i]) == set(op[i]):
            continue
        assert P < s.shape[1]
        gap = srt[i, P] - srt[i, P - 1]
        assert gap <= SCORE_TIE_RTOL * np.abs(srt[i]).max(), (i, gap)


def _stagewise(g, o, q, k):
    """GPU search vs the oracle fed the GPU's rotated queries and probe lists:
    short lists bit-exact, final results to the north-star bar."""
    gr = g.search_debug(q, k)
    _check_qrot(q, o.P, gr["q_rot"])
    own = o.search(q, k, debug=True, q_rot=gr["q_rot"])
    _check_probes(gr["probes"], own["probes"], gr["q_rot"], o)
    orr = o.search(q, k, debug=True, q_rot=gr["q_rot"], probes=gr["probes"])
    assert np.array_equal(gr["topck_pos"], orr["topck_pos"])
    assert np.array_equal(_bits(gr["topck_dist"]), _bits(orr["topck_dist"]))
    _check_final(gr["dists"], gr["ids"], orr["dists"], orr["ids"])
    return gr, orr


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_search_parity(gpu, case):
    g, o, base, q, k = _build(case)
    gr, orr = _stagewise(g, o, q, k)
    # end to end against the oracle's own fixed-order rotation: the rotated
    # queries differ in the last bits only, so results agree except where
    # distances nearly tie
    ed, ei = o.search(q, k)
    fin = np.isfinite(ed)
    rel = np.abs(gr["dists"][fin].astype(np.float64) - ed[fin]) / np.maximum(np.abs(ed[fin]), 1e-30)
    assert rel.max(initial=0.0) <= DIST_RTOL
    overlap = np.mean([len(set(a) & set(b)) / max(1, len(set(b) - {-1}))
                       for a, b in zip(gr["ids"], ei)])
    assert overlap >= 0.98, overlap
    # the plain API returns the same rows as the debug path
    d2, i2 = g.search(q, k)
    assert np.array_equal(i2, gr["ids"])
    assert np.array_equal(_bits(d2), _bits(gr["dists"]))


@pytest.mark.parametrize("name", ["d1024_m128", "qprod_d320_split5", "qprod_d576_b130"])
def test_query_product_repeatable(gpu, name):
    """The query product adds its split sums in a fixed order: repeated
    searches give bit-identical rotated queries, probes and results."""
    case = CASES[IDS.index(name)]
    g, o, base, q, k = _build(case)
    a = g.search_debug(q, k)
    for _ in range(2):
        b = g.search_debug(q, k)
        assert np.array_equal(_bits(a["q_rot"]), _bits(b["q_rot"]))
        assert np.array_equal(a["probes"], b["probes"])
        assert np.array_equal(a["ids"], b["ids"])
        assert np.array_equal(_bits(a["dists"]), _bits(b["dists"]))


@pytest.mark.parametrize("case", CASES[:2], ids=IDS[:2])
def test_search_device_matches_host(gpu, case):
    import torch
    g, o, base, q, k = _build(case)
    d1, i1 = g.search(q, k)
    qt = torch.from_numpy(q).to(gpu)
    od = torch.empty((q.shape[0], k), dtype=torch.float32, device=gpu)
    oi = torch.empty((q.shape[0], k), dtype=torch.int32, device=gpu)
    g.search_device(qt, k, od, oi, stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert np.array_equal(oi.cpu().numpy(), i1)
    assert np.array_equal(_bits(od.cpu().numpy()), _bits(d1))


@pytest.mark.parametrize("name", ["ds8_k1d2", "m64_ds4_ck100", "k100_ck400", "d1024_m128"])
def test_search_device_pipelined_batches(gpu, name):
    """A device search over many batches (the search lanes, each a workspace and a stream,
    joined into the caller's stream; consecutive batch pairs of a lane share one
    query product where the probe selection adds its split sums, as at d = 1024) returns what
    one call per batch and the host search return, including a ragged last
    batch (the second of the last pair)."""
    import torch
    case = CASES[IDS.index(name)]
    g, o, base, q, k = _build(case)
    batch = case[-1]
    g.reserve(k)  # device searches run in the reserved workspace only
    qq = np.ascontiguousarray(np.tile(q, (1 + 5 * batch // q.shape[0], 1))[:5 * batch + 3])
    d1, i1 = g.search(qq, k)
    qt = torch.from_numpy(qq).to(gpu)
    od = torch.full((qq.shape[0], k), -1.0, dtype=torch.float32, device=gpu)
    oi = torch.full((qq.shape[0], k), -2, dtype=torch.int32, device=gpu)
    s = torch.cuda.current_stream()
    for rep in range(2):
        g.search_device(qt, k, od, oi, stream=s)
        got_i, got_d = oi.cpu().numpy(), od.cpu().numpy()  # ordered after the join
        assert np.array_equal(got_i, i1), rep
        assert np.array_equal(_bits(got_d), _bits(d1)), rep
    od2 = torch.empty_like(od)
    oi2 = torch.empty_like(oi)
    for b0 in range(0, qq.shape[0], batch):
        g.search_device(qt[b0:b0 + batch], k, od2[b0:b0 + batch], oi2[b0:b0 + batch], stream=s)
    assert np.array_equal(oi2.cpu().numpy(), i1)
    assert np.array_equal(_bits(od2.cpu().numpy()), _bits(d1))


@pytest.mark.parametrize("name", ["m64_ds4_ck100", "m32_p80", "m128_p64"])
def test_skewed_scan_taken(gpu, name):
    """The M % 32 == 0 cases above exercise the skewed scan (not a fallback)."""
    g, _, _, _, k = _build(CASES[IDS.index(name)])
    assert g.scan_plan(k)[0] == "scan_skew_kernel"


@pytest.mark.parametrize("name", ["ds8_k1d2", "ds4_k1d4_d100", "m24_wave", "m16_p80",
                                  "flat_nlist1"])
def test_wave_scan_taken(gpu, name):
    g, _, _, _, k = _build(CASES[IDS.index(name)])
    assert g.scan_plan(k)[0] == "scan_wave_kernel"


# one-bit digits with M a multiple of 16 can take the integer-MFMA pre-scan;
# the default takes it for M >= 64 when a batch's queries share their lists.
# The byte-LUT scans these cases would otherwise run are checked here with
# scan kind 1, the pre-scan with scan kind 2
@pytest.mark.parametrize("name,default,lut_scan", [
    ("d1024_m128", "mfma_scan_kernel", "scan_skew_kernel"),
    ("m96_d768", "mfma_scan_kernel", "scan_skew_kernel"),
    ("m16_ck100", "scan_wave_kernel", "scan_wave_kernel")])
def test_lut_scans_of_mfma_cases(gpu, name, default, lut_scan):
    g, o, base, q, k = _build(CASES[IDS.index(name)])
    assert g.scan_plan(k)[0] == default
    try:
        g.set_scan_kind(1)
        assert g.scan_plan(k)[0] == lut_scan
        _stagewise(g, o, q, k)
        g.set_scan_kind(2)
        assert g.scan_plan(k)[0] == "mfma_scan_kernel"
        _stagewise(g, o, q, k)
    finally:
        g.set_scan_kind(0)


def test_k_larger_than_candidates(gpu):
    """Unfilled slots are (+inf, -1) like v14/search.cu:284-286."""
    g, o, base, q, _ = _build(CASES[3])
    _stagewise(g, o, q, 64)


def test_alpha_sweep_matches_oracle(gpu):
    g, o, base, q, k = _build(CASES[0])
    for alpha in (1.0, 2.5, 10.0):
        g.set_alpha(alpha)
        o.alpha = np.float32(alpha)
        _stagewise(g, o, q, k)
    g.set_alpha(CASES[0][7])
    o.alpha = np.float32(CASES[0][7])


def test_nprobe_sweep_matches_oracle(gpu):
    g, o, base, q, k = _build(CASES[0])
    for nprobe in (1, 7, 16, 40):
        g.set_nprobe(nprobe)
        o.nprobe = min(nprobe, o.nlist)
        _stagewise(g, o, q, k)
    g.set_nprobe(CASES[0][6])
    o.nprobe = CASES[0][6]


def test_call_order_errors(gpu):
    p = jg.Params(M=8, nlist=4, nprobe=2)
    g = jg.JHQGpuIndex(16, p)
    x = np.random.default_rng(1).standard_normal((100, 16)).astype(np.float32)
    with pytest.raises(RuntimeError, match="train"):
        g.add(x)
    with pytest.raises(RuntimeError, match="empty"):
        g.search(x[:2], 3)
    with pytest.raises(ValueError, match="nlist"):
        g.train(x[:3])
    g.train(x)
    g.add(x)
    with pytest.raises(RuntimeError, match="one add"):
        g.add(x)
    with pytest.raises(ValueError):
        g.search(x[:2], 0)
    d, i = g.search(x[:0], 3)
    assert d.shape == (0, 3)
