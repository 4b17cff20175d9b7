"""GPU parity at the shapes the benchmark runs, smaller N.

Every shape here has one-bit digits, so it can run the integer-MFMA pre-scan
with exact re-check (forced with scan kind 2) or the byte-LUT scans (scan kind
1); both are checked.

* Config 2: D=1024, M=128 (the skewed scan with the subspace-parity LUT),
  alpha=10 -> ck=100 (three 64-key wave buffers), nlist 256, nprobe 16 and
  64, batch 64 — many queries split over many workgroups (multi-segment work
  plan, the segment merge); the pre-scan's lists shared by many queries.
* Config 1's shape: the flat index (nlist = 1) at D=1024, M=128, one query
  per batch, so each query's single list is split across the chip and merged
  from ~256 segments (jhq_v1_plain/search.cu:126-228).
* Config 3's shape: uint8 rows at D=128, M=16 (Ds=8, K1D=2, the wave scan),
  nlist 1024, nprobe 64, batch 64.
* Config 4's shape: int8 heavy-tailed rows at D=100, M=25 (Ds=4, K1D=4),
  nlist 16,384, nprobe 48, batch 32.
* Config 2 at full size is in tests/test_gpu_fullsize.py.

Each case is checked stage-wise like tests/test_gpu_parity.py: codes and lists
bit-exact, the top-ck short list bit-exact from the GPU's rotated queries and
probes, final ids exact outside 1e-5 near-ties and distances within 1e-4."""
import sys
import zlib

import numpy as np
import pytest

import pyoracle as po
from datagen import byte_mixture, queries_and_base
from test_gpu_parity import _bits, _stagewise

import jhq_gpu_amd as jg

pytestmark = pytest.mark.gpu

_BUILT = {}


def _say(msg):
    print(f"[shapes] {msg}", file=sys.stderr, flush=True)


def _pair(name, d, M, nlist, nprobe, alpha, batch, base, ntrain):
    if name in _BUILT:
        return _BUILT[name]
    _say(f"build {name}: d={d} M={M} nlist={nlist} n={base.shape[0]} ntrain={ntrain}")
    p = jg.Params(M=M, B=8, Br=4, alpha=alpha, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                  batch_size=batch, seed=42)
    g = jg.JHQGpuIndex(d, p)
    o = po.OracleIndex(d, M=M, B=8, Br=4, alpha=alpha, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                       seed=42)
    g.train(base[:ntrain])
    o.train(np.asarray(base[:ntrain], np.float32))
    g.add(base)
    o.add(np.asarray(base, np.float32))
    _say(f"built {name}")
    _BUILT[name] = (g, o)
    return g, o


def _lists_equal(g, o):
    L = g.lists()
    assert np.array_equal(L["offsets"], o.list_offsets)
    assert np.array_equal(L["ids"], o.list_ids)
    assert np.array_equal(L["codes"], o.list_codes)
    assert np.array_equal(L["res"], o.list_res)
    assert np.array_equal(_bits(L["corr"]), _bits(o.list_corr))


def _cfg2():
    base, q = queries_and_base(50_000, 64, 1024, 512, seed=zlib.crc32(b"cfg2_shape") % 10000)
    g, o = _pair("cfg2_shape", 1024, 128, 256, 16, 10.0, 64, base, 4096)
    return g, o, q


def test_cfg2_shape_lists_bit_exact(gpu):
    g, o, _ = _cfg2()
    cb = g.codebooks()
    assert np.array_equal(_bits(cb["centroids"]), _bits(o.cent))
    assert np.array_equal(_bits(cb["res_c1d"]), _bits(o.res_c1d))
    _lists_equal(g, o)


@pytest.mark.parametrize("kind,scan", [(2, "mfma_scan_kernel"), (1, "scan_skew_kernel")])
@pytest.mark.parametrize("nprobe", [16, 64])
def test_cfg2_shape_benchmarked_scan(gpu, nprobe, kind, scan):
    """M=128 with ck=100 (the instance bench.py times): the pre-scan and the
    skewed scan."""
    g, o, q = _cfg2()
    g.set_nprobe(nprobe)
    g.set_scan_kind(kind)
    o.nprobe = nprobe
    try:
        assert g.scan_plan(10) == (scan, 100)
        _say(f"cfg2_shape nprobe={nprobe} kind={kind}: stage-wise search")
        gr, _ = _stagewise(g, o, q, 10)
        # queries really span several workgroups: the probed candidates of
        # one query exceed a workgroup's share of the batch
        sizes = np.diff(g.lists(include_payload=False)["offsets"])
        per_q = sizes[gr["probes"]].sum(1)
        assert per_q.sum() / 256 < per_q.max()
    finally:
        g.set_nprobe(16)
        g.set_scan_kind(0)
        o.nprobe = 16


@pytest.mark.parametrize("kind,scan", [(2, "mfma_scan_kernel"), (1, "scan_skew_kernel")])
def test_cfg2_shape_alpha4(gpu, kind, scan):
    """The same index at alpha=4 (ck=40, two 64-key wave buffers)."""
    g, o, q = _cfg2()
    g.set_alpha(4.0)
    g.set_scan_kind(kind)
    o.alpha = np.float32(4.0)
    try:
        assert g.scan_plan(10) == (scan, 40)
        _stagewise(g, o, q, 10)
    finally:
        g.set_alpha(10.0)
        g.set_scan_kind(0)
        o.alpha = np.float32(10.0)


@pytest.mark.parametrize("kind,scan", [(2, "mfma_scan_kernel"), (1, "scan_skew_kernel")])
def test_cfg1_shape_flat(gpu, kind, scan):
    """Flat index (nlist = 1) at D=1024, M=128, one query per batch
    (jhq_v1_plain/search.cu:126-228; v1's ck = min(ceil(alpha k), N) equals
    the short list here since N > ck)."""
    base, q = queries_and_base(20_000, 12, 1024, 64, seed=zlib.crc32(b"cfg1_flat") % 10000)
    g, o = _pair("cfg1_flat", 1024, 128, 1, 1, 4.0, 1, base, 5000)
    g.set_scan_kind(kind)
    try:
        assert g.scan_plan(10) == (scan, 40)
        _lists_equal(g, o)
        _say(f"cfg1_flat kind={kind}: stage-wise search")
        _stagewise(g, o, q, 10)
    finally:
        g.set_scan_kind(0)


@pytest.mark.parametrize("kind,scan", [(2, "mfma_scan_kernel"), (1, "scan_wave_kernel")])
def test_cfg3_shape_uint8(gpu, kind, scan):
    """uint8 rows at D=128, M=16 (wave scan), nlist 1024, nprobe 64, batch 64."""
    seed = zlib.crc32(b"cfg3_shape") % 10000
    base = byte_mixture(100_000, 128, 2048, seed, "uint8", comp_seed=seed + 1)
    qb = byte_mixture(64, 128, 2048, seed + 100, "uint8", comp_seed=seed + 1)
    g, o = _pair("cfg3_shape", 128, 16, 1024, 64, 4.0, 64, base, 16_384)
    g.set_scan_kind(kind)
    try:
        assert g.scan_plan(10)[0] == scan
        _lists_equal(g, o)
        _say(f"cfg3_shape kind={kind}: stage-wise search")
        _stagewise(g, o, qb.astype(np.float32), 10)
    finally:
        g.set_scan_kind(0)


def test_cfg4_shape_int8(gpu):
    """Config 4's shape: int8 rows from the heavy-tailed mixture (16 x
    Student-t, nu = 4) at D=100, M=25 (Ds=4, K1D=4: the wave scan, 25
    subspaces), nlist 16,384 (probe selection past 8,192 lists), nprobe 48,
    batch 32.  The GPU-built lists are checked against the oracle's encode and
    assignment on a sample (the oracle's k-means at this nlist would take
    hours on the CPU); search is checked stage-wise over the GPU-built lists."""
    seed = zlib.crc32(b"cfg4_shape") % 10000
    d, M, nlist, nprobe, batch, k = 100, 25, 16_384, 48, 32, 10
    xb = byte_mixture(300_000, d, 4096, seed, "int8", comp_seed=seed + 1)
    qb = byte_mixture(64, d, 4096, seed + 100, "int8", comp_seed=seed + 1)
    p = jg.Params(M=M, B=8, Br=4, alpha=4.0, nlist=nlist, nprobe=nprobe, ivf_iters=8,
                  batch_size=batch, seed=42)
    g = jg.JHQGpuIndex(d, p)
    _say("build cfg4_shape: n=300000 nlist=16384")
    g.train(xb)
    g.add(xb)
    assert g.scan_plan(k) == ("scan_wave_kernel", 40)
    cb = g.codebooks()
    L = g.lists()
    o = po.OracleIndex.from_state(d, g.params, cb["P"], cb["c1d"], cb["res_c1d"],
                                  cb["centroids"], cb["cent_norms"], L["offsets"], L["ids"],
                                  L["codes"], L["res"], L["corr"])
    pos = np.empty(xb.shape[0], np.int64)
    pos[L["ids"]] = np.arange(xb.shape[0])
    ns, na = 20_000, 2_000
    xf = xb[:ns].astype(np.float32)
    y = po.rotate(cb["P"], xf)
    codes = po.primary_encode(y, M, cb["c1d"])
    res, corr = po.residual_encode(y, codes, M, cb["c1d"], cb["res_c1d"], 4)
    assert np.array_equal(L["codes"][pos[:ns]], codes)
    assert np.array_equal(L["res"][pos[:ns]], res)
    assert np.array_equal(_bits(L["corr"][pos[:ns]]), _bits(corr))
    asg = po.assign(y[:na], cb["centroids"], cb["cent_norms"])
    lst = np.searchsorted(L["offsets"], pos[:na], side="right") - 1
    assert np.array_equal(lst, asg)
    _say("cfg4_shape: stage-wise search")
    _stagewise(g, o, qb.astype(np.float32), k)
