"""GPU parity at the benchmarked operating point, full size: config 2
with N = 1,000,000, D = 1024, nlist = 4096, M = 128,
batch 64, alpha 10 (ck = 100), nprobe 16 and 64.

The index is built by the GPU (train on the first 100,000 vectors, then one
add of all 1,000,000, as the reference demo does,
examples/demo_jhq_v14_streaming_add.cu:78-86).  The oracle then searches the
GPU-built lists (v14/search.cu:105-291 restated), fed the GPU's rotated
queries and probe lists, so every later stage is checked at this size:
* the top-ck short lists bit for bit (positions and primary distances), which
  pins the pre-scan's exact re-check at the benchmarked list sizes (a hub list
  of about 20 K vectors that every query probes);
* final ids exact outside 1e-5 near-ties, distances within 1e-4 relative;
* the first 20,000 vectors' codes, residual codes and corrections, and the
  first 2,000 vectors' lists, against the oracle's rotation, encode and
  assignment of the same rows;
* a device search over seven batches (every search lane takes one, the first
  two) returns the host debug search's rows bit for bit.
The base is the benchmark's own (bench.py's generator and seeds, drawn on the
device), so this is the index bench.py times; the queries come from the same
mixture."""
import math
import sys

import numpy as np
import pytest

import pyoracle as po
from test_gpu_parity import _bits, _check_final, _check_probes, _check_qrot

import jhq_gpu_amd as jg

pytestmark = pytest.mark.gpu

N, D, NLIST, M, NCOMP, BATCH = 1_000_000, 1024, 4096, 128, 10_000, 64
NQ_ORACLE = 128
NQ_DEVICE = 7 * BATCH
_STATE = {}


def _say(msg):
    print(f"[fullsize] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module", autouse=True)
def _release():
    """The 1M index and its host copies are dropped when the module ends."""
    yield
    _STATE.clear()


def _mixture(torch, dev, n, seed, means=None, scales=None, chunk=100_000):
    """bench.py's generator, draw for draw: per-component N(0, I) means,
    diagonal std log-uniform in [0.1, 1] (drawn first unless given), then per
    chunk the component ids and the noise; rows L2-normalised."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    if means is None:
        means = torch.randn(NCOMP, D, device=dev, generator=g)
        scales = torch.exp(torch.empty(NCOMP, D, device=dev).uniform_(math.log(0.1), 0.0,
                                                                     generator=g))
    out = torch.empty(n, D, device=dev)
    for i in range(0, n, chunk):
        m = min(chunk, n - i)
        c = torch.randint(0, NCOMP, (m,), device=dev, generator=g)
        x = means[c] + scales[c] * torch.randn(m, D, device=dev, generator=g)
        out[i:i + m] = x / x.norm(dim=1, keepdim=True)
    return out, means, scales


def _cfg2(gpu):
    if "cfg2" in _STATE:
        return _STATE["cfg2"]
    import torch
    _say("generate 1M x 1024 base and queries on the device (the benchmark's seeds)")
    base, means, scales = _mixture(torch, gpu, N, 0x4A48510002)
    q, _, _ = _mixture(torch, gpu, NQ_DEVICE, 0x4A48510002 + 0x100, means, scales)
    hb = base.cpu().numpy()
    hq = q.cpu().numpy()
    del base, q
    torch.cuda.empty_cache()
    p = jg.Params(M=M, B=8, Br=4, alpha=10.0, nlist=NLIST, nprobe=16, ivf_iters=8,
                  batch_size=BATCH, seed=42)
    g = jg.JHQGpuIndex(D, p)
    _say("train on 100K, add 1M")
    g.train(hb[:100_000])
    g.add(hb)
    cb = g.codebooks()
    L = g.lists()
    o = po.OracleIndex.from_state(D, g.params, cb["P"], cb["c1d"], cb["res_c1d"],
                                  cb["centroids"], cb["cent_norms"], L["offsets"], L["ids"],
                                  L["codes"], L["res"], L["corr"])
    _STATE["cfg2"] = (g, o, hb, hq, cb, L)
    _say("built")
    return _STATE["cfg2"]


def test_cfg2_full_build_matches_oracle(gpu):
    g, o, hb, hq, cb, L = _cfg2(gpu)
    pos = np.empty(N, np.int64)
    pos[L["ids"]] = np.arange(N)
    ns, na = 20_000, 2_000
    p = pos[:ns]
    y = po.rotate(cb["P"], np.ascontiguousarray(hb[:ns]))
    codes = po.primary_encode(y, M, cb["c1d"])
    res, corr = po.residual_encode(y, codes, M, cb["c1d"], cb["res_c1d"], 4)
    assert np.array_equal(L["codes"][p], codes)
    assert np.array_equal(L["res"][p], res)
    assert np.array_equal(_bits(L["corr"][p]), _bits(corr))
    asg = po.assign(y[:na], cb["centroids"], cb["cent_norms"])
    lst = np.searchsorted(L["offsets"], p[:na], side="right") - 1
    assert np.array_equal(lst, asg)
    # the benchmark's list shape: lists shared across a batch, one large hub
    sizes = np.diff(L["offsets"])
    assert sizes.sum() == N and sizes.max() > 4 * N / NLIST


@pytest.mark.parametrize("nprobe", [16, 64])
def test_cfg2_full_stagewise(gpu, nprobe):
    g, o, hb, hq, cb, L = _cfg2(gpu)
    g.set_nprobe(nprobe)
    o.nprobe = nprobe
    try:
        assert g.scan_plan(10) == ("mfma_scan_kernel", 100)
        q = hq[:NQ_ORACLE]
        gr = g.search_debug(q, 10)
        _check_qrot(q, o.P, gr["q_rot"])
        own = o.search(q, 10, debug=True, q_rot=gr["q_rot"])
        _check_probes(gr["probes"], own["probes"], gr["q_rot"], o)
        _say(f"nprobe {nprobe}: oracle over the GPU-built lists")
        orr = o.search(q, 10, debug=True, q_rot=gr["q_rot"], probes=gr["probes"])
        assert np.array_equal(gr["topck_pos"], orr["topck_pos"])
        assert np.array_equal(_bits(gr["topck_dist"]), _bits(orr["topck_dist"]))
        _check_final(gr["dists"], gr["ids"], orr["dists"], orr["ids"])
        # the probed candidates per query are the benchmark's (tens of thousands)
        per_q = np.diff(L["offsets"])[gr["probes"]].sum(1)
        assert per_q.mean() > 20_000
    finally:
        g.set_nprobe(16)
        o.nprobe = 16


@pytest.mark.parametrize("nprobe", [16, 64])
def test_cfg2_full_device_search_lanes(gpu, nprobe):
    """Seven batches through the pipelined device search (the search lanes; three
    pairs that each share one query product, then one batch alone) equal the
    debug search of the same queries, batch by batch on one stream."""
    import torch
    g, o, hb, hq, cb, L = _cfg2(gpu)
    g.set_nprobe(nprobe)
    try:
        g.reserve(10)
        want = g.search_debug(hq, 10)
        qt = torch.from_numpy(hq).to(gpu)
        od = torch.full((NQ_DEVICE, 10), -1.0, dtype=torch.float32, device=gpu)
        oi = torch.full((NQ_DEVICE, 10), -2, dtype=torch.int32, device=gpu)
        for rep in range(2):
            g.search_device(qt, 10, od, oi, stream=torch.cuda.current_stream())
            assert np.array_equal(oi.cpu().numpy(), want["ids"]), rep
            assert np.array_equal(_bits(od.cpu().numpy()), _bits(want["dists"])), rep
    finally:
        g.set_nprobe(16)
