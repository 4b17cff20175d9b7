"""Kernel-granular search stages in the reference's data layout, each checked
bit for bit against the oracle: jhq_k_build_lut (v14/search.cu:65-91),
jhq_k_scan_topck (:105-195, exact), jhq_k_refine (:198-242, the reference's
summation order) and jhq_k_final_topk (:244-291, exact by (dist, id)).

Inputs are the oracle's own index in the reference's layout: list_offsets,
primary codes transposed to [M, N] (v14/jhq_gpu_index.cu:512-517), residual
codes, corrections and ids in list order; rotated queries and probe lists come
from the oracle, so every stage's input is identical on both sides."""
import zlib

import numpy as np
import pytest

import pyoracle as po
from datagen import queries_and_base

import jhq_gpu_amd as jg

pytestmark = pytest.mark.gpu

# (name, d, M, nlist, nprobe, n, nq, k, alpha)
CASES = [
    ("d64_m16", 64, 16, 32, 5, 4000, 20, 10, 4.0),
    # M = 128: the query's LUT (128 KB) is copied to LDS
    ("d1024_m128", 1024, 128, 16, 3, 3000, 8, 10, 10.0),
    # M = 256 (Ds = 1, K1D = 256): the LUT does not fit in LDS and is read from HBM
    ("d256_m256_ds1", 256, 256, 16, 4, 2000, 8, 10, 4.0),
    # one probe of ~23 candidates and ck = 100: short lists padded with (+inf, -1)
    ("few_candidates", 64, 16, 64, 1, 1500, 16, 10, 10.0),
]
IDS = [c[0] for c in CASES]
_BUILT = {}


def _oracle(case):
    name, d, M, nlist, nprobe, n, nq, k, alpha = case
    if name not in _BUILT:
        base, q = queries_and_base(n, nq, d, 2 * nlist, seed=zlib.crc32(name.encode()) % 9999)
        o = po.OracleIndex(d, M=M, B=8, Br=4, alpha=alpha, nlist=nlist, nprobe=nprobe,
                           ivf_iters=4, seed=42)
        o.train(base[:1000])
        o.add(base)
        q_rot = po.rotate(o.P, q)
        probes = o.search(q, k, debug=True, q_rot=q_rot)["probes"]
        _BUILT[name] = (o, q_rot, probes)
    return _BUILT[name]


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _run_stages(o, q_rot, probes, k, ck, dev):
    import torch
    B = q_rot.shape[0]
    sizes = np.diff(o.list_offsets).astype(np.int32)
    poffs = np.zeros((B, probes.shape[1] + 1), np.int32)
    poffs[:, 1:] = np.cumsum(sizes[probes], axis=1)
    qtot = poffs[:, -1].copy()
    lut = torch.empty((B, o.M, 256), dtype=torch.float32, device=dev)
    jg.k_build_lut(_t(q_rot, dev), _t(o.c1d, dev), lut, o.M)
    tprim = torch.empty((B, ck), dtype=torch.float32, device=dev)
    tpos = torch.empty((B, ck), dtype=torch.int32, device=dev)
    jg.k_scan_topck(lut, _t(probes, dev), _t(poffs, dev), _t(o.list_offsets, dev),
                    _t(o.list_codes.T, dev), _t(qtot, dev), tprim, tpos)
    comp = torch.empty((B, ck), dtype=torch.float32, device=dev)
    jg.k_refine(_t(q_rot, dev), _t(o.res_c1d, dev), tpos, tprim, _t(o.list_res, dev),
                _t(o.list_corr, dev), comp, o.Br)
    fd = torch.empty((B, k), dtype=torch.float32, device=dev)
    fi = torch.empty((B, k), dtype=torch.int32, device=dev)
    jg.k_final_topk(comp, tpos, _t(o.list_ids, dev), fd, fi)
    torch.cuda.synchronize()
    return (lut.cpu().numpy(), tprim.cpu().numpy(), tpos.cpu().numpy(), fd.cpu().numpy(),
            fi.cpu().numpy())


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_stages_bit_exact(gpu, case):
    o, q_rot, probes = _oracle(case)
    k = case[7]
    ck = po.ck_of(o.alpha, k)
    lut, tprim, tpos, fd, fi = _run_stages(o, q_rot, probes, k, ck, gpu)
    for b in range(q_rot.shape[0]):
        assert np.array_equal(_bits(lut[b]), _bits(po.flat_lut(q_rot[b], o.M, o.c1d))), b
    want = o.search(np.zeros_like(q_rot), k, debug=True, q_rot=q_rot,
                    probes=probes)
    assert np.array_equal(tpos, want["topck_pos"])
    assert np.array_equal(_bits(tprim), _bits(want["topck_dist"]))
    assert np.array_equal(fi, want["ids"])
    assert np.array_equal(_bits(fd), _bits(want["dists"]))
    if case[0] == "few_candidates":
        assert (tpos == -1).any() and np.isinf(tprim[tpos == -1]).all()


@pytest.mark.parametrize("case", CASES[:2], ids=IDS[:2])
def test_refine_every_entry_bit_exact(gpu, case):
    """Final top-k over the whole short list (k = ck): every refined composite
    distance is compared, against the oracle run with alpha = 1 and k = ck."""
    o, q_rot, probes = _oracle(case)
    ck = po.ck_of(o.alpha, case[7])
    _, _, _, fd, fi = _run_stages(o, q_rot, probes, ck, ck, gpu)
    a0 = o.alpha
    o.alpha = np.float32(1.0)
    try:
        want = o.search(np.zeros_like(q_rot), ck, q_rot=q_rot, probes=probes)
    finally:
        o.alpha = a0
    assert np.array_equal(fi, want[1])
    assert np.array_equal(_bits(fd), _bits(want[0]))
