"""Kernel-granular parity through the C-ABI (jhq_k_* entry points) against the
CPU oracle: rotation, primary/residual encode and IVF assignment must be
bit-exact, including ragged shapes and exact ties."""
import numpy as np
import pytest

import pyoracle as po

import jhq_gpu_amd as jg

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("n,d", [(1, 8), (37, 64), (300, 100), (1000, 128), (129, 1024)])
def test_rotate_bit_exact(gpu, n, d):
    import torch
    rng = np.random.default_rng(n * 7 + d)
    x = rng.standard_normal((n, d)).astype(np.float32)
    P = po.rotation_rowmajor(d, 42) if d <= 256 else rng.standard_normal((d, d)).astype(np.float32)
    y = torch.empty((n, d), dtype=torch.float32, device=gpu)
    jg.k_rotate(_t(P, gpu), _t(x, gpu), y)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), po.rotate(P, x).view(np.uint32))


@pytest.mark.parametrize("d,M,B,Br,Kr", [(64, 8, 8, 4, 16), (100, 25, 8, 4, 16), (32, 32, 8, 8, 256),
                                          (48, 12, 4, 4, 16), (33, 33, 2, 4, 7), (1024, 128, 8, 4, 16)])
def test_encode_bit_exact(gpu, d, M, B, Br, Kr):
    import torch
    rng = np.random.default_rng(d * 31 + M)
    n = 777
    y = (rng.standard_normal((n, d)) * 0.05).astype(np.float32)
    y[0, :] = 0.0  # exact midpoint (0) for K1D=2 → upper codeword
    Ds = d // M
    K1D = 1 << (B // Ds)
    c1d = po.lloyd_max_c1d(0.05, K1D)
    res_c1d = np.sort(rng.standard_normal(Kr).astype(np.float32) * 0.02)
    codes = torch.empty((n, M), dtype=torch.uint8, device=gpu)
    jg.k_primary_encode(_t(y, gpu), codes, _t(c1d, gpu), M)
    torch.cuda.synchronize()
    oc = po.primary_encode(y, M, c1d)
    assert np.array_equal(codes.cpu().numpy(), oc)
    bpv = (d * Br + 7) // 8
    res = torch.empty((n, bpv), dtype=torch.uint8, device=gpu)
    corr = torch.empty((n,), dtype=torch.float32, device=gpu)
    jg.k_residual_encode(_t(y, gpu), codes, res, corr, _t(c1d, gpu), _t(res_c1d, gpu), M, Br)
    torch.cuda.synchronize()
    ores, ocorr = po.residual_encode(y, oc, M, c1d, res_c1d, Br)
    assert np.array_equal(res.cpu().numpy(), ores)
    assert np.array_equal(corr.cpu().numpy().view(np.uint32), ocorr.view(np.uint32))


@pytest.mark.parametrize("n,d,nlist", [(1000, 64, 16), (513, 100, 300), (64, 1024, 4096)])
def test_assign_bit_exact_with_ties(gpu, n, d, nlist):
    import torch
    rng = np.random.default_rng(n + d + nlist)
    y = rng.standard_normal((n, d)).astype(np.float32)
    cent = rng.standard_normal((nlist, d)).astype(np.float32)
    cent[nlist // 2] = cent[nlist // 3]  # duplicate centroid: ties go to the lower id
    norms = po.cent_norms(cent)
    a = torch.empty((n,), dtype=torch.int32, device=gpu)
    jg.k_assign(_t(y, gpu), _t(cent, gpu), _t(norms, gpu), a)
    torch.cuda.synchronize()
    assert np.array_equal(a.cpu().numpy(), po.assign(y, cent, norms))


@pytest.mark.parametrize("n,d,nlist", [(4096, 128, 1000), (5000, 1024, 4000), (300, 96, 129)])
def test_assign_near_ties_bit_exact(gpu, n, d, nlist):
    """The MFMA assignment with its fixed-order re-check against the oracle on
    rows built to sit on or next to decision boundaries: midpoints of two
    centroids (the fixed-order rounding decides), rows a hair off a midpoint,
    copies of centroids, duplicate centroids (ties to the lower list), plus
    ragged tiles (nlist not a multiple of 128)."""
    import torch
    rng = np.random.default_rng(7 * n + d)
    cent = rng.standard_normal((nlist, d)).astype(np.float32)
    cent[nlist - 1] = cent[0]
    cent[nlist // 2] = cent[nlist // 5]
    y = rng.standard_normal((n, d)).astype(np.float32)
    a_i = rng.integers(0, nlist, n)
    b_i = rng.integers(0, nlist, n)
    q = n // 4
    y[:q] = 0.5 * (cent[a_i[:q]] + cent[b_i[:q]])
    y[q:2 * q] = 0.5 * (cent[a_i[q:2 * q]] + cent[b_i[q:2 * q]]) + \
        rng.standard_normal((q, d)).astype(np.float32) * 1e-6
    y[2 * q:2 * q + 16] = cent[a_i[2 * q:2 * q + 16]]
    y[2 * q + 16] = 0.0
    norms = po.cent_norms(cent)
    a = torch.empty((n,), dtype=torch.int32, device=gpu)
    jg.k_assign(_t(y, gpu), _t(cent, gpu), _t(norms, gpu), a)
    torch.cuda.synchronize()
    want = po.assign(y, cent, norms)
    got = a.cpu().numpy()
    assert np.array_equal(got, want), np.argwhere(got != want)[:5]


@pytest.mark.parametrize("B,nlist,P", [(5, 100, 7), (4, 4096, 16), (3, 5000, 64), (2, 8191, 512),
                                       (64, 65536, 64), (2, 65536, 1)])
def test_select_probes_exact_with_ties(gpu, B, nlist, P):
    """Probe lists in (score, list) order, exactly, through both the one-pass
    selection and the sliced selection used for large nlist; scores with many
    exact ties (small integers), so the tie rule decides most slots."""
    import torch
    rng = np.random.default_rng(B * nlist + P)
    scores = rng.integers(-40, 40, (B, nlist)).astype(np.float32)
    scores[scores == 0] = 0.5  # keep -0.0 / +0.0 out of the tie rule
    scores[0, nlist // 2:] = -100.0  # the winners sit in the later slices
    sizes = rng.integers(0, 50, nlist).astype(np.int32)
    probes = torch.empty((B, P), dtype=torch.int32, device=gpu)
    gofs = torch.empty((B, P + 1), dtype=torch.int32, device=gpu)
    qtot = torch.empty((B,), dtype=torch.int32, device=gpu)
    jg.k_select_probes(_t(scores, gpu), _t(sizes, gpu), P, probes, gofs, qtot)
    torch.cuda.synchronize()
    tags = np.arange(nlist, dtype=np.int32)
    want = np.stack([po.select_topk_pairs(scores[b], tags, P)[1] for b in range(B)])
    assert np.array_equal(probes.cpu().numpy(), want)
    groups = (sizes[want] + 15) // 16
    wg = np.concatenate([np.zeros((B, 1), np.int64), np.cumsum(groups, 1)], 1)
    assert np.array_equal(gofs.cpu().numpy(), wg)
    assert np.array_equal(qtot.cpu().numpy(), wg[:, -1])


@pytest.mark.parametrize("nlist,P", [(65536, 64), (4100, 16), (8192, 128), (8192, 200)])
def test_select_probes_clustered_top(gpu, nlist, P):
    """The row's best lists packed into one stride class (lists 4*(5 + 512*j)
    + r and 5 + 512*j, the share one thread reads in either load layout), so a
    per-thread shortcut alone would lose some of them; the result must still
    be the exact top P."""
    import torch
    B = 3
    rng = np.random.default_rng(nlist + P)
    scores = rng.standard_normal((B, nlist)).astype(np.float32) + 10.0
    hot = np.array(sorted({4 * (5 + 512 * j) + r for j in range(64) for r in range(4)} |
                          {5 + 512 * j for j in range(64)}))
    hot = hot[hot < nlist]
    scores[:, hot] = -rng.random((B, hot.size)).astype(np.float32)
    sizes = rng.integers(0, 50, nlist).astype(np.int32)
    probes = torch.empty((B, P), dtype=torch.int32, device=gpu)
    gofs = torch.empty((B, P + 1), dtype=torch.int32, device=gpu)
    qtot = torch.empty((B,), dtype=torch.int32, device=gpu)
    jg.k_select_probes(_t(scores, gpu), _t(sizes, gpu), P, probes, gofs, qtot)
    torch.cuda.synchronize()
    tags = np.arange(nlist, dtype=np.int32)
    want = np.stack([po.select_topk_pairs(scores[b], tags, P)[1] for b in range(B)])
    assert np.array_equal(probes.cpu().numpy(), want)
