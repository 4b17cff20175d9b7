"""Pins the oracle's functions that no reference build covers (the GPU-side
semantics of v14/encode.cu, v14/search.cu, v14/jhq_gpu_index.cu and the exact
selection of jhq_v3_ivf/search.cu) through brute force in float64 on tiny
inputs, closed forms and invariants.  The checkers are written independently
of the oracle's loops (vectorised numpy, argmin/argsort over everything), and
the `planted` tests show that each checker rejects a plausible mistake."""
import numpy as np
import pytest

import pyoracle as po
from datagen import queries_and_base


def nearest_brute(v, cb):
    """Nearest codeword by distance; an exact midpoint goes to the upper one
    (the reference's `v < mid ? left : right`, v14/encode.cu:6-18)."""
    v = np.asarray(v, np.float64)[..., None]
    cb = np.asarray(cb, np.float64)
    dd = np.abs(v - cb)
    best = dd.min(-1, keepdims=True)
    # among tied codewords take the largest index
    return (dd == best).cumsum(-1).argmax(-1)


# -- sigma (cpu/jl_transform.cpp:73-83) ---------------------------------------
def test_sigma_closed_form():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((300, 24)).astype(np.float32)
    want = np.sqrt((x.astype(np.float64) ** 2).sum() / x.size)
    assert abs(float(po.estimate_sigma(x)) - want) <= 1e-7 * want
    ones = np.full((5, 8), 0.5, np.float32)
    assert po.estimate_sigma(ones) == np.float32(0.5)


# -- rotation (v14/jhq_gpu_index.cu:444-448, search.cu:338-339) ---------------
@pytest.mark.parametrize("n,d", [(3, 8), (17, 64), (5, 256)])
def test_rotate_matches_float64_product(n, d):
    rng = np.random.default_rng(n + d)
    x = rng.standard_normal((n, d)).astype(np.float32)
    P = po.rotation_rowmajor(d, 42)
    y = po.rotate(P, x)
    want = x.astype(np.float64) @ P.astype(np.float64).T
    assert np.max(np.abs(y - want)) < 1e-5 * np.sqrt(d)
    # an orthogonal rotation keeps the norm
    assert np.allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-5)


def test_rotate_transposed_operand_is_caught():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 32)).astype(np.float32)
    P = po.rotation_rowmajor(32, 42)
    want = x.astype(np.float64) @ P.astype(np.float64).T
    planted = po.rotate(np.ascontiguousarray(P.T), x)   # Pi^T x instead of Pi x
    assert np.max(np.abs(planted - want)) > 1e-2


# -- primary encode (v14/encode.cu:20-41) -------------------------------------
@pytest.mark.parametrize("d,M,B", [(64, 8, 8), (100, 25, 8), (32, 16, 8), (32, 32, 8), (48, 12, 4)])
def test_primary_encode_brute_force(d, M, B):
    Ds = d // M
    bpd = B // Ds
    K1D = 1 << bpd
    c1d = po.lloyd_max_c1d(0.05, K1D)
    rng = np.random.default_rng(d * M)
    y = (rng.standard_normal((64, d)) * 0.05).astype(np.float32)
    y[0] = 0.0
    y[1, :] = 0.5 * (c1d[0] + c1d[-1])
    codes = po.primary_encode(y, M, c1d)
    dig = nearest_brute(y, c1d).reshape(64, M, Ds)
    want = (dig << (np.arange(Ds) * bpd)).sum(-1).astype(np.uint8)
    assert np.array_equal(codes, want)
    if K1D == 2:  # closed form: the bit is [y >= 0]
        bitsv = ((codes[:, :, None] >> np.arange(Ds)) & 1).reshape(64, d)
        assert np.array_equal(bitsv, (y >= 0).astype(np.uint8))


# -- residual encode (v14/encode.cu:43-86) ------------------------------------
def _unpack_res(res, d, Br):
    if Br == 8:
        return res[:, :d].astype(np.int64)
    r = np.empty((res.shape[0], 2 * res.shape[1]), np.int64)
    r[:, 0::2] = res & 0x0F       # even dimension -> low nibble
    r[:, 1::2] = res >> 4
    return r[:, :d]


@pytest.mark.parametrize("d,M,Br,Kr", [(64, 8, 4, 16), (33, 33, 4, 9), (32, 32, 8, 256), (100, 25, 4, 16)])
def test_residual_encode_brute_force(d, M, Br, Kr):
    Ds = d // M
    K1D = 1 << (8 // Ds)
    rng = np.random.default_rng(d + Br)
    y = (rng.standard_normal((50, d)) * 0.05).astype(np.float32)
    c1d = po.lloyd_max_c1d(0.05, K1D)
    rc = np.sort((rng.standard_normal(Kr) * 0.02).astype(np.float32))
    codes = po.primary_encode(y, M, c1d)
    res, corr = po.residual_encode(y, codes, M, c1d, rc, Br)
    assert res.shape == (50, (d * Br + 7) // 8)
    yhat = po.reconstruct(codes, d, c1d)
    r = (y - yhat).astype(np.float32)
    ri = _unpack_res(res, d, Br)
    assert np.array_equal(ri, nearest_brute(r, rc))
    if Br == 4 and d % 2:
        assert np.all(res[:, -1] >> 4 == 0)          # unused high nibble stays 0
    want = 2.0 * (yhat.astype(np.float64) * rc[ri].astype(np.float64)).sum(1)
    assert np.allclose(corr, want, rtol=1e-5, atol=1e-9)
    # the composite identity behind the returned distance (v14/search.cu:240):
    # ||q-yhat||^2 + ||q-rhat||^2 + 2<yhat,rhat> = ||q-(yhat+rhat)||^2 + ||q||^2
    q = rng.standard_normal(d) * 0.05
    rhat = rc[ri].astype(np.float64)
    lhs = ((q - yhat) ** 2).sum(1) + ((q - rhat) ** 2).sum(1) + corr
    rhs = ((q - (yhat + rhat)) ** 2).sum(1) + (q ** 2).sum()
    assert np.allclose(lhs, rhs, rtol=1e-5)


def test_per_subspace_residual_codebooks_brute_force():
    """Extension with no reference counterpart: dimension j is quantised with
    codebook j // Ds; pinned by brute force and by the one-codebook case."""
    d, M, Kr = 48, 12, 16
    Ds = d // M
    rng = np.random.default_rng(44)
    y = (rng.standard_normal((40, d)) * 0.05).astype(np.float32)
    c1d = po.lloyd_max_c1d(0.05, 1 << (8 // Ds))
    books = np.sort((rng.standard_normal((M, Kr)) * 0.02).astype(np.float32), axis=1)
    codes = po.primary_encode(y, M, c1d)
    res, corr = po.residual_encode(y, codes, M, c1d, books, 4)
    r = y - po.reconstruct(codes, d, c1d)
    ri = _unpack_res(res, d, 4)
    for j in range(d):
        assert np.array_equal(ri[:, j], nearest_brute(r[:, j], books[j // Ds]))
    rhat = books[np.arange(d)[None, :] // Ds, ri].astype(np.float64)
    yhat = po.reconstruct(codes, d, c1d).astype(np.float64)
    assert np.allclose(corr, 2.0 * (yhat * rhat).sum(1), rtol=1e-5, atol=1e-9)
    # M identical codebooks == the one shared codebook, bit for bit
    same = np.repeat(books[:1], M, axis=0)
    r1, c1 = po.residual_encode(y, codes, M, c1d, same, 4)
    r0, c0 = po.residual_encode(y, codes, M, c1d, books[0], 4)
    assert np.array_equal(r1, r0) and np.array_equal(c1.view(np.uint32), c0.view(np.uint32))


def test_residual_nibble_swap_is_caught():
    rng = np.random.default_rng(8)
    y = (rng.standard_normal((20, 16)) * 0.05).astype(np.float32)
    c1d = po.lloyd_max_c1d(0.05, 2)
    rc = np.sort((rng.standard_normal(16) * 0.02).astype(np.float32))
    codes = po.primary_encode(y, 2, c1d)
    res, _ = po.residual_encode(y, codes, 2, c1d, rc, 4)
    planted = ((res & 0x0F) << 4) | (res >> 4)       # high nibble for even j
    r = y - po.reconstruct(codes, 16, c1d)
    assert not np.array_equal(_unpack_res(planted, 16, 4), nearest_brute(r, rc))


# -- LUT and ADC (v14/search.cu:65-91, 146-151) -------------------------------
@pytest.mark.parametrize("d,M,B", [(64, 8, 8), (100, 25, 8), (32, 32, 8), (48, 12, 4)])
def test_flat_lut_and_adc_closed_form(d, M, B):
    Ds = d // M
    bpd = B // Ds
    K1D = 1 << bpd
    c1d = po.lloyd_max_c1d(0.05, K1D)
    rng = np.random.default_rng(d)
    q = (rng.standard_normal(d) * 0.05).astype(np.float32)
    lut = po.flat_lut(q, M, c1d)
    v = np.arange(256)
    for m in range(M):
        dig = (v[:, None] >> (np.arange(Ds) * bpd)) & (K1D - 1)
        want = ((q[m * Ds:(m + 1) * Ds][None, :].astype(np.float64) - c1d[dig]) ** 2).sum(1)
        assert np.allclose(lut[m], want, rtol=2e-6, atol=0)
    y = (rng.standard_normal((30, d)) * 0.05).astype(np.float32)
    codes = po.primary_encode(y, M, c1d)
    adc = np.array([po.adc_flat(codes[i], lut) for i in range(30)])
    yhat = po.reconstruct(codes, d, c1d).astype(np.float64)
    assert np.allclose(adc, ((q - yhat) ** 2).sum(1), rtol=1e-5)
    fac = po.factored_lut(q, M, c1d)
    adcf = np.array([po.adc_factored(codes[i], d, K1D, fac) for i in range(30)])
    assert np.allclose(adc, adcf, rtol=1e-6)


# -- IVF assignment / k-means (v14/jhq_gpu_index.cu:23-40, 228-299) -----------
def test_assign_brute_force_and_ties():
    rng = np.random.default_rng(11)
    y = rng.standard_normal((400, 16)).astype(np.float32)
    cent = rng.standard_normal((9, 16)).astype(np.float32)
    cent[7] = cent[2]                                  # exact duplicate: ties -> 2
    norms = po.cent_norms(cent)
    assert np.allclose(norms, (cent.astype(np.float64) ** 2).sum(1), rtol=1e-7)
    a = po.assign(y, cent, norms)
    s = norms[None, :].astype(np.float64) - 2.0 * y.astype(np.float64) @ cent.T.astype(np.float64)
    srt = np.sort(s, 1)
    clear = (srt[:, 1] - srt[:, 0]) > 1e-4 * np.abs(srt[:, 0]).clip(1.0)
    assert np.array_equal(a[clear], s.argmin(1)[clear])
    assert not np.any(a == 7)


def test_train_ivf_iteration_relation():
    rng = np.random.default_rng(12)
    y = rng.standard_normal((300, 8)).astype(np.float32)
    y[:40] += 6.0                                      # a dense clump
    nlist = 6
    c_t = po.train_ivf(y, nlist, 2)
    c_t1 = po.train_ivf(y, nlist, 3)
    a = po.assign(y, c_t, po.cent_norms(c_t))
    n = y.shape[0]
    for c in range(nlist):
        sel = a == c
        if sel.any():
            want = (y[sel].astype(np.float64).sum(0) / sel.sum()).astype(np.float32)
        else:  # reseed row (c*1103515245 + iter*12345) mod n, iter = 2
            want = y[(c * 1103515245 + 2 * 12345) % n]
        assert np.array_equal(c_t1[c], want)
    # initialisation: centroid c = row c*n/nlist
    c0 = po.train_ivf(y, nlist, 0)
    assert np.array_equal(c0, y[[c * n // nlist for c in range(nlist)]])
    with pytest.raises(ValueError):
        po.train_ivf(y[:4], nlist, 1)


def test_build_lists_stable():
    rng = np.random.default_rng(13)
    asg = rng.integers(0, 7, 500).astype(np.int32)
    asg[asg == 3] = 4                                  # an empty list
    off, order = po.build_lists(asg, 7)
    want = np.lexsort((np.arange(500), asg))
    assert np.array_equal(order, want)
    assert np.array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(asg, minlength=7))]))
    assert off[4] == off[3]


# -- exact selection (jhq_v3_ivf/search.cu:22-25, 189-279) --------------------
def test_select_topk_pairs_brute_force():
    rng = np.random.default_rng(14)
    dist = rng.integers(0, 20, 300).astype(np.float32)   # many exact ties
    tag = rng.permutation(300).astype(np.int32)
    dist[5] = np.inf
    od, ot = po.select_topk_pairs(dist, tag, 37)
    order = np.lexsort((tag, dist))[:37]
    assert np.array_equal(ot, tag[order]) and np.array_equal(od, dist[order])
    # k beyond the finite entries: (+inf, -1) padding
    od, ot = po.select_topk_pairs(dist[:10], tag[:10], 15)
    assert np.sum(ot == -1) == 6 and np.all(np.isinf(od[ot == -1]))
    assert po.ck_of(4.0, 10) == 40 and po.ck_of(0.5, 10) == 10 and po.ck_of(2.5, 3) == 8


# -- whole search (v14/search.cu:315-386 with exact selection) ----------------
def test_search_brute_force_tiny_index():
    d, M, nlist, nprobe, k = 32, 8, 8, 3, 5
    base, q = queries_and_base(1500, 12, d, 16, seed=21)
    o = po.OracleIndex(d, M=M, B=8, Br=4, alpha=4.0, nlist=nlist, nprobe=nprobe, ivf_iters=3,
                       seed=42)
    o.train(base[:800])
    o.add(base)
    r = o.search(q, k, debug=True)
    qr = q.astype(np.float64) @ o.P.astype(np.float64).T
    cent = o.cent.astype(np.float64)
    scores = o.cent_norms[None, :] - 2.0 * qr @ cent.T
    ck = po.ck_of(4.0, k)
    Ds = d // M
    for i in range(q.shape[0]):
        srt = np.sort(scores[i])
        if srt[nprobe] - srt[nprobe - 1] > 1e-5:
            assert set(r["probes"][i]) == set(np.argsort(scores[i], kind="stable")[:nprobe])
        pos = np.concatenate([np.arange(o.list_offsets[l], o.list_offsets[l + 1])
                              for l in r["probes"][i]])
        yhat = po.reconstruct(o.list_codes[pos], d, o.c1d).astype(np.float64)
        prim = ((qr[i] - yhat) ** 2).sum(1)
        order = np.lexsort((pos, prim))
        assert np.allclose(r["topck_dist"][i][:min(ck, pos.size)], prim[order][:ck], rtol=1e-5)
        # composite = ||q - (yhat + rhat)||^2 + ||q||^2 over the short list
        sl = r["topck_pos"][i]
        sl = sl[sl >= 0]
        ri = _unpack_res(o.list_res[sl], d, 4)
        xh = po.reconstruct(o.list_codes[sl], d, o.c1d).astype(np.float64) + o.res_c1d[ri]
        comp = ((qr[i] - xh) ** 2).sum(1) + (qr[i] ** 2).sum()
        ids = o.list_ids[sl]
        fo = np.lexsort((ids, comp))[:k]
        assert np.allclose(r["dists"][i], comp[fo], rtol=1e-5)
        gaps = np.diff(np.sort(comp)[:k + 1]) > 1e-5 * comp.max()
        if gaps.all():
            assert np.array_equal(r["ids"][i], ids[fo])
    del Ds


def test_search_k_exceeds_candidates_pads():
    d, M = 16, 4
    base, q = queries_and_base(64, 3, d, 4, seed=2)
    o = po.OracleIndex(d, M=M, B=8, Br=4, alpha=1.0, nlist=4, nprobe=1, ivf_iters=2, seed=42)
    o.train(base)
    o.add(base)
    dist, ids = o.search(q, 200)
    for i in range(3):
        nfill = int(np.sum(ids[i] >= 0))
        assert nfill <= 64 and np.all(ids[i][nfill:] == -1)
        assert np.all(np.isinf(dist[i][nfill:])) and np.all(np.diff(dist[i][:nfill]) >= 0)


# -- the reference's approximate top-ck (jhq_v14_streaming_add/search.cu:105-195) --
class _P:
    """Params of a hand-built flat index (one list)."""
    M, B, Br, nlist, nprobe, ivf_iters, residual_per_subspace = 1, 8, 4, 1, 1, 1, 0

    def __init__(self, alpha):
        self.alpha = alpha


def _hand_index(codes, alpha):
    """d = 8, one subspace of 8 one-bit dimensions (code bit t picks
    c1d[(v >> t) & 1] = -1 or +1), identity rotation, zero residual codebook
    and corrections: a candidate's primary distance to q = (+1, ..., +1) is 4x
    the number of zero bits of its code."""
    n = len(codes)
    d = 8
    return po.OracleIndex.from_state(
        d, _P(alpha), np.eye(d, dtype=np.float32), np.array([-1.0, 1.0], np.float32),
        np.zeros(16, np.float32), np.zeros((1, d), np.float32), np.zeros(1, np.float32),
        np.array([0, n], np.int32), np.arange(n, dtype=np.int32),
        np.asarray(codes, np.uint8).reshape(n, 1), np.zeros((n, 4), np.uint8),
        np.zeros(n, np.float32))


def test_reference_selection_drops_a_threads_fifth_candidate():
    """Known answer worked out by hand from the reference's selection: 256
    threads stride the candidates, each keeps its 4 best (a candidate enters
    only if strictly below the fourth), and each of the ck rounds takes a
    block argmin: thread t scans slots t, t + 256, ... of the 1024 kept values
    (slot 4 t + i = thread t's i-th), then a halving tree keeps the left value
    on ties.  Five distance-0 candidates sit on thread 0's stride (positions
    0, 256, 512, 768, 1024): exact selection returns the five; the reference's
    keeps only the first four (slots 0-3).  Round 1 takes slot 0.  Round 2:
    slots 1, 2, 3 tie; the tree pairs thread 0's side (now holding thread
    2's 0 after the stride-2 step) against thread 1's, keeping the left:
    slot 2 (position 512); round 3 slot 1 (256); round 4 slot 3 (768).  Round 5
    among the distance-4 candidates at positions 1 (slot 4, scanned by thread
    4), 2 (slot 8, thread 8) and 300 (thread 44's slot 176, thread 176): the
    stride-128 step moves thread 176's 4 to thread 48, stride 32 to thread 16,
    stride 16 to thread 0, which keeps it against thread 4's equal value at
    stride 4: position 300."""
    n = 1300
    codes = np.full(n, 0x0F, np.uint8)          # four zero bits: distance 16
    codes[[0, 256, 512, 768, 1024]] = 0xFF       # distance 0
    codes[[1, 2, 300]] = 0xFE                    # one zero bit: distance 4
    o = _hand_index(codes, alpha=1.0)
    q = np.ones((1, 8), np.float32)
    pr = np.zeros((1, 1), np.int32)
    ex = o.search(q, 5, debug=True, q_rot=q, probes=pr, mode=0)
    ap = o.search(q, 5, debug=True, q_rot=q, probes=pr, mode=1)
    assert list(ex["topck_pos"][0]) == [0, 256, 512, 768, 1024]
    assert list(ex["topck_dist"][0]) == [0.0] * 5
    assert list(ap["topck_pos"][0]) == [0, 512, 256, 768, 300]
    assert list(ap["topck_dist"][0]) == [0.0, 0.0, 0.0, 0.0, 4.0]


def test_reference_selection_is_exact_with_one_candidate_per_thread():
    """With at most 256 candidates every thread holds at most one, so the
    reference's selection keeps all of them: its ck distances are exactly the
    ck smallest (the same values as exact selection), and the two short lists
    hold the same candidates below the ck-th distance (at that distance a tie
    may be broken another way: the argmin tree, not the position, decides)."""
    rng = np.random.default_rng(11)
    codes = rng.integers(0, 256, 250).astype(np.uint8)
    codes[rng.integers(0, 250, 40)] = 0xF0  # many equal distances
    o = _hand_index(codes, alpha=4.0)
    q = np.ones((1, 8), np.float32)
    pr = np.zeros((1, 1), np.int32)
    ex = o.search(q, 10, debug=True, q_rot=q, probes=pr, mode=0)
    ap = o.search(q, 10, debug=True, q_rot=q, probes=pr, mode=1)
    de, da = ex["topck_dist"][0], ap["topck_dist"][0]
    assert np.array_equal(np.sort(de).view(np.uint32), np.sort(da).view(np.uint32))
    last = de.max()
    assert set(ex["topck_pos"][0][de < last]) == set(ap["topck_pos"][0][da < last])
    # and the brute-force distances: 4 x the number of zero bits
    zeros = np.array([8 - bin(int(c)).count("1") for c in codes])
    assert np.array_equal(np.sort(de), np.sort(4.0 * zeros)[:de.size].astype(np.float32))
