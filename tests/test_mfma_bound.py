"""The re-check bound of the integer-MFMA pre-scan (mfma_plan_kernel and
mfma_recheck_kernel in jhq_gpu_amd/csrc/kernels.hip), pinned on the CPU.

With one-bit digits (K1D = 2, Ds = 8) the pre-scan rounds each query's
dl_k = (q_k - c1)^2 - (q_k - c0)^2 to integer steps of s = max|dl| / 32000,
splits the integers into int8 halves hi * 256 + lo, and ranks candidates by
the exact integer I(x) = sum_k b_k round(dl_k / s).  It then re-checks every
candidate with I(x) <= R(T), T the ck-th smallest I, where
    R(T) = (((1 + g)(C + s T + e) + ab) / (1 - g) + e - C) / s,
    e = s D / 2 (+ slack),  g = (M + 16) 2^-23.
These checks take the reference's fp32 distances from the oracle's byte LUT
and ADC (flat_lut / adc_flat, v14/search.cu:65-91,146-151) and confirm, on
random and adversarial queries, that
  * the int8 halves stay in range and I is the exact integer sum,
  * |C + s I(x) - a(x)| <= e and |a_ref(x) - a(x)| <= g a(x) with a(x) the
    distance in float64 (the two halves of the bound), with room to spare,
  * every candidate of the exact top-ck by (a_ref, position) is re-checked,
  * re-checking only I(x) <= T would miss candidates on these inputs."""
import numpy as np
import pytest

import pyoracle as po


def quantize(q, c1d):
    # the plan kernel's per-query arithmetic (float64)
    q = q.astype(np.float64)
    c0, c1 = float(c1d[0]), float(c1d[1])
    t0, t1 = q - c0, q - c1
    dl = t1 * t1 - t0 * t0
    C, sA, mx = float((t0 * t0).sum()), float(np.abs(dl).sum()), float(np.abs(dl).max())
    s = mx / 32000.0 if mx > 0 else 1.0
    iq = np.rint(dl / s).astype(np.int64)
    hi = (iq + 128) >> 8
    lo = iq - hi * 256
    e = 0.5000001 * s * q.size + 1e-12 * (C + sA)
    return dl, C, s, e, iq, hi, lo


def bound(C, s, e, T, M, use_e=True, use_g=True):
    g = (M + 16) * 2.0 ** -23 if use_g else 0.0
    ee = e if use_e else 0.0
    ab = 1e-30
    U = (1 + g) * (C + s * T + ee) + ab
    R = ((U + ab) / (1 - g) + ee - C) / s
    return np.floor(R + 1e-9 * abs(R) + 1.0)


def bits_of(codes):
    # bit k of code byte m is dimension 8 m + k
    return np.unpackbits(codes[:, :, None], axis=2, bitorder="little").reshape(codes.shape[0], -1)


def exact_topck(a_ref, ck):
    order = np.lexsort((np.arange(a_ref.size), a_ref))
    return order[:ck]


def make_case(kind, M, n, seed):
    rng = np.random.default_rng(seed)
    D = 8 * M
    sigma = np.float32(1.0)
    c1d = po.lloyd_max_c1d(sigma, 2)
    c0, c1 = float(c1d[0]), float(c1d[1])
    if kind == "gauss":
        q = rng.standard_normal(D).astype(np.float32)
        codes = rng.integers(0, 256, (n, M), dtype=np.uint8)
    elif kind == "near_codes":
        # candidates are small perturbations of the query's own sign pattern:
        # many distances bunch up near the minimum
        q = rng.standard_normal(D).astype(np.float32)
        base = (q.reshape(M, 8) > (c0 + c1) / 2)
        b = np.repeat(base[None], n, 0) ^ (rng.random((n, M, 8)) < 0.03)
        codes = np.packbits(b, axis=2, bitorder="little").reshape(n, M)
    elif kind == "offset":
        # large common offset: C dominates and the spread is small
        q = (rng.standard_normal(D) * 0.05 + 40.0).astype(np.float32)
        codes = rng.integers(0, 256, (n, M), dtype=np.uint8)
    elif kind == "midpoints":
        # query coordinates at the midpoint of c0 and c1: dl ~ 0 except a few
        q = np.full(D, (c0 + c1) / 2, np.float32)
        idx = rng.choice(D, 8, replace=False)
        q[idx] = rng.standard_normal(8).astype(np.float32) * 3
        codes = rng.integers(0, 256, (n, M), dtype=np.uint8)
    elif kind == "wide":
        q = (rng.standard_normal(D) * np.exp(rng.uniform(-8, 3, D))).astype(np.float32)
        codes = rng.integers(0, 256, (n, M), dtype=np.uint8)
    else:
        raise ValueError(kind)
    return q, c1d, codes


CASES = [("gauss", 16, 4000), ("gauss", 128, 3000), ("near_codes", 128, 3000),
         ("offset", 16, 4000), ("offset", 128, 3000), ("midpoints", 64, 3000),
         ("wide", 128, 3000), ("near_codes", 16, 4000)]


@pytest.mark.parametrize("kind,M,n", CASES)
def test_recheck_covers_exact_topck(kind, M, n):
    D = 8 * M
    worst_q, worst_r = 0.0, 0.0
    for rep in range(3):
        q, c1d, codes = make_case(kind, M, n, 1000 * M + 17 * rep + len(kind))
        dl, C, s, e, iq, hi, lo = quantize(q, c1d)
        assert hi.min() >= -128 and hi.max() <= 127 and lo.min() >= -128 and lo.max() <= 127
        assert np.array_equal(hi * 256 + lo, iq)
        assert np.abs(iq).max() <= 32000
        b = bits_of(codes).astype(np.int64)
        I = b @ iq
        assert np.array_equal(I, b @ hi * 256 + b @ lo)
        # the reference's distances: oracle byte LUT, then ADC in m order
        lut = po.flat_lut(q, M, c1d)
        a_ref = np.array([po.adc_flat(codes[i], lut) for i in range(n)], np.float64)
        x = po.reconstruct(codes, D, c1d).astype(np.float64)
        a = ((q.astype(np.float64)[None, :] - x) ** 2).sum(1)
        g = (M + 16) * 2.0 ** -23
        errq = np.abs(C + s * I - a).max()
        errr = (np.abs(a_ref - a) / np.maximum(a, 1e-300)).max()
        assert errq <= e, (errq, e)
        assert errr <= g, (errr, g)
        worst_q, worst_r = max(worst_q, errq / e), max(worst_r, errr / g)
        for ck in (10, 40, 100):
            top = exact_topck(a_ref, ck)
            T = np.sort(I)[ck - 1]
            members = I <= bound(C, s, e, T, M)
            assert members[top].all(), (kind, M, ck, np.count_nonzero(~members[top]))
            assert members.sum() >= ck
    # both halves of the bound are used well below their limits
    assert worst_q < 0.5 and worst_r < 0.5, (worst_q, worst_r)


def test_window_is_needed():
    """Rounding can reverse an order: x with four bits of dl = 0.45 s each
    (I = 0, a = 1.8 s above the base) against y with two bits of dl = 0.55 s
    (I = 2, a = 1.1 s).  y is the exact nearest, yet x has the smaller I;
    re-checking only I <= T + 1 would miss y, the window keeps it."""
    M, D = 16, 128
    c1d = po.lloyd_max_c1d(np.float32(1.0), 2)
    c0, c1 = float(c1d[0]), float(c1d[1])
    s0 = 1e-3
    dl = np.zeros(D)
    dl[0] = 32000 * s0              # sets the step s = s0
    dl[8:12] = 0.45 * s0            # subspace 1, bits 0..3
    dl[16:18] = 0.55 * s0           # subspace 2, bits 0..1
    # dl = (c0 - c1)(2 q - c0 - c1) is linear in q
    q = ((dl / (c0 - c1) + c0 + c1) / 2).astype(np.float32)
    codes = np.zeros((50, M), np.uint8)
    codes[0, 1] = 0x0f              # x
    codes[1, 2] = 0x03              # y
    codes[2:, 0] = 1                # far: bit 0 of subspace 0
    codes[2:, 3] = np.arange(48)
    _, C, s, e, iq, hi, lo = quantize(q, c1d)
    I = bits_of(codes).astype(np.int64) @ iq
    lut = po.flat_lut(q, M, c1d)
    a_ref = np.array([po.adc_flat(codes[i], lut) for i in range(codes.shape[0])], np.float64)
    assert exact_topck(a_ref, 1)[0] == 1 and I[0] < I[1]
    T = np.sort(I)[0]
    assert I[1] > bound(C, s, e, T, M, use_e=False, use_g=False)
    assert I[1] <= bound(C, s, e, T, M)
