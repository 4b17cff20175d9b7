"""Pins the CPU oracle (oracle/jhq_oracle.c) against known answers that do not
come from the oracle: the committed golden vectors of tests/golden/ (written by
tests/golden/make_golden.py from the reference's own cpu/codebook.cpp build,
libstdc++'s RNG and scipy's LAPACK / ndtri), the C++ standard's mt19937 known
answer, and — when oracle/_ref/libjhq_ref.so is present — the reference code
itself on fresh inputs.

Each test names the reference function it pins (file:line)."""
import os

import numpy as np
import pytest

import pyoracle as po

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "jhq_golden.npz")
CB_SHAPES = [(64, 8, 8), (100, 25, 8), (32, 16, 8), (32, 32, 8), (48, 12, 4)]
SIGMAS = [0.03125, 0.7, 1.0]


@pytest.fixture(scope="module")
def g():
    return np.load(GOLDEN)


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


# -- RNG (cpu/jl_transform.cpp:27-29) ----------------------------------------
def test_mt19937_known_answer():
    # C++ [rand.predef]: the 10000th invocation of a default-constructed
    # std::mt19937 (seed 5489) produces 4123659995.
    assert int(po.mt_fill(5489, 10000)[-1]) == 4123659995


@pytest.mark.parametrize("seed,n", [(42, 4096), (7, 1000)])
def test_normal_draws_match_libstdcxx(g, seed, n):
    assert np.array_equal(bits(po.normal_fill(seed, n)), bits(g[f"normal_seed{seed}"]))


# -- erfinv / Lloyd-Max (cpu/erfinv.h:7-27, cpu/codebook.cpp:60-80) ----------
def test_erfinv_bit_exact_vs_reference(g):
    got = np.array([po.erfinv(x) for x in g["erfinv_x"]], np.float32)
    assert np.array_equal(bits(got), bits(g["erfinv_ref"]))


def test_erfinv_special_values():
    assert po.erfinv(0.0) == 0.0
    assert po.erfinv(1.0) == np.inf and po.erfinv(-1.0) == -np.inf
    assert po.erfinv(-0.3) == -po.erfinv(0.3)


@pytest.mark.parametrize("shape", CB_SHAPES, ids=[f"d{d}M{m}B{b}" for d, m, b in CB_SHAPES])
@pytest.mark.parametrize("si", range(len(SIGMAS)))
def test_c1d_reference_and_closed_form(g, shape, si):
    d, M, B = shape
    tag = f"cb_d{d}_M{M}_B{B}_s{si}"
    K1D = 1 << (B // (d // M))
    c = po.lloyd_max_c1d(SIGMAS[si], K1D)
    assert np.array_equal(bits(c), bits(g[tag + "_c1d"]))
    # Winitzki + one Newton step: ~1e-5 relative of the exact Gaussian quantile
    nd = g[tag + "_ndtri"]
    assert np.allclose(c, nd, rtol=2e-5, atol=1e-7 * SIGMAS[si])
    assert np.all(np.diff(c) > 0) and np.allclose(c, -c[::-1], rtol=1e-6, atol=1e-9)


def test_c1d_known_quantiles():
    # Phi^-1(3/4) = 0.6744898, Phi^-1(5/8) = 0.3186394, Phi^-1(7/8) = 1.1503494
    assert np.allclose(po.lloyd_max_c1d(1.0, 2), [-0.6744898, 0.6744898], rtol=1e-5)
    assert np.allclose(po.lloyd_max_c1d(1.0, 4), [-1.1503494, -0.3186394, 0.3186394, 1.1503494],
                       rtol=1e-5)


# -- encode / LUT / ADC (cpu/codebook.cpp:96-171, v14/encode.cu:20-41) -------
@pytest.mark.parametrize("shape", CB_SHAPES, ids=[f"d{d}M{m}B{b}" for d, m, b in CB_SHAPES])
@pytest.mark.parametrize("si", range(len(SIGMAS)))
def test_encode_lut_adc_vs_reference(g, shape, si):
    d, M, B = shape
    tag = f"cb_d{d}_M{M}_B{B}_s{si}"
    c1d = g[tag + "_c1d"]
    K1D = c1d.size
    y = g[tag + "_y"]
    codes = po.primary_encode(y, M, c1d)
    assert np.array_equal(codes, g[tag + "_codes"])
    q = g[tag + "_q"]
    fac = po.factored_lut(q, M, c1d)
    assert np.array_equal(bits(fac), bits(g[tag + "_factored_lut"]))
    if tag + "_flat_lut" in g.files:
        # The oracle's flat LUT follows the GPU kernel (v14/search.cu:65-91):
        # nvcc --use_fast_math contracts `sum += diff*diff` into an fma chain.
        # The reference's host twin build_flat_lut (cpu/codebook.cpp:112-129)
        # is fused or not depending on how g++ -O3 -march=native vectorises
        # the k loop for each Ds (for Ds=8 it squares all differences in one
        # vector op and adds them unfused).  Both orders agree to within Ds
        # rounding steps, which is what is asserted.
        ref_flat = g[tag + "_flat_lut"]
        Ds = d // M
        flat = po.flat_lut(q, M, c1d)
        assert np.all(np.abs(flat.astype(np.float64) - ref_flat) <=
                      Ds * np.spacing(np.abs(ref_flat)).astype(np.float64))
        # byte LUT == flat expansion of the factored LUT: a dropped or
        # misindexed digit would move entries by a whole term, far beyond this
        assert np.allclose(flat, ref_flat, rtol=1e-6, atol=0)
    adc = np.array([po.adc_factored(codes[i], d, K1D, fac) for i in range(codes.shape[0])],
                   np.float32)
    assert np.array_equal(bits(adc), bits(g[tag + "_adc_factored"]))
    rec = po.reconstruct(codes[:4], d, c1d)
    assert np.array_equal(bits(rec), bits(g[tag + "_reconstruct4"]))


# -- 1-D k-means (cpu/codebook.cpp:8-58) --------------------------------------
KM = ["hand7", "dups", "kr_gt_n", "normal1000", "laplace8000", "uniform5000_kr256", "bimodal3000"]


@pytest.mark.parametrize("name", KM)
def test_train_1d_kmeans_vs_reference(g, name):
    vals = g[f"km_{name}_vals"]
    Kr = int(g[f"km_{name}_Kr"])
    got = po.train_1d_kmeans(vals, Kr)
    assert np.array_equal(bits(got), bits(g[f"km_{name}_ref"]))


def test_train_1d_kmeans_hand_case():
    # quantile init picks sorted[int((i+0.5)/3*7)] = sorted[1], [3], [5]
    # = 0.1, 5.0, 9.0; Lloyd converges to {0.1}, {5.05}, {9.25}.
    c = po.train_1d_kmeans(np.array([0.0, 0.1, 0.2, 5.0, 5.1, 9.0, 9.5], np.float32), 3)
    assert np.allclose(c, [0.1, 5.05, 9.25], rtol=1e-6)
    # Kr > n clamps Kr to n: the codewords are the points themselves
    c = po.train_1d_kmeans(np.array([3.0, -1.0, 2.0], np.float32), 5)
    assert np.array_equal(c, np.array([-1.0, 2.0, 3.0], np.float32))


def test_train_1d_kmeans_fixed_point():
    rng = np.random.default_rng(5)
    v = rng.standard_normal(4000).astype(np.float32)
    c = po.train_1d_kmeans(v, 8, max_iter=200)
    assert np.all(np.diff(c) > 0)
    # converged: every codeword is the (double) mean of its midpoint cell
    mids = 0.5 * (c[:-1] + c[1:])
    cell = np.searchsorted(mids, v, side="right")
    for i in range(c.size):
        assert np.float32(v[cell == i].astype(np.float64).mean()) == c[i]


# -- QR rotation (cpu/jl_transform.cpp:25-56) ---------------------------------
@pytest.mark.parametrize("d", [8, 64, 128])
def test_qr_matches_lapack(g, d):
    Q = po.build_rotation(d, 42)
    ref = g[f"qr_d{d}_Q_colmajor"]
    # LAPACK sgeqrf/sorgqr in fp32 vs this restatement in fp64: same column signs
    assert np.max(np.abs(Q - ref)) < 1e-5 * np.sqrt(d)
    assert np.all(np.sign(Q.reshape(d, d)[0]) == np.sign(ref.reshape(d, d)[0]))


@pytest.mark.parametrize("d", [16, 100, 256])
def test_qr_invariants(d):
    G = po.normal_fill(42, d * d)
    Q = po.householder_qr(G, d).reshape(d, d).T        # row-major view of column-major Q
    Qd = Q.astype(np.float64)
    assert np.max(np.abs(Qd.T @ Qd - np.eye(d))) < 1e-5
    # R = Q^T G is upper triangular with a positive-or-negative diagonal fixed by
    # the LAPACK convention beta = -sign(alpha) * norm: diag(R) has sign -sign(G[k,k]) for
    # the first column
    Gm = G.reshape(d, d).T.astype(np.float64)
    R = Qd.T @ Gm
    assert np.max(np.abs(np.tril(R, -1))) < 1e-4
    assert np.sign(R[0, 0]) == -np.sign(Gm[0, 0])
    assert np.max(np.abs(Qd @ R - Gm)) < 1e-4


def test_rotation_known_seed_is_stable():
    P1 = po.rotation_rowmajor(32, 42)
    P2 = po.rotation_rowmajor(32, 42)
    P3 = po.rotation_rowmajor(32, 43)
    assert np.array_equal(P1, P2) and not np.array_equal(P1, P3)


# -- the reference code itself on fresh inputs (when oracle/_ref is built) ---
def test_fresh_inputs_vs_reference_build():
    # checked at run time, so collecting this module never loads the library
    if not os.path.exists(po.REF_LIB):
        pytest.skip("oracle/_ref/libjhq_ref.so not built")
    r = po.ref()
    if r is None:
        pytest.skip("oracle/_ref/libjhq_ref.so does not load")
    rng = np.random.default_rng(99)
    for (d, M, B) in CB_SHAPES:
        sigma = 0.05
        K1D = 1 << (B // (d // M))
        c_ref = np.empty(K1D, np.float32)
        r.ref_c1d(d, M, B, sigma, c_ref.ctypes.data_as(po._VP))
        assert np.array_equal(bits(po.lloyd_max_c1d(sigma, K1D)), bits(c_ref))
        y = (rng.standard_normal((200, d)) * sigma).astype(np.float32)
        codes = np.empty((200, M), np.uint8)
        r.ref_encode(d, M, B, sigma, y.ctypes.data_as(po._VP), 200, codes.ctypes.data_as(po._VP))
        assert np.array_equal(po.primary_encode(y, M, c_ref), codes)
    vals = (rng.standard_normal(30000) * 0.01).astype(np.float32)
    out = np.empty(16, np.float32)
    m = r.ref_train_1d_kmeans(vals.ctypes.data_as(po._VP), vals.size, 16, 25,
                              out.ctypes.data_as(po._VP))
    assert np.array_equal(bits(po.train_1d_kmeans(vals, 16)), bits(out[:m]))
