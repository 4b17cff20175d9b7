#!/usr/bin/env python3
"""Writes tests/golden/jhq_golden.npz: known-answer vectors that pin the CPU
oracle (oracle/jhq_oracle.c) independently of the oracle itself.

Sources of the expected values
  * oracle/_ref/libjhq_ref.so — the reference's own host code
    (cpu/codebook.cpp, cpu/erfinv.h) compiled where it lies in the reference
    checkout by oracle/Makefile with the reference's host flags
    (-O3 -march=native, CMakeLists.txt:25), plus libstdc++'s std::mt19937 and
    std::normal_distribution<float> drawn exactly as cpu/jl_transform.cpp:27-29
    draws them:
      erfinv_f, LloydMaxCodebook (c1d, encode, build_flat_lut, build_lut,
      adc_distance, reconstruct), train_1d_kmeans, normal draws.
  * scipy.linalg.lapack.sgeqrf / sorgqr — the LAPACK routines the reference
    calls in JLTransform::build_rotation (cpu/jl_transform.cpp:35-53), applied
    to the libstdc++ Gaussian matrix: golden Q for d = 8, 64, 128.
  * scipy.special.ndtri — the closed form c1d/sigma = Phi^-1((i+1/2)/K1D)
    that the Winitzki erfinv approximates (cpu/codebook.cpp:60-80).

Run from the repository root after building oracle/_ref (make -C oracle ref):
    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
from scipy.linalg import lapack
from scipy.special import ndtri

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import pyoracle as po  # noqa: E402

OUT = os.path.join(HERE, "jhq_golden.npz")

# (d, M, B) -> K1D = 2^(B / (d/M)); one shape per codeword count
CB_SHAPES = [(64, 8, 8), (100, 25, 8), (32, 16, 8), (32, 32, 8), (48, 12, 4)]
SIGMAS = [0.03125, 0.7, 1.0]


def ref_lib():
    r = po.ref()
    if r is None:
        sys.exit("oracle/_ref/libjhq_ref.so is missing: run `make -C oracle ref` first")
    return r


def f32p(a):
    return a.ctypes.data_as(po._VP)


def main():
    r = ref_lib()
    g = {}

    # -- libstdc++ normal draws (drift detector for the rotation's input) ----
    for seed, n in ((42, 4096), (7, 1000)):
        out = np.empty(n, np.float32)
        r.ref_normal_fill(seed, f32p(out), n)
        g[f"normal_seed{seed}"] = out

    # -- erfinv_f ------------------------------------------------------------
    xs = np.concatenate([
        np.linspace(-0.999, 0.999, 181, dtype=np.float32),
        np.array([-0.5, 0.5, -1e-6, 1e-6, 0.0, 0.9999, -0.9999], np.float32),
    ])
    g["erfinv_x"] = xs
    g["erfinv_ref"] = np.array([r.ref_erfinv(float(x)) for x in xs], np.float32)

    # -- Lloyd-Max c1d, encode, LUTs, ADC, reconstruct ------------------------
    rng = np.random.default_rng(20240611)
    for (d, M, B) in CB_SHAPES:
        Ds = d // M
        K1D = 1 << (B // Ds)
        for si, sigma in enumerate(SIGMAS):
            tag = f"cb_d{d}_M{M}_B{B}_s{si}"
            c = np.empty(K1D, np.float32)
            r.ref_c1d(d, M, B, sigma, f32p(c))
            g[tag + "_c1d"] = c
            g[tag + "_ndtri"] = (ndtri((np.arange(K1D) + 0.5) / K1D) * sigma).astype(np.float64)
            n = 24
            y = (rng.standard_normal((n, d)) * sigma).astype(np.float32)
            y[0, :] = 0.0                       # exact midpoint for even K1D
            if K1D > 1:
                y[1, :] = 0.5 * (c[0] + c[1])   # exact midpoint of the first cell
            codes = np.empty((n, M), np.uint8)
            r.ref_encode(d, M, B, sigma, f32p(y), n, f32p(codes))
            g[tag + "_y"] = y
            g[tag + "_codes"] = codes
            q = (rng.standard_normal(d) * sigma).astype(np.float32)
            flat = np.empty((M, 256), np.float32)
            r.ref_flat_lut(d, M, B, sigma, f32p(q), f32p(flat))
            fac = np.empty(M * Ds * K1D, np.float32)
            r.ref_build_lut(d, M, B, sigma, f32p(q), f32p(fac))
            adc = np.array([r.ref_adc_distance(d, M, B, sigma, f32p(np.ascontiguousarray(codes[i])),
                                               f32p(fac)) for i in range(n)], np.float32)
            rec = np.empty((4, d), np.float32)
            for i in range(4):
                r.ref_reconstruct(d, M, B, sigma, f32p(np.ascontiguousarray(codes[i])),
                                  f32p(rec[i]))
            g[tag + "_q"] = q
            if si == 0:
                g[tag + "_flat_lut"] = flat
            g[tag + "_factored_lut"] = fac
            g[tag + "_adc_factored"] = adc
            g[tag + "_reconstruct4"] = rec

    # -- 1-D k-means ----------------------------------------------------------
    km_cases = [
        ("hand7", np.array([0.0, 0.1, 0.2, 5.0, 5.1, 9.0, 9.5], np.float32), 3),
        ("dups", np.array([1.0, 1.0, 1.0, 1.0, 2.0, 2.0, 3.0, 3.0, 3.0], np.float32), 4),
        ("kr_gt_n", np.array([3.0, -1.0, 2.0], np.float32), 5),
        ("normal1000", rng.standard_normal(1000).astype(np.float32), 16),
        ("laplace8000", rng.laplace(0.0, 0.05, 8000).astype(np.float32), 16),
        ("uniform5000_kr256", rng.uniform(-1, 1, 5000).astype(np.float32), 256),
        ("bimodal3000", np.concatenate([rng.normal(-1, 0.01, 1500),
                                        rng.normal(1, 0.01, 1500)]).astype(np.float32), 4),
    ]
    for name, vals, Kr in km_cases:
        out = np.empty(max(Kr, 1), np.float32)
        m = r.ref_train_1d_kmeans(f32p(vals), vals.size, Kr, 25, f32p(out))
        g[f"km_{name}_vals"] = vals
        g[f"km_{name}_Kr"] = np.int32(Kr)
        g[f"km_{name}_ref"] = out[:m].copy()

    # -- Householder QR against LAPACK sgeqrf / sorgqr ------------------------
    for d in (8, 64, 128):
        G = np.empty(d * d, np.float32)
        r.ref_normal_fill(42, f32p(G), d * d)
        A = np.asfortranarray(G.reshape(d, d, order="F"))
        qr, tau, _, info = lapack.sgeqrf(A)
        assert info == 0
        Q, _, info = lapack.sorgqr(qr, tau)
        assert info == 0
        g[f"qr_d{d}_Q_colmajor"] = np.asarray(Q, np.float32).reshape(-1, order="F")

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(g)} arrays)")


if __name__ == "__main__":
    main()
