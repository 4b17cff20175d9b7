"""Seeded synthetic data for tests: L2-normalised anisotropic Gaussian mixture,
the same family as the benchmark configs (smaller)."""
import numpy as np


def mixture(n, d, ncomp, seed, normalise=True, comp_seed=None):
    rng = np.random.default_rng(seed)
    crng = np.random.default_rng(seed + 7919 if comp_seed is None else comp_seed)
    means = crng.standard_normal((ncomp, d)).astype(np.float32)
    scales = np.exp(crng.uniform(np.log(0.1), np.log(1.0), (ncomp, d))).astype(np.float32)
    comp = rng.integers(0, ncomp, n)
    x = means[comp] + scales[comp] * rng.standard_normal((n, d)).astype(np.float32)
    if normalise:
        x /= np.linalg.norm(x, axis=1, keepdims=True)
    return np.ascontiguousarray(x, np.float32)


def queries_and_base(n, nq, d, ncomp, seed):
    """Base and query sets drawn from one mixture (shared components)."""
    base = mixture(n, d, ncomp, seed, comp_seed=seed + 1)
    q = mixture(nq, d, ncomp, seed + 100, comp_seed=seed + 1)
    return base, q


def byte_mixture(n, d, ncomp, seed, kind="uint8", comp_seed=None):
    """Byte-valued mixture rows like the 100M configs (smaller).  uint8:
    component means ~ N(34, 60^2) per coordinate plus N(0, 20^2) noise,
    rounded and clipped to 0..255 (about 30% zeros).  int8: means ~ N(0, 32^2)
    plus 16 * Student-t(nu=4) noise, clipped to -128..127."""
    rng = np.random.default_rng(seed)
    crng = np.random.default_rng(seed + 7919 if comp_seed is None else comp_seed)
    mu, sd = (34.0, 60.0) if kind == "uint8" else (0.0, 32.0)
    means = (mu + sd * crng.standard_normal((ncomp, d))).astype(np.float32)
    comp = rng.integers(0, ncomp, n)
    z = rng.standard_normal((n, d)).astype(np.float32)
    if kind == "uint8":
        x = means[comp] + 20.0 * z
        return np.clip(np.rint(x), 0, 255).astype(np.uint8)
    chi = (rng.standard_normal((n, d, 4)).astype(np.float32) ** 2).sum(2)
    x = means[comp] + 16.0 * z / np.sqrt(chi / 4.0)
    return np.clip(np.rint(x), -128, 127).astype(np.int8)
