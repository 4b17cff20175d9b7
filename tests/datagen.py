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
