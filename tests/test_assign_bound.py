"""The re-check bound of the MFMA IVF assignment (jhq_gpu_amd/csrc/assign_mfma.hip).

A row's MFMA scores and its fixed-order scores (fmaf chain in k order, then
fmaf(-2, dot, ||c||^2)) may differ only by summation order and rounding; the
kernel accepts the MFMA argmin when the gap between the two best MFMA scores
exceeds 2E with
    E = 4 * ((4 (K + 4) + 5) u ||y|| Cmax + 3 u Nmax),   u = 2^-24.
These CPU checks pin that E bounds |score(order A) - score(order B)| for
orders an MFMA can take (4-term groups added to the accumulator, groups in
any order, k interleaved across lane groups), with the factor 4 of headroom
left unused: the observed difference stays below E / 4 on data built to make
cancellation large (offset means, mixed signs, wide dynamic range)."""
import numpy as np
import pytest

U = 2.0 ** -24


def fma32(a, b, c):
    # float32 fused multiply-add: the float64 product of two float32 values is
    # exact; the one rounding left is the float32 rounding of the sum
    return np.float32(np.float64(a) * np.float64(b) + np.float64(c))


def chain_dot(y, c, order):
    acc = np.float32(0.0)
    for k in order:
        acc = fma32(y[k], c[k], acc)
    return acc


def grouped_dot(y, c, groups):
    # one MFMA k-step: the accumulator plus four products, each step rounded
    acc = np.float32(0.0)
    for g in groups:
        s = np.float64(acc)
        for k in g:
            s = np.float64(np.float32(s + np.float64(y[k]) * np.float64(c[k])))
        acc = np.float32(s)
    return acc


def score(dot, norm):
    return fma32(np.float32(-2.0), dot, norm)


def bound(y, cmax, nmax, K):
    ny = np.sqrt(np.sum(y.astype(np.float64) ** 2)) * (1 + 4 * U)
    nm = nmax * (1 + 4 * U)
    cm = np.sqrt(nm)
    return 4.0 * ((4.0 * (K + 4) + 5.0) * U * ny * cm + 3.0 * U * nm)


@pytest.mark.parametrize("K,offset,spread", [(128, 100.0, 30.0), (100, 0.0, 1.0),
                                            (1024, 0.0, 1.0), (768, 5.0, 1e3)])
def test_order_difference_within_quarter_bound(K, offset, spread):
    rng = np.random.default_rng(K + int(offset))
    rows, cols = 24, 24
    y = (rng.standard_normal((rows, K)) * spread + offset).astype(np.float32)
    c = (rng.standard_normal((cols, K)) * spread + offset).astype(np.float32)
    c[:, ::7] *= -1.0  # mixed signs: cancellation in the dots
    norms = np.array([np.float32(np.sum(cc.astype(np.float64) ** 2)) for cc in c])
    nmax = float(norms.max())
    cmax = np.sqrt(nmax)
    worst = 0.0
    for i in range(rows):
        E = bound(y[i], cmax, nmax, K)
        for j in range(cols):
            fixed = score(chain_dot(y[i], c[j], range(K)), norms[j])
            # MFMA-like: lane group g holds k = 16 s + 4 g + e, steps in order
            groups = [[16 * s + 4 * g + e for g in range(4) if 16 * s + 4 * g + e < K]
                      for s in range((K + 15) // 16) for e in range(4)]
            groups = [gr for gr in groups if gr]
            alt1 = score(grouped_dot(y[i], c[j], groups), norms[j])
            perm = rng.permutation(K)
            alt2 = score(chain_dot(y[i], c[j], perm), norms[j])
            d = max(abs(float(fixed) - float(alt1)), abs(float(fixed) - float(alt2)))
            worst = max(worst, d / E)
    assert worst < 0.25, worst


def test_bound_catches_a_dropped_term():
    """A plausible kernel mistake (one product left out) moves a score by far
    more than E, so the acceptance test could not hide it."""
    rng = np.random.default_rng(5)
    K = 128
    y = rng.standard_normal(K).astype(np.float32)
    c = rng.standard_normal(K).astype(np.float32)
    norm = np.float32(np.sum(c.astype(np.float64) ** 2))
    E = bound(y, np.sqrt(float(norm)), float(norm), K)
    good = score(chain_dot(y, c, range(K)), norm)
    bad = score(chain_dot(y, c, range(1, K)), norm)
    assert abs(float(good) - float(bad)) > 10 * E
