"""The re-check bound of the MFMA IVF assignment (jhq_gpu_amd/csrc/assign_mfma.hip).

The first pass splits every float x into two bf16 (hi = bf16(x), lo =
bf16(x - hi)) and sums hi*hi + hi*lo + lo*hi with bf16 MFMAs accumulating in
fp32; the fixed-order pass is an fmaf chain in k order, then fmaf(-2, dot,
||c||^2).  The kernel accepts the first pass's argmin when the gap between
its two best scores exceeds 2E with
    e_dot = (2u * 1.02 * 33 * 3 * dp/32 + 3.01 * 2^-16 + (d + 4) u) ||y|| Cmax
    E = 2 (2 e_dot + 2u Nmax + 4u ||y|| Cmax) + 6d (2^-126 (||y|| + Cmax) + 2^-149)
(u = 2^-24, dp = d rounded up to 32).  These CPU checks pin that E bounds the
difference of the two passes' scores for accumulation orders an MFMA can take
(one rounding per instruction of 32 products, or a rounding after every
product in any order inside the instruction; the three product sums
interleaved as the kernel issues them), with the factor 2 of headroom left
unused: the observed difference stays below E / 4 on data built to make
cancellation large (offset means, mixed signs, wide dynamic range); and that
gross kernel mistakes (a skipped k step, a lane group's k values left out, an
operand off by one in k) move a score by far more than E."""
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


def bf16(x):
    # float32 -> bf16 (round to nearest even), returned as float32
    b = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def split(x):
    hi = bf16(x)
    lo = bf16((x - hi).astype(np.float32))  # x - hi is exact in float32
    return hi, lo


def mfma_dot(y, c, rng, mode, skip_step=None, drop_group=None):
    """The first pass's dot: steps of 32 k, three instructions per step
    (hi*hi, hi*lo, lo*hi), each adding its 32 exact products to the fp32
    accumulator.  mode 'one': one rounding per instruction; 'seq': a
    rounding after every product, in a random order inside the
    instruction."""
    K = y.shape[0]
    dp = (K + 31) // 32 * 32
    yp = np.zeros(dp, np.float32)
    cp = np.zeros(dp, np.float32)
    yp[:K], cp[:K] = y, c
    yh, yl = split(yp)
    ch, cl = split(cp)
    acc = np.float32(0.0)
    for s in range(dp // 32):
        if s == skip_step:
            continue
        ks = np.arange(32 * s, 32 * s + 32)
        if drop_group is not None:
            ks = ks[(ks % 32) // 8 != drop_group]
        for a, b in ((yh, ch), (yh, cl), (yl, ch)):
            p = a[ks].astype(np.float64) * b[ks].astype(np.float64)  # exact
            if mode == "one":
                acc = np.float32(np.float64(acc) + p.sum())
            else:
                for v in p[rng.permutation(len(p))]:
                    acc = np.float32(np.float64(acc) + v)
    return acc


def score(dot, norm):
    return fma32(np.float32(-2.0), dot, norm)


def bound(y, cmax, nmax, K):
    ny = np.sqrt(np.sum(y.astype(np.float64) ** 2)) * (1 + 4 * U)
    nm = nmax * (1 + 4 * U)
    cm = np.sqrt(nm)
    steps = (K + 31) // 32
    e_dot = (2 * U * 1.02 * 33 * 3 * steps + 3.01 / 65536.0 + (K + 4) * U) * ny * cm
    tiny = 6.0 * K * (2.0 ** -126 * (ny + cm) + 2.0 ** -149)
    return 2.0 * (2.0 * e_dot + 2.0 * U * nm + 4.0 * U * ny * cm) + tiny


def make(K, offset, spread, seed, rows=16, cols=16):
    rng = np.random.default_rng(seed)
    y = (rng.standard_normal((rows, K)) * spread + offset).astype(np.float32)
    c = (rng.standard_normal((cols, K)) * spread + offset).astype(np.float32)
    c[:, ::7] *= -1.0  # mixed signs: cancellation in the dots
    y[:, 3::11] *= np.float32(1e-3)  # wide dynamic range inside a row
    norms = np.array([np.float32(np.sum(cc.astype(np.float64) ** 2)) for cc in c])
    return rng, y, c, norms


@pytest.mark.parametrize("K,offset,spread", [(128, 100.0, 30.0), (100, 0.0, 1.0),
                                            (1024, 0.0, 1.0), (768, 5.0, 1e3)])
def test_order_difference_within_quarter_bound(K, offset, spread):
    rng, y, c, norms = make(K, offset, spread, K + int(offset))
    nmax = float(norms.max())
    cmax = np.sqrt(nmax)
    worst = 0.0
    for i in range(y.shape[0]):
        E = bound(y[i], cmax, nmax, K)
        for j in range(c.shape[0]):
            fixed = score(chain_dot(y[i], c[j], range(K)), norms[j])
            for mode in ("one", "seq"):
                alt = score(mfma_dot(y[i], c[j], rng, mode), norms[j])
                worst = max(worst, abs(float(fixed) - float(alt)) / E)
    assert worst < 0.25, worst


def test_split_is_within_two_to_minus_16():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(4096) * np.exp(rng.uniform(-30, 30, 4096))).astype(np.float32)
    hi, lo = split(x)
    err = np.abs(x.astype(np.float64) - hi.astype(np.float64) - lo.astype(np.float64))
    assert np.all(err <= 2.0 ** -16 * np.abs(x.astype(np.float64)))
    # hi is bf16(x) itself: 8 significant bits, nearest (unit roundoff 2^-8)
    assert np.all(np.abs(x.astype(np.float64) - hi) <= 2.0 ** -8 * np.abs(x.astype(np.float64)))


@pytest.mark.parametrize("mistake", ["skip_step", "drop_group", "shift"])
def test_bound_catches_gross_mistakes(mistake):
    """Plausible kernel mistakes move a score by far more than E, so the
    acceptance test could not hide them."""
    rng = np.random.default_rng(5)
    K = 256
    y = rng.standard_normal(K).astype(np.float32)
    c = rng.standard_normal(K).astype(np.float32)
    norm = np.float32(np.sum(c.astype(np.float64) ** 2))
    E = bound(y, np.sqrt(float(norm)), float(norm), K)
    good = score(chain_dot(y, c, range(K)), norm)
    if mistake == "skip_step":
        bad = score(mfma_dot(y, c, rng, "one", skip_step=3), norm)
    elif mistake == "drop_group":
        bad = score(mfma_dot(y, c, rng, "one", drop_group=1), norm)
    else:
        bad = score(mfma_dot(y, np.roll(c, 1), rng, "one"), norm)
    assert abs(float(good) - float(bad)) > 4 * E
