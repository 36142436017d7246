"""Error bounds of the split fp16 products used by the chunked GDN prefill
(kraken-infer_amd/csrc/gdn_chunked.hip: split_f16, mfma_split).

A value x is held as hi = f16(x) (zero below the smallest normal f16, 2^-14)
and lo = f16((x - hi) * 2^11); a product of two such values is summed as
hi*hi + 2^-11 (hi*lo + lo*hi).  The kernel's matrix-core inputs may flush f16
denormals, so every check here runs with f16 denormals flushed to zero, the
worst case.  CPU only: the GPU tests hold the kernels to 1e-4 of the oracle.
"""
import numpy as np

MIN_NORMAL = 2.0 ** -14


def ftz(h):
    h = np.asarray(h, np.float64)
    return np.where(np.abs(h) < MIN_NORMAL, 0.0, h)


def split(x, flush_hi=True):
    x = np.asarray(x, np.float32).astype(np.float64)
    src = np.where(np.abs(x) < MIN_NORMAL, 0.0, x) if flush_hi else x
    hi = src.astype(np.float16).astype(np.float64)
    lo = ((x - hi) * 2048.0).astype(np.float32).astype(np.float16).astype(np.float64)
    return ftz(hi), ftz(lo)


def split_dot(a, b, flush_hi=True):
    ah, al = split(a, flush_hi)
    bh, bl = split(b, flush_hi)
    return ah @ bh + (ah @ bl + al @ bh) / 2048.0


def test_representation_error_over_magnitudes():
    rng = np.random.default_rng(0)
    mags = 10.0 ** rng.uniform(-9, 4, 200000)
    x = (mags * rng.choice([-1.0, 1.0], mags.size)).astype(np.float32)
    hi, lo = split(x)
    err = np.abs(x.astype(np.float64) - (hi + lo / 2048.0))
    # 2^-21 relative from rounding lo, plus at most a flushed denormal lo (2^-25).
    assert np.all(err <= 2.0 ** -21 * np.abs(x) + 2.0 ** -25)


def test_products_within_two_to_minus_19():
    """Relative 2^-19 of sum |a||b|, plus 2^-25 per unit of the other operand
    for entries below 2^-14 (carried by lo alone, at f16 precision)."""
    rng = np.random.default_rng(1)
    for n in (32, 128, 64):
        a = (rng.standard_normal((64, n)) * 10.0 ** rng.uniform(-3, 1, (64, 1))).astype(np.float32)
        b = (rng.standard_normal((n, 16)) * 10.0 ** rng.uniform(-3, 1, (1, 16))).astype(np.float32)
        exact = a.astype(np.float64) @ b.astype(np.float64)
        aa, bb = np.abs(a).astype(np.float64), np.abs(b).astype(np.float64)
        bound = 2.0 ** -19 * (aa @ bb) + 2.0 ** -25 * (aa.sum(1, keepdims=True) + bb.sum(0))
        assert np.all(np.abs(split_dot(a, b) - exact) <= bound)


def test_hi_below_min_normal_goes_to_lo():
    # Values in the f16 denormal range: with hi taken as zero the whole value is
    # carried by lo (normal after the 2^11 scale, f16 precision); an f16
    # denormal hi flushed by the matrix core would lose most of the value.
    rng = np.random.default_rng(2)
    a = (rng.uniform(1e-7, 6e-5, (16, 128)) * rng.choice([-1, 1], (16, 128))).astype(np.float32)
    b = rng.standard_normal((128, 16)).astype(np.float32)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    good = np.abs(split_dot(a, b, flush_hi=True) - exact) / scale
    bad = np.abs(split_dot(a, b, flush_hi=False) - exact) / scale
    assert good.max() < 2.0 ** -10
    assert bad.max() > 0.1


def test_range_is_the_f16_range():
    """The split is defined for |x| up to the largest f16 (65504), which the
    kernels' operands stay within (L2-normalised q/k, bounded GDN state, and the
    log2-scaled decode query for |q| below about 7e5 at head_dim 256); from
    65520 on, hi rounds to inf and the products are not finite.  This pins that
    documented edge rather than a fallback."""
    x = np.array([65504.0, -65504.0, 65519.0, 65520.0, -1e5], np.float32)
    with np.errstate(over="ignore"):
        hi, lo = split(x)
    assert np.all(np.isfinite(hi[:3])) and np.all(hi[:3] + lo[:3] / 2048.0 == x[:3])
    assert np.all(np.isinf(hi[3:]))
