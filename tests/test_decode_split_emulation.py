"""Precision of the decode kernels' split fp16 products, emulated on the CPU
(kraken-infer_amd/csrc/attention_decode_short.hip and attention_decode.hip,
attention_decode_mfma_kernel).

The reference multiplies an f32 query with f32-converted f16 keys and weights
f32 probabilities into the f16 values (mps_backend.mm:2979-2997).  The matrix
cores take f16 operands, so the kernels hold the log2-scaled query x and every
probability p as hi = f16(x) (zero below the smallest normal f16, 2^-14) and
lo = f16((x - hi) 2^11), and sum hi products and lo products in separate fp32
accumulators, the lo ones scaled by 2^-11 at the end (device_common.hpp
split_f16).  The matrix core may flush f16 denormal operands, so the
emulation flushes every f16 denormal, the worst case.  An unscaled lo
(lo = f16(x - hi)) is an f16 denormal for |x| < 2^-3, which is nearly every
element of an N(0,1) query at this scale: with those flushed the decode runs on
an f16 query.  These checks show that the scaled split keeps the f32 result
where the unscaled one does not, at the C1 shape and on a sink key over a long
flat tail, whose weights fall below 2^-14.
"""
import numpy as np
import pytest

MIN_NORMAL = 2.0 ** -14
LOG2E = 1.4426950408889634


def ftz(h):
    return np.where(np.abs(h) < MIN_NORMAL, 0.0, h)


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


def split_scaled(x):
    """The kernels' split: hi zero below 2^-14, lo scaled by 2^11; flushed."""
    x = np.asarray(x, np.float32).astype(np.float64)
    hi = f16(np.where(np.abs(x) < MIN_NORMAL, 0.0, x))
    lo = f16((x - hi) * 2048.0)
    return ftz(hi), ftz(lo) / 2048.0


def split_unscaled(x):
    """hi = f16(x), lo = f16(x - hi) without a scale; flushed."""
    x = np.asarray(x, np.float32).astype(np.float64)
    hi = f16(x)
    lo = f16(x - hi)
    return ftz(hi), ftz(lo)


def emulate(q, k, v, split):
    """One query head against keys k [L][D] and values v [L][D] (f16 values):
    log2-domain scores from the split query, probabilities against the max,
    numerator from the split probabilities, denominator from the f32 ones."""
    d = q.size
    x = (q.astype(np.float32) * np.float32(1.0 / np.sqrt(np.float32(d)) * LOG2E))
    xh, xl = split(x)
    s = k @ xh + k @ xl
    p = np.exp2((s - s.max()).astype(np.float32)).astype(np.float32)
    ph, pl = split(p)
    return (ph @ v + pl @ v) / p.astype(np.float64).sum()


def exact(q, k, v):
    d = q.size
    s = k @ q.astype(np.float64) / np.sqrt(np.float32(d))
    w = np.exp(s - s.max())
    return w @ v / w.sum()


@pytest.mark.parametrize("scale,good_bound,bad_floor", [(1.0, 2e-7, 5e-6), (8.0, 2e-6, 5e-5)])
def test_c1_query_split_keeps_f32_precision(scale, good_bound, bad_floor):
    """C1: L = 4096 keys, N(0,1) q, K, V (K, V in f16), at unit and 8x query
    scale.  The scaled split stays near f32 rounding; the unscaled split with
    flushed denormals is off by the f16 rounding of the query."""
    rng = np.random.default_rng(1)
    L, D = 4097, 256
    k = f16(rng.standard_normal((L, D)))
    v = f16(rng.standard_normal((L, D)))
    good = bad = 0.0
    for _ in range(4):
        q = (scale * rng.standard_normal(D)).astype(np.float32)
        ref = exact(q, k, v)
        good = max(good, np.abs(emulate(q, k, v, split_scaled) - ref).max())
        bad = max(bad, np.abs(emulate(q, k, v, split_unscaled) - ref).max())
    assert good < good_bound
    assert bad > bad_floor


def test_sink_over_flat_tail_keeps_the_tail():
    """One key 10 nats above 16383 equal keys: the tail's weights, e^-10 =
    4.5e-5, are below the smallest normal f16 and together carry 43% of the
    softmax mass.  The scaled split keeps them; an unscaled split whose
    denormals are flushed drops the whole tail.  The tail's weights are carried
    by lo alone, at f16 precision (all 16383 round the same way), which bounds
    the scaled split at a few 1e-6."""
    rng = np.random.default_rng(2)
    L, D = 16384, 256
    q = rng.standard_normal(D).astype(np.float32)
    k = np.zeros((L, D))
    # Sink key along q: its score is 10 nats (f16 rounding of k moves it slightly).
    k[0] = f16(q * (10.0 * np.sqrt(D) / float(q.astype(np.float64) @ q)))
    v = f16(rng.standard_normal((L, D)))
    ref = exact(q, k, v)
    good = np.abs(emulate(q, k, v, split_scaled) - ref).max()
    bad = np.abs(emulate(q, k, v, split_unscaled) - ref).max()
    assert good < 5e-6
    assert bad > 1e-2


def test_split_scaled_representation_bound():
    """x = hi + 2^-11 lo within 2^-21 relative plus 2^-25 absolute over the
    probability range [0, 2^8] and the query range, with denormals flushed."""
    rng = np.random.default_rng(3)
    x = np.concatenate([2.0 ** rng.uniform(-30, 8, 200000),
                        -(2.0 ** rng.uniform(-30, 8, 1000))]).astype(np.float32)
    hi, lo = split_scaled(x)
    err = np.abs(x.astype(np.float64) - (hi + lo))
    assert np.all(err <= 2.0 ** -21 * np.abs(x) + 2.0 ** -25)
