"""GPU parity of the decoder-layer ops around the hot path against the oracle:
rms_norm_f32_f32_batched (mps_backend.mm:1890-1920), add_f32_in_place
(:2529-2537) and silu_mul_f32_in_place (:2620-2629).  Tolerances: 1e-5
relative for the norm (float32 sums of up to 3584 squares against the
oracle's float64), exact for add, 1e-6 relative for silu_mul."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,size", [(1, 1024), (7, 1024), (3, 3584), (5, 100), (2, 1)])
@pytest.mark.parametrize("in_place", [False, True])
def test_rms_norm_batched(hip_ctx, rows, size, in_place):
    rng = np.random.default_rng(rows * size)
    x = (3 * rng.standard_normal(rows * size)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(size)).astype(np.float32)
    xb = hip_ctx.buffer(x)
    out = xb if in_place else hip_ctx.buffer(byte_size=4 * x.size)
    hip_ctx.rms_norm_f32_f32_batched(xb, hip_ctx.buffer(w), rows, size, 1e-6, out)
    want = oracle.rms_norm_batched(x, w, rows, size, 1e-6)
    np.testing.assert_allclose(out.download(x.size), want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("size", [1, 1000, 3584, 1 << 20])
def test_add_and_silu_mul(hip_ctx, size):
    rng = np.random.default_rng(size)
    a = (4 * rng.standard_normal(size)).astype(np.float32)
    b = rng.standard_normal(size).astype(np.float32)
    ab = hip_ctx.buffer(a)
    hip_ctx.add_f32_in_place(ab, hip_ctx.buffer(b), size)
    np.testing.assert_array_equal(ab.download(size), oracle.add(a, b))
    gb = hip_ctx.buffer(a)
    hip_ctx.silu_mul_f32_in_place(gb, hip_ctx.buffer(b), size)
    np.testing.assert_allclose(gb.download(size), oracle.silu_mul(a, b), rtol=1e-6, atol=1e-7)
