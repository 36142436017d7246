"""The decode loop's three-launch linear-attention layer against the one-kernel
form it replaces, on the GPU, through the C ABI.

Three launches (include/kraken/qwen35_decode.hpp, linear_layer_decode_split):
- kraken_hip_kquant_matvec_multi_conv_f32: the joint input projection
  (RMSNorm folded in) whose qkv rows take the conv and SiLU and shift the conv
  state as they are written;
- kraken_hip_qwen35_gdn_state_ragged_decode_f32: the gated delta rule, each
  head spread over 16 workgroups, which also writes the norm-gated epilogue's
  norm_weight * silu(z);
- kraken_hip_kquant_matvec_head_norm_f32: ssm_out with the rest of the
  epilogue (the per-head RMS scale) on its input and the residual add on its
  output.
The one-kernel form: kraken_hip_kquant_matvec_multi_f32, then
kraken_hip_qwen35_gdn_layer_ragged_decode_f32, then
kraken_hip_kquant_matvec_fused_f32 with the residual.

The conv state and the recurrent state come out bit-identical: the conv runs
the same arithmetic per channel, and the split kernel repeats the one-kernel
layer's normalisation and per-row update.  The layer output differs only in
the order of the norm-gated epilogue's sum of squares (a different lane
layout) and in multiplying by the precomputed norm_weight * silu(z), so it is
held to 1e-5 relative to its magnitude.  Weights are
synthetic Qwen3.5-0.8B shapes (Q5_K qkv 6144 x 1024, Q4_K z 2048 x 1024,
Q4_K beta and alpha 16 x 1024, Q4_K ssm_out 1024 x 2048).
"""
import numpy as np
import pytest

import kquant_cases as kc

pytestmark = pytest.mark.gpu

H, D, HIDDEN, K = 16, 128, 1024, 4
CH = 3 * H * D
GGML = {"q4_k": 12, "q5_k": 13, "q6_k": 14}
EPS = 1e-6


def _model(rng):
    m = dict(
        qkv=("q5_k", CH, kc.random_weight_fast("q5_k", CH, HIDDEN, 11)),
        z=("q4_k", H * D, kc.random_weight_fast("q4_k", H * D, HIDDEN, 12)),
        beta=("q4_k", H, kc.random_weight_fast("q4_k", H, HIDDEN, 13)),
        alpha=("q4_k", H, kc.random_weight_fast("q4_k", H, HIDDEN, 14)),
        out=("q4_k", HIDDEN, kc.random_weight_fast("q4_k", HIDDEN, H * D, 15)),
        attn_norm=(1 + 0.1 * rng.standard_normal(HIDDEN)).astype(np.float32),
        conv_w=(0.5 * rng.standard_normal(CH * K)).astype(np.float32),
        dtb=rng.standard_normal(H).astype(np.float32),
        ssa=(-rng.random(H)).astype(np.float32),
        nw=(1 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    return m


def _dev(ctx, m):
    d = {k: ctx.buffer(v[2] if isinstance(v, tuple) else v) for k, v in m.items()}
    return d


def _states(ctx, rng, conv_at, state_at):
    conv = rng.standard_normal(conv_at + CH * (K - 1) + 64).astype(np.float32)
    state = (0.1 * rng.standard_normal(state_at + H * D * D + 256)).astype(np.float32)
    return (ctx.buffer(conv), ctx.buffer(np.array([conv_at], np.uint64)), ctx.buffer(state),
            ctx.buffer(np.array([state_at], np.uint64)))


def _one_kernel(ctx, m, dm, hidden, conv, coff, state, soff):
    outs = [ctx.buffer(byte_size=4 * m[k][1]) for k in ("qkv", "z", "beta", "alpha")]
    ctx.kquant_matvec_multi([GGML[m[k][0]] for k in ("qkv", "z", "beta", "alpha")],
                            [dm[k] for k in ("qkv", "z", "beta", "alpha")],
                            [m[k][1] for k in ("qkv", "z", "beta", "alpha")], HIDDEN, hidden,
                            dm["attn_norm"], EPS, None, [None] * 4, outs)
    y = ctx.buffer(byte_size=4 * H * D)
    ctx.qwen35_gdn_layer_ragged_decode_f32(outs[0], conv, coff, dm["conv_w"], K, outs[3], outs[2],
                                           dm["dtb"], dm["ssa"], outs[1], dm["nw"], state, soff, 1,
                                           H, H, D, EPS, y)
    ctx.kquant_matvec_fused_f32(GGML["q4_k"], dm["out"], HIDDEN, H * D, y, None, EPS, None,
                                hidden, hidden)


def _three_launch(ctx, m, dm, hidden, conv, coff, state, soff):
    outs = [ctx.buffer(byte_size=4 * m[k][1]) for k in ("qkv", "z", "beta", "alpha")]
    ctx.kquant_matvec_multi_conv([GGML[m[k][0]] for k in ("qkv", "z", "beta", "alpha")],
                                 [dm[k] for k in ("qkv", "z", "beta", "alpha")],
                                 [m[k][1] for k in ("qkv", "z", "beta", "alpha")], HIDDEN, hidden,
                                 dm["attn_norm"], EPS, outs, conv, coff, dm["conv_w"])
    y = ctx.buffer(byte_size=4 * H * D)
    gf = ctx.buffer(byte_size=4 * H * D)
    ctx.qwen35_gdn_state_ragged_decode_f32(outs[0], outs[3], outs[2], dm["dtb"], dm["ssa"],
                                           outs[1], dm["nw"], state, soff, 1, H, H, D, EPS, y, gf)
    ctx.kquant_matvec_head_norm_f32(GGML["q4_k"], dm["out"], HIDDEN, H * D, y, gf, D, EPS, hidden,
                                    hidden)


def test_three_launch_layer_equals_one_kernel_layer(hip_ctx):
    rng = np.random.default_rng(5)
    m = _model(rng)
    dm = _dev(hip_ctx, m)
    x = rng.standard_normal(HIDDEN).astype(np.float32)
    conv_at, state_at = 192, 128 * 128 * 3
    a = _states(hip_ctx, np.random.default_rng(6), conv_at, state_at)
    b = _states(hip_ctx, np.random.default_rng(6), conv_at, state_at)
    ha, hb = hip_ctx.buffer(x), hip_ctx.buffer(x)
    for step in range(3):
        print(f"gdn decode split step {step}", flush=True)
        _one_kernel(hip_ctx, m, dm, ha, *a)
        _three_launch(hip_ctx, m, dm, hb, *b)
        conv_a, conv_b = a[0].download(), b[0].download()
        state_a, state_b = a[2].download(), b[2].download()
        assert np.array_equal(conv_a.view(np.uint32), conv_b.view(np.uint32)), step
        assert np.array_equal(state_a.view(np.uint32), state_b.view(np.uint32)), step
        out_a, out_b = ha.download(), hb.download()
        scale = float(np.abs(out_a).max())
        np.testing.assert_allclose(out_b, out_a, rtol=0, atol=1e-5 * scale, err_msg=str(step))
        # Carry the same hidden state into the next step.
        hb.upload(out_a)


def test_head_norm_gemv_equals_epilogue_then_gemv(hip_ctx):
    """The head-norm input transform, given norm_weight * silu(z), against
    qwen35_norm_gated_f32_in_place followed by the plain fused GEMV with the
    residual (Q4_K and Q6_K ssm_out)."""
    rng = np.random.default_rng(8)
    for fmt in ("q4_k", "q6_k"):
        w = kc.random_weight_fast(fmt, HIDDEN, H * D, 21)
        y = rng.standard_normal(H * D).astype(np.float32) * 3.0
        z = rng.standard_normal(H * D).astype(np.float32)
        nw = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
        res = rng.standard_normal(HIDDEN).astype(np.float32)
        gate = (np.tile(nw, H).astype(np.float64) * z / (1 + np.exp(-z.astype(np.float64))))
        wb, zb, nb = hip_ctx.buffer(w), hip_ctx.buffer(z), hip_ctx.buffer(nw)
        yb = hip_ctx.buffer(y)
        want = hip_ctx.buffer(res)
        hip_ctx.qwen35_norm_gated_f32_in_place(yb, nb, zb, 1, H, D, EPS)
        hip_ctx.kquant_matvec_fused_f32(GGML[fmt], wb, HIDDEN, H * D, yb, None, EPS, None, want,
                                        want)
        got = hip_ctx.buffer(res)
        hip_ctx.kquant_matvec_head_norm_f32(GGML[fmt], wb, HIDDEN, H * D, hip_ctx.buffer(y),
                                            hip_ctx.buffer(gate.astype(np.float32)), D, EPS, got,
                                            got)
        a, b = want.download(), got.download()
        np.testing.assert_allclose(b, a, rtol=0, atol=1e-5 * float(np.abs(a).max()), err_msg=fmt)


def test_offsets_outside_the_pools_leave_memory_untouched(hip_ctx):
    """A conv offset past the pool: matrix 0's output and the conv pool stay as
    they were (the other matrices are written).  A state offset past the pool:
    the state kernel writes nothing."""
    rng = np.random.default_rng(9)
    m = _model(rng)
    dm = _dev(hip_ctx, m)
    hidden = hip_ctx.buffer(rng.standard_normal(HIDDEN).astype(np.float32))
    conv = rng.standard_normal(CH * (K - 1) + 64).astype(np.float32)
    cb = hip_ctx.buffer(conv)
    sentinel = np.full(CH, 7.0, np.float32)
    outs = [hip_ctx.buffer(sentinel)] + [hip_ctx.buffer(byte_size=4 * m[k][1])
                                         for k in ("z", "beta", "alpha")]
    hip_ctx.kquant_matvec_multi_conv([GGML[m[k][0]] for k in ("qkv", "z", "beta", "alpha")],
                                     [dm[k] for k in ("qkv", "z", "beta", "alpha")],
                                     [m[k][1] for k in ("qkv", "z", "beta", "alpha")], HIDDEN,
                                     hidden, dm["attn_norm"], EPS, outs, cb,
                                     hip_ctx.buffer(np.array([200], np.uint64)), dm["conv_w"])
    assert np.array_equal(outs[0].download(), sentinel)
    assert np.array_equal(cb.download(), conv)
    assert np.isfinite(outs[1].download()).all()
    state = (0.1 * rng.standard_normal(H * D * D)).astype(np.float32)
    sb = hip_ctx.buffer(state)
    yb = hip_ctx.buffer(np.full(H * D, 3.0, np.float32))
    gb = hip_ctx.buffer(np.full(H * D, 5.0, np.float32))
    hip_ctx.qwen35_gdn_state_ragged_decode_f32(
        hip_ctx.buffer(rng.standard_normal(CH).astype(np.float32)),
        hip_ctx.buffer(rng.standard_normal(H).astype(np.float32)),
        hip_ctx.buffer(rng.standard_normal(H).astype(np.float32)), dm["dtb"], dm["ssa"],
        hip_ctx.buffer(rng.standard_normal(H * D).astype(np.float32)), dm["nw"], sb,
        hip_ctx.buffer(np.array([4], np.uint64)), 1, H, H, D, EPS, yb, gb)
    assert np.array_equal(sb.download(), state)
    assert np.array_equal(yb.download(), np.full(H * D, 3.0, np.float32))
    assert np.array_equal(gb.download(), np.full(H * D, 5.0, np.float32))
