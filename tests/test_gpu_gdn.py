"""GPU parity of the gated-delta-net path against the CPU oracle.

Tolerance: 1e-4 absolute on the fp32 recurrent state and
outputs.  C3 inputs: H=16, dk=dv=128, conv K=4 over C=6144 channels;
x ~ N(0,1), conv weights ~ 0.5 N(0,1), beta = sigmoid(N(0,1)),
g = -softplus(N(0,1)), q/k L2-normalised (by the fused conv/split/L2 prologue).
"""
import numpy as np
import pytest

import kraken_hip as kh
import oracle

ATOL = 1e-4


def gdn_inputs(seed, tokens, hk=16, hv=16, d=128, state_scale=0.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((tokens, hk, d)).astype(np.float32)
    k = rng.standard_normal((tokens, hk, d)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((tokens, hv, d)).astype(np.float32)
    g = (-np.logaddexp(0, rng.standard_normal((tokens, hv)))).astype(np.float32)
    b = (1 / (1 + np.exp(-rng.standard_normal((tokens, hv))))).astype(np.float32)
    s = (rng.standard_normal(hv * d * d) * state_scale).astype(np.float32)
    return q.ravel(), k.ravel(), v.ravel(), g.ravel(), b.ravel(), s


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [
    # tokens, key_heads, value_heads, head_dim
    (1, 16, 16, 128), (7, 16, 16, 128), (64, 2, 4, 128), (33, 1, 3, 64), (5, 2, 2, 40),
    (9, 1, 1, 256), (3, 4, 8, 96), (2, 16, 16, 128), (65, 16, 16, 128), (130, 2, 6, 128),
    (200, 16, 16, 128),
])
def test_gdn_shapes(hip_ctx, shape):
    tokens, hk, hv, d = shape
    print(f"gdn {shape}", flush=True)
    q, k, v, g, b, s = gdn_inputs(1, tokens, hk, hv, d, state_scale=0.1)
    out, st = kh.NumpyOps(hip_ctx).gated_delta_net(q, k, v, g, b, s, tokens, hk, hv, d)
    out_ref, st_ref = oracle.gated_delta_net(q, k, v, g, b, s, tokens, hk, hv, d)
    np.testing.assert_allclose(out, out_ref, rtol=0, atol=ATOL)
    np.testing.assert_allclose(st, st_ref, rtol=0, atol=ATOL)


@pytest.mark.gpu
def test_gdn_state_offset_and_neighbours_untouched(hip_ctx):
    tokens, h, d = 4, 2, 64
    q, k, v, g, b, s = gdn_inputs(2, tokens, h, h, d, state_scale=0.2)
    layers = 3
    big = np.random.default_rng(3).standard_normal(layers * h * d * d).astype(np.float32)
    off = h * d * d  # layer 1
    out, st = kh.NumpyOps(hip_ctx).gated_delta_net(q, k, v, g, b, big, tokens, h, h, d,
                                                   state_offset=off)
    out_ref, st1 = oracle.gated_delta_net(q, k, v, g, b, big[off:2 * off], tokens, h, h, d)
    np.testing.assert_allclose(out, out_ref, rtol=0, atol=ATOL)
    np.testing.assert_allclose(st[off:2 * off], st1, rtol=0, atol=ATOL)
    np.testing.assert_array_equal(st[:off], big[:off])
    np.testing.assert_array_equal(st[2 * off:], big[2 * off:])


@pytest.mark.gpu
@pytest.mark.parametrize("offset_extra", [0, 1])
def test_gdn_prefill_state_offset_d128(hip_ctx, offset_extra):
    """head_dim 128 multi-token calls at a state offset: a 16-byte aligned offset
    takes the LDS-staged prefill kernel, an odd one the generic kernel; both must
    update exactly their own state block."""
    tokens, h, d = 97, 4, 128
    q, k, v, g, b, _ = gdn_inputs(12, tokens, h, h, d)
    blk = h * d * d
    big = (0.1 * np.random.default_rng(13).standard_normal(3 * blk + 4)).astype(np.float32)
    off = blk + offset_extra
    out, st = kh.NumpyOps(hip_ctx).gated_delta_net(q, k, v, g, b, big, tokens, h, h, d,
                                                   state_offset=off)
    out_ref, st1 = oracle.gated_delta_net(q, k, v, g, b, big[off:off + blk], tokens, h, h, d)
    np.testing.assert_allclose(out, out_ref, rtol=0, atol=ATOL)
    np.testing.assert_allclose(st[off:off + blk], st1, rtol=0, atol=ATOL)
    np.testing.assert_array_equal(st[:off], big[:off])
    np.testing.assert_array_equal(st[off + blk:], big[off + blk:])


@pytest.mark.gpu
@pytest.mark.parametrize("tokens", [64, 257, 1024])
def test_gdn_prefill_kernels_agree(hip_ctx, monkeypatch, tokens):
    """The three multi-token kernels for head_dim 128 -- chunked WY (default),
    LDS-staged sequential (KRAKEN_GDN_PREFILL=sequential) and the generic
    recurrence (KRAKEN_GDN_PREFILL=generic) -- give the same outputs and state,
    and each matches the oracle."""
    hk = hv = 16
    d = 128
    q, k, v, g, b, s = gdn_inputs(14, tokens, hk, hv, d, state_scale=0.1)
    ops = kh.NumpyOps(hip_ctx)
    out_ref, st_ref = oracle.gated_delta_net(q, k, v, g, b, s, tokens, hk, hv, d)
    results = {}
    for mode in (None, "sequential", "generic"):
        if mode is None:
            monkeypatch.delenv("KRAKEN_GDN_PREFILL", raising=False)
        else:
            monkeypatch.setenv("KRAKEN_GDN_PREFILL", mode)
        results[mode] = ops.gated_delta_net(q, k, v, g, b, s, tokens, hk, hv, d)
        np.testing.assert_allclose(results[mode][0], out_ref, rtol=0, atol=ATOL, err_msg=str(mode))
        np.testing.assert_allclose(results[mode][1], st_ref, rtol=0, atol=ATOL, err_msg=str(mode))
    monkeypatch.delenv("KRAKEN_GDN_PREFILL", raising=False)
    for mode in ("sequential", "generic"):
        np.testing.assert_allclose(results[None][0], results[mode][0], rtol=0, atol=2e-5)
        np.testing.assert_allclose(results[None][1], results[mode][1], rtol=0, atol=2e-5)


@pytest.mark.gpu
def test_gdn_chunked_crosses_pass_boundary(hip_ctx, monkeypatch):
    """The chunked path works through the tokens in passes of 64 chunks (4096
    tokens) with the state carried between passes; 4166 tokens make a second,
    ragged pass.  Grouped heads (key_heads < value_heads)."""
    tokens, hk, hv, d = 64 * 64 + 70, 2, 4, 128
    q, k, v, g, b, s = gdn_inputs(16, tokens, hk, hv, d, state_scale=0.1)
    ops = kh.NumpyOps(hip_ctx)
    monkeypatch.delenv("KRAKEN_GDN_PREFILL", raising=False)
    out, st = ops.gated_delta_net(q, k, v, g, b, s, tokens, hk, hv, d)
    out_ref, st_ref = oracle.gated_delta_net(q, k, v, g, b, s, tokens, hk, hv, d)
    np.testing.assert_allclose(out, out_ref, rtol=0, atol=ATOL)
    np.testing.assert_allclose(st, st_ref, rtol=0, atol=ATOL)
    monkeypatch.setenv("KRAKEN_GDN_PREFILL", "sequential")
    out_s, st_s = ops.gated_delta_net(q, k, v, g, b, s, tokens, hk, hv, d)
    np.testing.assert_allclose(out, out_s, rtol=0, atol=2e-5)
    np.testing.assert_allclose(st, st_s, rtol=0, atol=2e-5)


@pytest.mark.gpu
def test_gdn_chunked_decay_and_beta_extremes(hip_ctx):
    """Chunked path with strong decay (g down to -8, exp(g) ~ 3e-4), beta near
    0 and 1, and a large initial state: the per-chunk factors exp(G_t - G_j)
    span many orders of magnitude."""
    tokens, hk, hv, d = 192, 4, 8, 128
    rng = np.random.default_rng(15)
    q, k, v, _, _, s = gdn_inputs(15, tokens, hk, hv, d, state_scale=1.0)
    g = (-8.0 * rng.random(tokens * hv)).astype(np.float32)
    b = np.where(rng.random(tokens * hv) < 0.5, 0.999, 0.001).astype(np.float32)
    out, st = kh.NumpyOps(hip_ctx).gated_delta_net(q, k, v, g, b, s, tokens, hk, hv, d)
    out_ref, st_ref = oracle.gated_delta_net(q, k, v, g, b, s, tokens, hk, hv, d)
    np.testing.assert_allclose(out, out_ref, rtol=0, atol=ATOL)
    np.testing.assert_allclose(st, st_ref, rtol=0, atol=ATOL)


@pytest.mark.gpu
def test_gdn_c3_prefill_4096_in_chunks_then_decode(hip_ctx):
    """C3: 4096-token prefill in 1024-token chunks, then its 256 decode steps, state
    carried on the device; oracle runs the same sequence.  Checks the output and the
    state after every chunk and every decode step."""
    hk = hv = 16
    d = 128
    total, chunk, decode = 4096, 1024, 256
    q, k, v, g, b, _ = gdn_inputs(3, total + decode, hk, hv, d)
    ctx = hip_ctx
    s_dev = ctx.buffer(np.zeros(hv * d * d, np.float32))
    s_ref = np.zeros(hv * d * d, np.float32)
    kd, vd, gd = hk * d, hv * d, hv
    steps = [(i, chunk) for i in range(0, total, chunk)] + [(total + i, 1) for i in range(decode)]
    for t0, n in steps:
        sl = lambda a, w: a[t0 * w:(t0 + n) * w]
        bufs = [ctx.buffer(sl(q, kd)), ctx.buffer(sl(k, kd)), ctx.buffer(sl(v, vd)),
                ctx.buffer(sl(g, gd)), ctx.buffer(sl(b, gd))]
        out = ctx.buffer(byte_size=4 * n * vd)
        ctx.gated_delta_net_f32_batched_in_place_at(*bufs, s_dev, 0, n, hk, hv, d, out)
        out_ref, s_ref = oracle.gated_delta_net(sl(q, kd), sl(k, kd), sl(v, vd), sl(g, gd),
                                                sl(b, gd), s_ref, n, hk, hv, d)
        np.testing.assert_allclose(out.download(), out_ref, rtol=0, atol=ATOL,
                                   err_msg=f"out t0={t0}")
        np.testing.assert_allclose(s_dev.download(), s_ref, rtol=0, atol=ATOL,
                                   err_msg=f"state t0={t0}")


@pytest.mark.gpu
def test_gdn_beta_zero_is_pure_decay(hip_ctx):
    tokens, h, d = 6, 2, 128
    q, k, v, g, b, s = gdn_inputs(4, tokens, h, h, d, state_scale=1.0)
    out, st = kh.NumpyOps(hip_ctx).gated_delta_net(q, k, v, g, np.zeros_like(b), s, tokens, h,
                                                   h, d)
    decay = np.exp(g.reshape(tokens, h).astype(np.float64).sum(0))
    expect = s.reshape(h, d * d) * decay[:, None]
    np.testing.assert_allclose(st.reshape(h, d * d), expect, rtol=1e-5, atol=1e-6)


# ----------------------------------------------------------- conv prologue --

def conv_inputs(seed, tokens, hk=16, hv=16, d=128, kk=4):
    rng = np.random.default_rng(seed)
    channels = (2 * hk + hv) * d
    x = rng.standard_normal(tokens * channels).astype(np.float32)
    w = (rng.standard_normal(channels * kk) * 0.5).astype(np.float32)
    state = rng.standard_normal(channels * (kk - 1)).astype(np.float32)
    return x, w, state, channels


def conv_reference(x, w, state, tokens, hk, hv, d, kk, eps=1e-6):
    channels = (2 * hk + hv) * d
    ci, st = oracle.build_ssm_conv_state(state, x, kk, channels, tokens)
    y = oracle.ssm_conv(ci, w, kk, channels, tokens, 1)
    y = oracle.silu(y)
    q, k, v = oracle.split_qkv_l2_norm(y, tokens, hk, hv, d, eps)
    return q, k, v, st


@pytest.mark.gpu
@pytest.mark.parametrize("tokens,hk,hv,d,kk", [
    (1, 16, 16, 128, 4), (2, 16, 16, 128, 4), (37, 16, 16, 128, 4), (1024, 16, 16, 128, 4),
    (5, 2, 4, 64, 3), (17, 1, 2, 256, 2), (3, 2, 2, 100, 8),
])
def test_fused_conv_split_l2_matches_reference_chain(hip_ctx, tokens, hk, hv, d, kk):
    """The fused prologue equals build_ssm_conv_state -> ssm_conv -> silu ->
    split_qkv_l2_norm (qwen35_runtime.cpp:2746-2796), including the new conv state."""
    print(f"conv split T={tokens} hk={hk} hv={hv} d={d} K={kk}", flush=True)
    x, w, state, channels = conv_inputs(5, tokens, hk, hv, d, kk)
    ctx = hip_ctx
    xb, wb, sb = ctx.buffer(x), ctx.buffer(w), ctx.buffer(state)
    qb = ctx.buffer(byte_size=4 * tokens * hk * d)
    kb = ctx.buffer(byte_size=4 * tokens * hk * d)
    vb = ctx.buffer(byte_size=4 * tokens * hv * d)
    ctx.qwen35_conv_split_l2_f32(xb, sb, 0, wb, kk, tokens, hk, hv, d, 1e-6, qb, kb, vb)
    q, k, v, st = conv_reference(x, w, state, tokens, hk, hv, d, kk)
    np.testing.assert_allclose(qb.download(), q, rtol=0, atol=1e-5)
    np.testing.assert_allclose(kb.download(), k, rtol=0, atol=1e-5)
    np.testing.assert_allclose(vb.download(), v, rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(sb.download(), st)


@pytest.mark.gpu
def test_unfused_conv_ops_match_oracle(hip_ctx):
    tokens, hk, hv, d, kk = 9, 2, 2, 32, 4
    x, w, state, channels = conv_inputs(6, tokens, hk, hv, d, kk)
    ops = kh.NumpyOps(hip_ctx)
    ci, st = ops.build_ssm_conv_state(state, x, kk, channels, tokens)
    ci_ref, st_ref = oracle.build_ssm_conv_state(state, x, kk, channels, tokens)
    np.testing.assert_array_equal(ci, ci_ref)
    np.testing.assert_array_equal(st, st_ref)
    y = ops.ssm_conv(ci, w, kk, channels, tokens, 1)
    np.testing.assert_allclose(y, oracle.ssm_conv(ci_ref, w, kk, channels, tokens, 1),
                               rtol=1e-5, atol=1e-5)
    out, st1 = ops.ssm_conv1_stateful(state, x[:channels], w, kk, channels)
    out_ref, st1_ref = oracle.ssm_conv1_stateful(state, x[:channels], w, kk, channels)
    np.testing.assert_allclose(out, out_ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(st1, st1_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("tokens", [1, 64, 300])
def test_gdn_gated_fused_matches_reference_chain(hip_ctx, tokens):
    """prepare_gate_beta + GDN + norm-gated epilogue fused vs the reference op chain
    (qwen35_runtime.cpp:2913-3008) on the oracle."""
    hk = hv = 16
    d = 128
    rng = np.random.default_rng(7)
    q, k, v, _, _, s = gdn_inputs(8, tokens, hk, hv, d, state_scale=0.05)
    alpha = rng.standard_normal(tokens * hv).astype(np.float32)
    beta_raw = rng.standard_normal(tokens * hv).astype(np.float32)
    dt_bias = rng.standard_normal(hv).astype(np.float32)
    ssm_a = (-np.abs(rng.standard_normal(hv))).astype(np.float32)
    z = rng.standard_normal(tokens * hv * d).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    ctx = hip_ctx
    bufs = [ctx.buffer(a) for a in (q, k, v, alpha, beta_raw, dt_bias, ssm_a, z, w)]
    sb = ctx.buffer(s)
    out = ctx.buffer(byte_size=4 * tokens * hv * d)
    ctx.qwen35_gdn_gated_f32(*bufs, sb, 0, tokens, hk, hv, d, 1e-6, out)
    g_ref, b_ref = oracle.prepare_gdn_gate_beta(alpha, beta_raw, dt_bias, ssm_a, tokens, hv)
    y_ref, s_ref = oracle.gated_delta_net(q, k, v, g_ref, b_ref, s, tokens, hk, hv, d)
    y_ref = oracle.norm_gated(y_ref, w, z, tokens, hv, d, 1e-6)
    np.testing.assert_allclose(out.download(), y_ref, rtol=0, atol=ATOL)
    np.testing.assert_allclose(sb.download(), s_ref, rtol=0, atol=ATOL)
