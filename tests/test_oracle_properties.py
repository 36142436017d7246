"""Pins the CPU oracle beyond the smoke-test fixtures.

Each check is chosen so a plausible restatement mistake (dropped term, wrong
sign, transposed operand, wrong GQA map, off-by-one causal bound) fails it:
exhaustive/IEEE comparisons for fp16 conversion, closed forms, invariants, and
brute force against independent numpy formulations written differently from
the oracle's loops (matrix forms, complex rotation, explicit softmax).
"""
import numpy as np
import pytest

import oracle


# ------------------------------------------------------------------ f16 ----

def test_f16_to_f32_exhaustive_against_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_against_numpy():
    rng = np.random.default_rng(0)
    raw = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    x = raw.view(np.float32)
    # Edge values: ties to even, subnormal boundary, overflow boundary, signed zero.
    edges = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e-8, 2**-24,
                      2**-25, 3 * 2**-26, 2**-14, 2**-14 - 2**-25, 1 + 2**-11, 1 + 3 * 2**-11,
                      np.inf, -np.inf], np.float32)
    x = np.concatenate([x, edges, rng.standard_normal(100_000).astype(np.float32)])
    got = oracle.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


# ------------------------------------------------------------ attention ----

def numpy_attention(q, kc, vc, start, tokens, cap, heads, kv_heads, d, layer=0):
    """Explicit softmax attention, written from the math (not the oracle's loops)."""
    q = q.reshape(tokens, heads, d).astype(np.float64)
    k = kc.reshape(-1, cap, kv_heads, d)[layer].astype(np.float64)
    v = vc.reshape(-1, cap, kv_heads, d)[layer].astype(np.float64)
    group = heads // kv_heads
    out = np.zeros((tokens, heads, d))
    for t in range(tokens):
        n = start + t + 1
        for h in range(heads):
            g = h // group
            s = k[:n, g, :] @ q[t, h] / np.sqrt(np.float32(d))
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ v[:n, g, :]
    return out.reshape(-1)


@pytest.mark.parametrize("kv_f16", [False, True])
@pytest.mark.parametrize("shape", [(3, 5, 12, 4, 2, 16), (0, 7, 7, 2, 1, 8), (9, 1, 10, 8, 2, 32)])
def test_attention_brute_force(kv_f16, shape):
    start, tokens, cap, heads, kv_heads, d = shape
    rng = np.random.default_rng(1)
    layers = 2
    q = rng.standard_normal(tokens * heads * d).astype(np.float32)
    kc = rng.standard_normal(layers * cap * kv_heads * d).astype(np.float32)
    vc = rng.standard_normal(layers * cap * kv_heads * d).astype(np.float32)
    if kv_f16:
        kb, vb = oracle.f32_to_f16_bits(kc), oracle.f32_to_f16_bits(vc)
        kref, vref = oracle.f16_bits_to_f32(kb), oracle.f16_bits_to_f32(vb)
    else:
        kb, vb, kref, vref = kc, vc, kc, vc
    got = oracle.attention_batched(q, kb, vb, 1, start, tokens, cap, heads, kv_heads, d)
    ref = numpy_attention(q, kref, vref, start, tokens, cap, heads, kv_heads, d, layer=1)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)


def test_attention_round_query_matches_prerounded_query():
    rng = np.random.default_rng(2)
    heads, kv_heads, d, tokens, cap = 4, 2, 16, 3, 3
    q = rng.standard_normal(tokens * heads * d).astype(np.float32)
    kc = oracle.f32_to_f16_bits(rng.standard_normal(cap * kv_heads * d))
    vc = oracle.f32_to_f16_bits(rng.standard_normal(cap * kv_heads * d))
    a = oracle.attention_batched(q, kc, vc, 0, 0, tokens, cap, heads, kv_heads, d,
                                 round_query_f16=True)
    b = oracle.attention_batched(q.astype(np.float16).astype(np.float32), kc, vc, 0, 0, tokens,
                                 cap, heads, kv_heads, d)
    np.testing.assert_array_equal(a, b)
    c = oracle.attention_batched(q, kc, vc, 0, 0, tokens, cap, heads, kv_heads, d)
    assert not np.array_equal(a, c)


def test_attention_gqa_heads_with_equal_query_agree_and_groups_differ():
    rng = np.random.default_rng(3)
    heads, kv_heads, d, cap = 8, 2, 32, 6
    qh = rng.standard_normal(d).astype(np.float32)
    q = np.tile(qh, heads)
    kc = rng.standard_normal(cap * kv_heads * d).astype(np.float32)
    vc = rng.standard_normal(cap * kv_heads * d).astype(np.float32)
    out = oracle.attention_batched(q, kc, vc, 0, cap - 1, 1, cap, heads, kv_heads, d)
    out = out.reshape(heads, d)
    for h in range(heads):
        np.testing.assert_array_equal(out[h], out[(h // 4) * 4])
    assert not np.allclose(out[0], out[4])


def test_attention_key_permutation_invariance_for_last_query():
    rng = np.random.default_rng(4)
    d, cap = 16, 9
    q = rng.standard_normal(d).astype(np.float32)
    kc = rng.standard_normal((cap, d)).astype(np.float32)
    vc = rng.standard_normal((cap, d)).astype(np.float32)
    perm = rng.permutation(cap)
    a = oracle.attention_batched(q, kc, vc, 0, cap - 1, 1, cap, 1, 1, d)
    b = oracle.attention_batched(q, kc[perm], vc[perm], 0, cap - 1, 1, cap, 1, 1, d)
    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------------ GDN ----

def numpy_gdn_matrix_form(q, k, v, g, b, s0, tokens, hk, hv, d):
    """S_t = e^g S (I - b k k^T) + b v k^T ; y = S_t q / sqrt(d), in matrix form."""
    q = q.reshape(tokens, hk, d).astype(np.float64)
    k = k.reshape(tokens, hk, d).astype(np.float64)
    v = v.reshape(tokens, hv, d).astype(np.float64)
    g = g.reshape(tokens, hv).astype(np.float64)
    b = b.reshape(tokens, hv).astype(np.float64)
    s = s0.reshape(hv, d, d).astype(np.float64).copy()
    y = np.zeros((tokens, hv, d))
    eye = np.eye(d)
    for t in range(tokens):
        for h in range(hv):
            kk = k[t, h % hk]
            s[h] = np.exp(g[t, h]) * s[h] @ (eye - b[t, h] * np.outer(kk, kk)) + \
                b[t, h] * np.outer(v[t, h], kk)
            y[t, h] = s[h] @ q[t, h % hk] / np.sqrt(d)
    return y.reshape(-1), s.reshape(-1)


def test_gdn_matches_matrix_form_with_gqa_repeat():
    rng = np.random.default_rng(5)
    tokens, hk, hv, d = 6, 2, 4, 8
    q = rng.standard_normal(tokens * hk * d).astype(np.float32)
    k = rng.standard_normal(tokens * hk * d).astype(np.float32) * 0.3
    v = rng.standard_normal(tokens * hv * d).astype(np.float32)
    g = -np.abs(rng.standard_normal(tokens * hv)).astype(np.float32)
    b = (1 / (1 + np.exp(-rng.standard_normal(tokens * hv)))).astype(np.float32)
    s0 = rng.standard_normal(hv * d * d).astype(np.float32)
    y, s = oracle.gated_delta_net(q, k, v, g, b, s0, tokens, hk, hv, d)
    y_ref, s_ref = numpy_gdn_matrix_form(q, k, v, g, b, s0, tokens, hk, hv, d)
    np.testing.assert_allclose(y, y_ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(s, s_ref, rtol=1e-5, atol=1e-5)


def test_gdn_beta_zero_is_pure_decay():
    rng = np.random.default_rng(6)
    tokens, d = 4, 8
    q = rng.standard_normal(tokens * d).astype(np.float32)
    k = rng.standard_normal(tokens * d).astype(np.float32)
    v = rng.standard_normal(tokens * d).astype(np.float32)
    g = np.array([-0.1, -0.2, -0.3, -0.4], np.float32)
    s0 = rng.standard_normal(d * d).astype(np.float32)
    y, s = oracle.gated_delta_net(q, k, v, g, np.zeros(tokens, np.float32), s0, tokens, 1, 1, d)
    np.testing.assert_allclose(s, s0 * np.exp(g.astype(np.float64).sum()), rtol=1e-5)
    last = s0.reshape(d, d).astype(np.float64) * np.exp(g.astype(np.float64).sum())
    np.testing.assert_allclose(y[-d:], last @ q[-d:] / np.sqrt(d), rtol=1e-5, atol=1e-6)


def test_gdn_unit_key_from_zero_state():
    d, i = 8, 3
    q = np.arange(1, d + 1, dtype=np.float32)
    k = np.zeros(d, np.float32)
    k[i] = 1.0
    v = np.linspace(-1, 1, d).astype(np.float32)
    y, s = oracle.gated_delta_net(q, k, v, [0.0], [1.0], np.zeros(d * d, np.float32), 1, 1, 1, d)
    np.testing.assert_allclose(y, v * q[i] / np.sqrt(d), rtol=1e-6)
    expect = np.zeros((d, d))
    expect[:, i] = v
    np.testing.assert_allclose(s.reshape(d, d), expect, atol=0)


# ------------------------------------------------------------ conv/rope ----

def test_conv_chunked_equals_whole_sequence():
    rng = np.random.default_rng(7)
    kk, c, t = 4, 5, 9
    x = rng.standard_normal(t * c).astype(np.float32)
    w = rng.standard_normal(c * kk).astype(np.float32)
    state = np.zeros(c * (kk - 1), np.float32)
    ci, _ = oracle.build_ssm_conv_state(state, x, kk, c, t)
    whole = oracle.ssm_conv(ci, w, kk, c, t, 1)
    # numpy: causal depthwise conv, y[t,c] = sum_j w[c,j] x[t-(K-1)+j, c]
    xp = np.concatenate([np.zeros((kk - 1, c)), x.reshape(t, c)])
    ref = np.stack([(xp[tt:tt + kk] * w.reshape(c, kk).T).sum(0) for tt in range(t)])
    np.testing.assert_allclose(whole.reshape(t, c), ref, rtol=1e-5, atol=1e-6)
    # Same sequence fed as chunks 4 + 5 through the carried state; and token by token.
    st = np.zeros_like(state)
    parts = []
    for lo, hi in ((0, 4), (4, 9)):
        ci, st = oracle.build_ssm_conv_state(st, x[lo * c:hi * c], kk, c, hi - lo)
        parts.append(oracle.ssm_conv(ci, w, kk, c, hi - lo, 1))
    np.testing.assert_allclose(np.concatenate(parts), whole, rtol=1e-6, atol=1e-7)
    st = np.zeros_like(state)
    steps = []
    for tt in range(t):
        out, st = oracle.ssm_conv1_stateful(st, x[tt * c:(tt + 1) * c], w, kk, c)
        steps.append(out)
    np.testing.assert_allclose(np.concatenate(steps), whole, rtol=1e-6, atol=1e-7)


def test_mrope_matches_complex_rotation_and_leaves_tail():
    rng = np.random.default_rng(8)
    tokens, heads, d, n_dims, sections, theta = 3, 2, 32, 16, (3, 3, 2, 0), 1e7
    x = rng.standard_normal(tokens * heads * d).astype(np.float32)
    pos = rng.integers(0, 5000, size=4 * tokens).astype(np.int32)
    got = oracle.mrope(x, pos, tokens, heads, d, n_dims, sections, theta).reshape(tokens, heads, d)
    xr = x.reshape(tokens, heads, d).astype(np.float64)
    half = n_dims // 2
    bounds = np.cumsum(sections)
    for t in range(tokens):
        for i in range(half):
            row = int(np.searchsorted(bounds, i % sum(sections), side="right"))
            ang = pos[t + tokens * row] * theta ** (-2 * i / n_dims)
            z = (xr[t, :, i] + 1j * xr[t, :, half + i]) * np.exp(1j * ang)
            np.testing.assert_allclose(got[t, :, i], z.real, rtol=1e-5, atol=1e-5)
            np.testing.assert_allclose(got[t, :, half + i], z.imag, rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(got[:, :, n_dims:], x.reshape(tokens, heads, d)[:, :, n_dims:])


def test_mrope_positions_rows_are_token_index():
    pos = oracle.make_mrope_positions(7, 3).reshape(4, 3)
    assert (pos == np.array([7, 8, 9])).all()


# ------------------------------------------------------------- norms -------

def test_qk_norm_unit_rms_and_l2_unit_norm():
    rng = np.random.default_rng(9)
    x = rng.standard_normal(3 * 4 * 16).astype(np.float32) * 5
    y = oracle.qk_norm_f32_batched(x, np.ones(16), 3, 4, 16, 0.0).reshape(-1, 16)
    np.testing.assert_allclose(np.sqrt((y.astype(np.float64) ** 2).mean(1)), 1.0, rtol=1e-6)
    z = oracle.l2_norm(x, 12, 16, 1e-6).reshape(-1, 16)
    np.testing.assert_allclose(np.linalg.norm(z.astype(np.float64), axis=1), 1.0, rtol=1e-6)
    tiny = oracle.l2_norm(np.full(4, 1e-9, np.float32), 1, 4, 1e-6)
    np.testing.assert_allclose(tiny, 1e-9 / 1e-6, rtol=1e-6)


# ------------------------------------------------------- legacy Qwen3 ------

def test_legacy_qwen3_attention_agrees_with_generic_attention():
    rng = np.random.default_rng(10)
    heads, kv_heads, d, positions = 4, 2, 16, 7
    q = rng.standard_normal(positions * heads * d).astype(np.float32)
    k = rng.standard_normal(positions * kv_heads * d).astype(np.float32)
    v = rng.standard_normal(positions * kv_heads * d).astype(np.float32)
    ones = np.ones(d, np.float32)
    kc, vc, qo, out = oracle.qwen3_attention_sequence(q, k, v, positions, heads, kv_heads, d,
                                                      ones, ones, 1e-6, 1e6)
    ref = oracle.attention_batched(qo, kc, vc, 0, 0, positions, positions, heads, kv_heads, d)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)
    # Position 0 rope is the identity; qk_norm with unit weights gives unit RMS.
    q0 = oracle.qwen3_qk_norm(q[:heads * d], heads, d, ones, 1e-6)
    np.testing.assert_array_equal(oracle.qwen3_rope(q0, heads, d, 0, 1e6), q0)
    np.testing.assert_allclose(qo[:heads * d], q0, rtol=0, atol=0)


def test_qwen3_rope_is_complex_rotation_at_nonzero_positions():
    """Pair (i, i + d/2) of each head turns by position * theta^(-2i/d): the
    closed form as a complex rotation, at positions far from 0, and the
    rotations compose (rope(rope(x, a), b) = rope(x, a + b))."""
    rng = np.random.default_rng(11)
    heads, d, theta = 3, 128, 1e6
    half = d // 2
    x = rng.standard_normal(heads * d).astype(np.float32)
    xr = x.reshape(heads, d).astype(np.float64)
    for p in (1, 7, 511, 4096, 100003):
        got = oracle.qwen3_rope(x, heads, d, p, theta).reshape(heads, d)
        ang = p * theta ** (-2.0 * np.arange(half) / d)
        z = (xr[:, :half] + 1j * xr[:, half:]) * np.exp(1j * ang)
        np.testing.assert_allclose(got[:, :half], z.real, rtol=1e-5, atol=2e-6)
        np.testing.assert_allclose(got[:, half:], z.imag, rtol=1e-5, atol=2e-6)
    twice = oracle.qwen3_rope(oracle.qwen3_rope(x, heads, d, 300, theta), heads, d, 211, theta)
    np.testing.assert_allclose(twice, oracle.qwen3_rope(x, heads, d, 511, theta), rtol=0,
                               atol=1e-5)


def test_qwen3_qk_norm_applies_weight_after_normalising():
    """RMSNorm with weight w equals the unit-weight result times w, element by
    element, and the unit-weight result has unit RMS per head."""
    rng = np.random.default_rng(12)
    heads, d = 4, 128
    x = (3 * rng.standard_normal(heads * d)).astype(np.float32)
    w = (1 + 0.2 * rng.standard_normal(d)).astype(np.float32)
    unit = oracle.qwen3_qk_norm(x, heads, d, np.ones(d, np.float32), 1e-6).reshape(heads, d)
    got = oracle.qwen3_qk_norm(x, heads, d, w, 1e-6).reshape(heads, d)
    np.testing.assert_allclose(got, unit * w, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(np.sqrt((unit.astype(np.float64) ** 2).mean(1)), 1.0, rtol=1e-5)


def test_add_silu_mul_and_batched_rms_norm_closed_forms():
    """add is the float32 sum; silu_mul is g * sigmoid(g) * up (0 at g = 0, up * g
    for large g, -> 0 for very negative g); the batched RMSNorm is the per-row
    RMSNorm with weight."""
    rng = np.random.default_rng(13)
    a = rng.standard_normal(1000).astype(np.float32)
    b = rng.standard_normal(1000).astype(np.float32)
    np.testing.assert_array_equal(oracle.add(a, b), a + b)
    g = np.array([0.0, 30.0, -30.0, 1.0, -2.0], np.float32)
    up = np.array([5.0, 2.0, 3.0, 4.0, -1.5], np.float32)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * up
    np.testing.assert_allclose(oracle.silu_mul(g, up), want, rtol=1e-6, atol=1e-30)
    assert oracle.silu_mul(g, up)[0] == 0.0
    x = (3 * rng.standard_normal(3 * 1024)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(1024)).astype(np.float32)
    got = oracle.rms_norm_batched(x, w, 3, 1024, 1e-6).reshape(3, 1024)
    xr = x.reshape(3, 1024).astype(np.float64)
    ref = xr / np.sqrt((xr ** 2).mean(1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)


# ------------------------------------------------- gate and KV append ----

def test_sigmoid_gate_mul_equals_mul_of_sigmoid_and_closed_forms():
    """The fused output gate (qwen35_runtime.cpp:3347-3355: sigmoid_f32_in_place on G,
    then mul_f32_in_place into o) equals o * sigmoid(G) built from the smoke-pinned
    sigmoid and mul ops, up to the one f32 rounding of sigmoid(G) those two round
    separately; G = 0 halves o, large G keeps o, very negative G zeroes it, and
    negating G must change the result (sigmoid(-g) = 1 - sigmoid(g))."""
    rng = np.random.default_rng(21)
    o = (3 * rng.standard_normal(4096)).astype(np.float32)
    g = (2 * rng.standard_normal(4096)).astype(np.float32)
    got = oracle.sigmoid_gate_mul(o, g)
    chained = oracle.mul(o, oracle.sigmoid(g))
    np.testing.assert_allclose(got, chained, rtol=2.5e-7, atol=0)
    want = o.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))
    np.testing.assert_allclose(got, want, rtol=1.2e-7, atol=0)
    flipped = oracle.sigmoid_gate_mul(o, -g)
    np.testing.assert_allclose(flipped, o.astype(np.float64) - want, rtol=2e-6, atol=2e-6)
    big = np.abs(g) > 0.5
    assert np.all(np.abs(flipped - got)[big] > 1e-3 * np.abs(o)[big])
    edge_o = np.array([5.0, -3.0, 7.0, 2.0], np.float32)
    edge_g = np.array([0.0, 0.0, 40.0, -120.0], np.float32)
    np.testing.assert_array_equal(oracle.sigmoid_gate_mul(edge_o, edge_g),
                                  np.array([2.5, -1.5, 7.0, 0.0], np.float32))
    # The output buffer is the first operand: gate and output must not be swapped.
    assert not np.allclose(oracle.sigmoid_gate_mul(g, o), got)


def test_copy_f32_rows_to_f16_equals_rounded_row_copy_with_distinct_strides():
    """The KV append (mps_backend.mm:2655-2666: cache[dst_off + r dst_stride + c] =
    half(x[src_off + r src_stride + c])) equals the smoke-pinned f32 row copy followed by
    the exhaustively pinned f32 -> f16 rounding, and an independent numpy scatter; four
    distinct strides and offsets make any swap of source and destination geometry fail,
    and bytes outside the copied rows keep their values."""
    rng = np.random.default_rng(22)
    rows, row_size = 5, 24
    src_stride, src_off, dst_stride, dst_off = 37, 3, 29, 11
    src = (4 * rng.standard_normal(src_off + rows * src_stride)).astype(np.float32)
    # Long enough for both geometries, so the swapped call below stays in bounds.
    dst_len = max(dst_off + rows * dst_stride, src_off + rows * src_stride) + 7
    background = rng.integers(0, 2**16, dst_len, dtype=np.uint16)
    got = oracle.copy_f32_rows_to_f16(src, background, rows, row_size, src_stride, src_off,
                                      dst_stride, dst_off)
    via_f32 = oracle.copy_f32_rows(src, np.zeros(dst_len, np.float32), rows, row_size,
                                   src_stride, src_off, dst_stride, dst_off)
    ref = background.copy()
    idx_d = dst_off + np.arange(rows)[:, None] * dst_stride + np.arange(row_size)[None, :]
    idx_s = src_off + np.arange(rows)[:, None] * src_stride + np.arange(row_size)[None, :]
    ref[idx_d] = src[idx_s].astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(got[idx_d], oracle.f32_to_f16_bits(via_f32[idx_d]))
    untouched = np.ones(dst_len, bool)
    untouched[idx_d.ravel()] = False
    np.testing.assert_array_equal(got[untouched], background[untouched])
    swapped = oracle.copy_f32_rows_to_f16(src, background, rows, row_size, dst_stride, dst_off,
                                          src_stride, src_off)
    assert not np.array_equal(swapped, got)
