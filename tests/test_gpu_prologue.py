"""GPU parity of the fused full-attention prologue
(kraken_hip_qwen35_attention_prologue_f16_kv) with the op chain it replaces,
qwen35_runtime.cpp:3229-3326: copy_f32_rows x2 (Q/gate split), qk_norm x2,
mrope x2, copy_f32_rows_to_f16 x2 (K/V append).

* Against the same chain of unfused HIP ops: equal bit for bit (the fused
  kernel keeps their element layout, reduction order and double-precision
  angles), query, gate, and both caches, including rows outside the chunk.
* Against the CPU oracle chain: query within 1e-5, K cache rows within one f16
  unit in the last place, V cache and gate exact.
Shapes: C1/C2's 8 Q / 2 KV heads at head_dim 256 with Qwen3.5's MRoPE sections
(11, 11, 10, 0) and theta 1e7, a 128-dim case with every section in use and
head_dim == n_dims, text positions generated on the device and explicit
positions that differ per section row.
"""
import numpy as np
import pytest

import kraken_hip as kh
import oracle

EPS = 1e-6


def chain_inputs(seed, tokens, heads, kv_heads, d, cap, layers):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    return dict(
        qg=f(tokens, heads, 2, d), key=f(tokens, kv_heads * d), value=f(tokens, kv_heads * d),
        q_norm=(1 + 0.1 * f(d)).astype(np.float32), k_norm=(1 + 0.1 * f(d)).astype(np.float32),
        kc=oracle.f32_to_f16_bits(f(layers * cap * kv_heads * d)),
        vc=oracle.f32_to_f16_bits(f(layers * cap * kv_heads * d)))


CASES = [
    # tokens, start, cap, layers, layer, heads, kv_heads, d, n_dims, sections, explicit positions
    (1, 37, 40, 2, 1, 8, 2, 256, 64, (11, 11, 10, 0), False),
    (5, 0, 8, 1, 0, 8, 2, 256, 64, (11, 11, 10, 0), True),
    (70, 100, 180, 3, 2, 8, 2, 256, 64, (11, 11, 10, 0), False),
    (9, 3, 12, 1, 0, 4, 4, 128, 128, (24, 20, 12, 8), True),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES)
def test_prologue_matches_unfused_chain_and_oracle(hip_ctx, case):
    tokens, start, cap, layers, layer, heads, kv_heads, d, n_dims, sections, explicit = case
    print(f"prologue {case}", flush=True)
    x = chain_inputs(7 + tokens, tokens, heads, kv_heads, d, cap, layers)
    kv_dim = kv_heads * d
    theta = 1e7
    if explicit:
        rng = np.random.default_rng(tokens)
        pos = rng.integers(0, 5000, size=4 * tokens).astype(np.int32)
    else:
        pos = oracle.make_mrope_positions(start, tokens)
    ctx = hip_ctx

    # Fused.
    b = {k: ctx.buffer(v) for k, v in x.items()}
    pos_b = ctx.buffer(pos) if explicit else None
    qo = ctx.buffer(byte_size=4 * tokens * heads * d)
    go = ctx.buffer(byte_size=4 * tokens * heads * d)
    ctx.qwen35_attention_prologue_f16_kv(b["qg"], b["key"], b["value"], b["q_norm"], b["k_norm"],
                                         pos_b, start, b["kc"], b["vc"], layer, start, tokens, cap,
                                         heads, kv_heads, d, n_dims, *sections, theta, EPS, qo, go)
    fq = qo.download(tokens * heads * d)
    fg = go.download(tokens * heads * d)
    fkc = b["kc"].download(dtype=np.uint16)
    fvc = b["vc"].download(dtype=np.uint16)
    np.testing.assert_array_equal(b["key"].download(), x["key"].ravel())  # key not modified

    # The unfused HIP chain.
    c = {k: ctx.buffer(v) for k, v in x.items()}
    pos_c = ctx.buffer(pos)
    q = ctx.buffer(byte_size=4 * tokens * heads * d)
    g = ctx.buffer(byte_size=4 * tokens * heads * d)
    off = (layer * cap + start) * kv_dim
    ctx.copy_f32_rows(c["qg"], q, tokens * heads, d, 2 * d, 0, d, 0)
    ctx.copy_f32_rows(c["qg"], g, tokens * heads, d, 2 * d, d, d, 0)
    ctx.qk_norm_f32_f32_batched(q, c["q_norm"], tokens, heads, d, EPS)
    ctx.qk_norm_f32_f32_batched(c["key"], c["k_norm"], tokens, kv_heads, d, EPS)
    ctx.mrope_f32_in_place(q, pos_c, tokens, heads, d, n_dims, *sections, theta)
    ctx.mrope_f32_in_place(c["key"], pos_c, tokens, kv_heads, d, n_dims, *sections, theta)
    ctx.copy_f32_rows_to_f16(c["key"], c["kc"], tokens, kv_dim, kv_dim, 0, kv_dim, off)
    ctx.copy_f32_rows_to_f16(c["value"], c["vc"], tokens, kv_dim, kv_dim, 0, kv_dim, off)
    np.testing.assert_array_equal(fq, q.download(tokens * heads * d))
    np.testing.assert_array_equal(fg, g.download(tokens * heads * d))
    np.testing.assert_array_equal(fkc, c["kc"].download(dtype=np.uint16))
    np.testing.assert_array_equal(fvc, c["vc"].download(dtype=np.uint16))

    # The oracle chain.
    qg = x["qg"]
    oq = np.ascontiguousarray(qg[:, :, 0, :]).ravel()
    og = np.ascontiguousarray(qg[:, :, 1, :]).ravel()
    oq = oracle.qk_norm_f32_batched(oq, x["q_norm"], tokens, heads, d, EPS)
    ok = oracle.qk_norm_f32_batched(x["key"].ravel(), x["k_norm"], tokens, kv_heads, d, EPS)
    oq = oracle.mrope(oq, pos, tokens, heads, d, n_dims, sections, theta)
    ok = oracle.mrope(ok, pos, tokens, kv_heads, d, n_dims, sections, theta)
    okc = oracle.copy_f32_rows_to_f16(ok, x["kc"], tokens, kv_dim, kv_dim, 0, kv_dim, off)
    ovc = oracle.copy_f32_rows_to_f16(x["value"].ravel(), x["vc"], tokens, kv_dim, kv_dim, 0,
                                      kv_dim, off)
    np.testing.assert_allclose(fq, oq, rtol=0, atol=1e-5)
    np.testing.assert_array_equal(fg, og)
    assert np.abs(fkc.astype(np.int32) - okc.astype(np.int32)).max() <= 1
    np.testing.assert_array_equal(fvc, ovc)


# ------------------------------------- prologue folded into decode attention --
# kraken_hip_qwen35_attention_prologue_gated_f16_kv: one decode token with
# head_dim 256, G in {1, 2, 4} and at most 256 keys runs as one launch (the
# short-split decode kernel normalises and rotates its heads, appends the K/V
# row and uses it in place of the loaded row); other shapes run the prologue
# entry then the gated attention entry.  Either way the output and both caches
# equal, bit for bit, those of the two entries called one after the other, and
# the output is within the attention tests' tolerance of the oracle chain.
GATED_CASES = [
    # heads, kv_heads, tokens, start, cap, layers, layer, explicit positions
    (8, 2, 1, 0, 8, 1, 0, False),
    (8, 2, 1, 15, 40, 2, 1, False),
    (8, 2, 1, 16, 40, 2, 1, True),
    (8, 2, 1, 37, 64, 2, 1, False),
    (8, 2, 1, 255, 300, 1, 0, False),   # 256 keys: the last one-launch length
    (8, 2, 1, 256, 300, 1, 0, False),   # 257 keys: two launches (split decode)
    (4, 4, 1, 20, 32, 1, 0, False),     # G = 1
    (8, 4, 1, 70, 80, 1, 0, True),      # G = 2
    (16, 2, 1, 5, 8, 1, 0, False),      # G = 8: two launches
    (8, 2, 3, 9, 16, 1, 0, False),      # three tokens: two launches
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", GATED_CASES)
def test_prologue_gated_equals_two_entries_and_oracle(hip_ctx, case):
    heads, kv_heads, tokens, start, cap, layers, layer, explicit = case
    print(f"prologue gated {case}", flush=True)
    d, n_dims, sections, theta = 256, 64, (11, 11, 10, 0), 1e7
    x = chain_inputs(100 + start, tokens, heads, kv_heads, d, cap, layers)
    if explicit:
        pos = np.random.default_rng(start).integers(0, 5000, size=4 * tokens).astype(np.int32)
    else:
        pos = oracle.make_mrope_positions(start, tokens)
    ctx = hip_ctx
    n = tokens * heads * d

    def run(one_call):
        b = {k: ctx.buffer(v) for k, v in x.items()}
        pos_b = ctx.buffer(pos) if explicit else None
        qo = ctx.buffer(np.full(n, 3.0, np.float32))
        go = ctx.buffer(np.full(n, 3.0, np.float32))
        out = ctx.buffer(byte_size=4 * n)
        args = (b["qg"], b["key"], b["value"], b["q_norm"], b["k_norm"], pos_b, start, b["kc"],
                b["vc"], layer, start, tokens, cap, heads, kv_heads, d, n_dims, *sections, theta,
                EPS, qo, go)
        if one_call:
            ctx.qwen35_attention_prologue_gated_f16_kv(*args, out)
        else:
            ctx.qwen35_attention_prologue_f16_kv(*args)
            ctx.attention_f32_batched_f16_kv_gated(qo, b["kc"], b["vc"], go, layer, start, tokens,
                                                   cap, heads, kv_heads, d, out)
        return (out.download(n), b["kc"].download(dtype=np.uint16),
                b["vc"].download(dtype=np.uint16), qo.download(n))

    got, gkc, gvc, gq = run(True)
    want, wkc, wvc, _ = run(False)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(gkc, wkc)
    np.testing.assert_array_equal(gvc, wvc)
    one_launch = tokens == 1 and heads // kv_heads in (1, 2, 4) and start < 256
    # The one-launch form leaves the two-launch scratch as it was.
    assert np.all(gq == 3.0) == one_launch

    # The oracle chain: prologue, attention over the updated caches, gate.
    kv_dim = kv_heads * d
    qg = x["qg"]
    oq = np.ascontiguousarray(qg[:, :, 0, :]).ravel()
    og = np.ascontiguousarray(qg[:, :, 1, :]).ravel()
    oq = oracle.qk_norm_f32_batched(oq, x["q_norm"], tokens, heads, d, EPS)
    ok = oracle.qk_norm_f32_batched(x["key"].ravel(), x["k_norm"], tokens, kv_heads, d, EPS)
    oq = oracle.mrope(oq, pos, tokens, heads, d, n_dims, sections, theta)
    ok = oracle.mrope(ok, pos, tokens, kv_heads, d, n_dims, sections, theta)
    off = (layer * cap + start) * kv_dim
    okc = oracle.copy_f32_rows_to_f16(ok, x["kc"], tokens, kv_dim, kv_dim, 0, kv_dim, off)
    ovc = oracle.copy_f32_rows_to_f16(x["value"].ravel(), x["vc"], tokens, kv_dim, kv_dim, 0,
                                      kv_dim, off)
    ref = oracle.attention_batched(oq, okc, ovc, layer, start, tokens, cap, heads, kv_heads, d)
    ref = oracle.sigmoid_gate_mul(ref, og)
    np.testing.assert_allclose(got, ref, rtol=2e-3, atol=1e-3)
