"""C0: the legacy Qwen3-0.6B-shaped attention of the reference's CPU path on the GPU.

16 Q heads, 8 KV heads, head_dim 128, per-head RMSNorm on q/k with non-unit
weights (1 + 0.2 N(0,1), different for q and k),
RoPE theta 1e6, a 512-token prefill then 64 decode steps; q/k/v fp32 ~ N(0,1),
seed 0, batch 1, one layer.  The oracle restates qwen_cpu_model.cpp:1019-1130
(token-by-token, double-precision norm and rope angles).  The HIP path runs
the same math through the C ABI: qk_norm_f32_f32_batched, mrope_f32_in_place
with all pairs on the text position row (sections (64,0,0,0), n_dims = 128 --
identical to full-rotary RoPE), copy_f32_rows into an F32 KV cache, then
attention_f32_batched for the 512-token prefill chunk and each decode token.
Tolerance: 1e-4 (f32 KV, no fp16 rounding anywhere).
"""
import numpy as np
import pytest

import kraken_hip as kh
import oracle


@pytest.mark.gpu
def test_c0_prefill_then_decode_matches_cpu_reference(hip_ctx):
    heads, kv_heads, d = 16, 8, 128
    prefill, decode = 512, 64
    total = prefill + decode
    rng = np.random.default_rng(0)
    q = rng.standard_normal(total * heads * d).astype(np.float32)
    k = rng.standard_normal(total * kv_heads * d).astype(np.float32)
    v = rng.standard_normal(total * kv_heads * d).astype(np.float32)
    qw = (1 + 0.2 * rng.standard_normal(d)).astype(np.float32)
    kw = (1 + 0.2 * rng.standard_normal(d)).astype(np.float32)
    _, _, _, ref = oracle.qwen3_attention_sequence(q, k, v, total, heads, kv_heads, d, qw, kw,
                                                   1e-6, 1e6)
    ctx = hip_ctx
    kc = ctx.buffer(np.zeros(total * kv_heads * d, np.float32))
    vc = ctx.buffer(np.zeros(total * kv_heads * d, np.float32))
    qwb, kwb = ctx.buffer(qw), ctx.buffer(kw)
    outs = []
    for t0, n in [(0, prefill)] + [(prefill + i, 1) for i in range(decode)]:
        qb = ctx.buffer(q[t0 * heads * d:(t0 + n) * heads * d])
        kb = ctx.buffer(k[t0 * kv_heads * d:(t0 + n) * kv_heads * d])
        vb = ctx.buffer(v[t0 * kv_heads * d:(t0 + n) * kv_heads * d])
        pos = ctx.buffer(oracle.make_mrope_positions(t0, n))
        out = ctx.buffer(byte_size=4 * n * heads * d)
        ctx.begin_graph()
        ctx.qk_norm_f32_f32_batched(qb, qwb, n, heads, d, 1e-6)
        ctx.qk_norm_f32_f32_batched(kb, kwb, n, kv_heads, d, 1e-6)
        ctx.mrope_f32_in_place(qb, pos, n, heads, d, d, d // 2, 0, 0, 0, 1e6)
        ctx.mrope_f32_in_place(kb, pos, n, kv_heads, d, d, d // 2, 0, 0, 0, 1e6)
        kvd = kv_heads * d
        ctx.copy_f32_rows(kb, kc, n, kvd, kvd, 0, kvd, t0 * kvd)
        ctx.copy_f32_rows(vb, vc, n, kvd, kvd, 0, kvd, t0 * kvd)
        ctx.attention_f32_batched(qb, kc, vc, 0, t0, n, total, heads, kv_heads, d, out)
        ctx.commit_graph()
        outs.append(out.download())
    got = np.concatenate(outs)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)
