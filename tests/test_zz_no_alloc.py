"""The allocation-free attention entry point
(kraken_hip_attention_f32_batched_f16_kv_gated_no_alloc) against the entry it
varies (kraken_hip_attention_f32_batched_f16_kv_gated): same inputs, same
kernels, so the outputs must be bit-identical.  Two calls in a row on the
shared static scratch, the second with a smaller input (a shorter KV cache and
fewer splits), then a prefill that uses no scratch; shapes whose partials do
not fit the array are rejected without launching."""
import numpy as np
import pytest

import kraken_hip as kh

HEADS, KV_HEADS, D = 8, 2, 256


def case(seed, tokens, start):
    rng = np.random.default_rng(seed)
    cap = start + tokens
    q = rng.standard_normal(tokens * HEADS * D).astype(np.float32)
    gate = rng.standard_normal(tokens * HEADS * D).astype(np.float32)
    k = rng.standard_normal(cap * KV_HEADS * D).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(cap * KV_HEADS * D).astype(np.float16).view(np.uint16)
    return q, gate, k, v, cap


def run(ctx, name, q, gate, k, v, start, tokens, cap):
    bufs = [ctx.buffer(a) for a in (q, k, v, gate)]
    out = ctx.buffer(byte_size=4 * q.size)
    ctx.call(name, bufs[0], bufs[1], bufs[2], bufs[3], 0, start, tokens, cap, HEADS, KV_HEADS,
             D, out)
    return out.download(q.size)


@pytest.mark.gpu
def test_no_alloc_attention_matches_allocating_entry(hip_ctx):
    # Decode at a long then a short KV cache (split partials in the scratch
    # array, the second call over fewer of them), then a 64-token prefill.
    for seed, tokens, start in ((1, 1, 16383), (2, 1, 700), (3, 64, 0)):
        print(f"no-alloc attention tokens={tokens} start={start}", flush=True)
        q, gate, k, v, cap = case(seed, tokens, start)
        want = run(hip_ctx, "attention_f32_batched_f16_kv_gated", q, gate, k, v, start, tokens,
                   cap)
        got = run(hip_ctx, "attention_f32_batched_f16_kv_gated_no_alloc", q, gate, k, v, start,
                  tokens, cap)
        assert np.all(np.isfinite(got))
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
def test_no_alloc_attention_rejects_oversized_partials(hip_ctx):
    tokens, start = 1024, 7168  # long prefill split over the KV: 33 MB of partials
    cap = start + tokens
    q = hip_ctx.buffer(byte_size=4 * tokens * HEADS * D)
    kv = hip_ctx.buffer(byte_size=2 * cap * KV_HEADS * D)
    code = hip_ctx.status("attention_f32_batched_f16_kv_gated_no_alloc", q, kv, kv, q, 0, start,
                          tokens, cap, HEADS, KV_HEADS, D, q)
    assert code == kh.INVALID_ARGUMENT
    assert "allocation-free entry point has 8388608" in kh.last_error()
