"""The two numpy products of the oracle's chunked prompt pass
(tests/qwen35_decode_cases.py: gemm_f16, causal_attention_f16q) against the C
oracle they stand in for, on cases small enough for the oracle's loops:
kquant_matmul with f16 weights and inputs (run_qwen35_quant_matmul above 8
tokens), and attention_batched with the query rounded to f16 (the flash
path).  CPU only."""
import numpy as np
import pytest

import gguf_writer as gw
import oracle
import qwen35_decode_cases as qc


@pytest.mark.parametrize("ggml_type", [gw.GGML_Q4_K, gw.GGML_Q5_K, gw.GGML_Q6_K])
def test_gemm_f16_matches_oracle_kquant_matmul(ggml_type):
    rng = np.random.default_rng(ggml_type)
    rows, cols, tokens = 48, 512, 13
    data = qc.quant(rng, ggml_type, rows, cols)
    x = (3 * rng.standard_normal(tokens * cols)).astype(np.float32)
    w = oracle.kquant_dequantize(qc.FMT[ggml_type], data, rows * cols // 256).reshape(rows, cols)
    got = qc.gemm_f16(w, x, tokens)
    want = oracle.kquant_matmul(qc.FMT[ggml_type], data, rows, cols, x, tokens, weight_f16=True,
                                input_f16=True)
    scale = np.abs(qc.f16_round(x).reshape(tokens, cols)) @ np.abs(qc.f16_round(w)).T
    assert np.all(np.abs(got - want) <= 1e-6 * scale.reshape(-1) + 1e-7)
    # Without the f16 rounding of the input the products differ: the rule matters.
    plain = oracle.kquant_matmul(qc.FMT[ggml_type], data, rows, cols, x, tokens)
    assert np.abs(plain - want).max() > 1e-4 * np.abs(want).max()


@pytest.mark.parametrize("start,tokens", [(0, 9), (5, 7), (20, 1)])
def test_causal_attention_f16q_matches_oracle_attention(start, tokens):
    rng = np.random.default_rng(start + tokens)
    heads, kv_heads, d = 8, 2, 256
    cap = start + tokens + 3
    q = (2 * rng.standard_normal(tokens * heads * d)).astype(np.float32)
    kc = rng.standard_normal(cap * kv_heads * d).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(cap * kv_heads * d).astype(np.float16).view(np.uint16)
    got = qc.causal_attention_f16q(q, kc, vc, start, tokens, cap, heads, kv_heads, d)
    want = oracle.attention_batched(q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d,
                                    round_query_f16=True)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    f32q = oracle.attention_batched(q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d)
    assert np.abs(f32q - want).max() > 1e-5
