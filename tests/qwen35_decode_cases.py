"""A synthetic Qwen3.5-0.8B GGUF and the oracle's greedy decode over it.

The model has the 0.8B plan's shapes (hidden 1024, 24 layers: linear
attention except every fourth, 8/2 attention heads of 256, 16 GDN heads of
128, conv kernel 4, FFN 3584, vocabulary 248320, LM head tied to token_embd)
and GGUF tensor names of the reference's weight map (qwen35_weight_map.cpp).
Projection weights are random K-quant blocks whose f16 scales are set so a
weight is a few hundredths, which keeps activations O(1) through the layers;
norm weights are 1 + 0.1 N(0,1).

OracleDecoder replays run_qwen35_decode_tokens (qwen35_runtime.cpp:3860-3936)
for one token per step through the oracle's functions: each layer's RMSNorm,
K-quant projections (fp32, as the reference multiplies one token), the
linear-attention or full-attention core, residual adds and the SwiGLU FFN;
then the output norm and the LM head's argmax.  Its prefill_chunk replays the
prompt pass of generate_qwen35_metal (qwen35_runtime.cpp:5787-6004) for one
chunk of many tokens: the same ops over the whole chunk, with the chunk's
projections at the reference's GEMM precision (weights and inputs rounded to
f16, run_qwen35_quant_matmul for more than 8 tokens) and its attention at the
flash kernel's (query rounded to f16, mps_backend.mm:3458-3461).  Those two
products go through numpy (float32 sums of f16 products, and float64 softmax
attention) for speed; everything else is the C oracle's, and
tests/test_qwen35_prefill_cases.py checks both numpy products against the
oracle's own kquant_matmul and attention_batched on small cases.
"""
import numpy as np

import gguf_writer as gw
import oracle

HIDDEN, LAYERS, VOCAB, FFN = 1024, 24, 248320, 3584
HEADS, KV_HEADS, HEAD_DIM = 8, 2, 256
HK = HV = 16
DK = 128
CONV_K = 4
CONV_CH = (2 * HK + HV) * DK
INNER = HV * DK
ROPE_DIMS, SECTIONS, THETA, EPS = 64, (11, 11, 10, 0), 1.0e7, 1.0e-6
FMT = {gw.GGML_Q4_K: "q4_k", gw.GGML_Q5_K: "q5_k", gw.GGML_Q6_K: "q6_k"}
BLOCK = {gw.GGML_Q4_K: 144, gw.GGML_Q5_K: 176, gw.GGML_Q6_K: 210}
# f16 scale ranges (d, dmin) that give weights of a few hundredths.
SCALE = {gw.GGML_Q4_K: (1.5e-4, 1.0e-3), gw.GGML_Q5_K: (8e-5, 1.0e-3), gw.GGML_Q6_K: (4e-5, 0)}


def full_attention(layer):
    return (layer + 1) % 4 == 0


def quant(rng, ggml_type, rows, cols):
    """Random blocks with d in [0.5, 1.5] x SCALE and dmin in [0, 1] x SCALE."""
    nb = BLOCK[ggml_type]
    blocks = rows * cols // 256
    w = rng.integers(0, 256, size=(blocks, nb), dtype=np.uint8)
    d_scale, m_scale = SCALE[ggml_type]
    d = (d_scale * rng.uniform(0.5, 1.5, blocks)).astype(np.float16).view(np.uint8)
    if ggml_type == gw.GGML_Q6_K:
        w[:, 208:210] = d.reshape(-1, 2)
    else:
        w[:, 0:2] = d.reshape(-1, 2)
        dm = (m_scale * rng.uniform(0, 1, blocks)).astype(np.float16).view(np.uint8)
        w[:, 2:4] = dm.reshape(-1, 2)
    return w.reshape(-1)


def build_model(seed=35):
    """name -> (shape innermost first, ggml type, data)."""
    rng = np.random.default_rng(seed)
    t = {}

    def q(name, ggml_type, rows, cols):
        t[name] = ((cols, rows), ggml_type, quant(rng, ggml_type, rows, cols))

    def f(name, values):
        values = np.asarray(values, np.float32)
        t[name] = ((values.size,) if values.ndim == 1 else values.shape[::-1], gw.GGML_F32,
                   values)

    def norm(n):
        return 1 + 0.1 * rng.standard_normal(n)

    q("token_embd.weight", gw.GGML_Q6_K, VOCAB, HIDDEN)
    f("output_norm.weight", norm(HIDDEN))
    for i in range(LAYERS):
        p = f"blk.{i}."
        f(p + "attn_norm.weight", norm(HIDDEN))
        f(p + "post_attention_norm.weight", norm(HIDDEN))
        q(p + "ffn_gate.weight", gw.GGML_Q4_K, FFN, HIDDEN)
        q(p + "ffn_up.weight", gw.GGML_Q4_K, FFN, HIDDEN)
        q(p + "ffn_down.weight", gw.GGML_Q6_K, HIDDEN, FFN)
        if full_attention(i):
            q(p + "attn_q.weight", gw.GGML_Q4_K, HEADS * 2 * HEAD_DIM, HIDDEN)
            q(p + "attn_k.weight", gw.GGML_Q4_K, KV_HEADS * HEAD_DIM, HIDDEN)
            q(p + "attn_v.weight", gw.GGML_Q6_K, KV_HEADS * HEAD_DIM, HIDDEN)
            q(p + "attn_output.weight", gw.GGML_Q4_K, HIDDEN, HEADS * HEAD_DIM)
            f(p + "attn_q_norm.weight", norm(HEAD_DIM))
            f(p + "attn_k_norm.weight", norm(HEAD_DIM))
        else:
            q(p + "attn_qkv.weight", gw.GGML_Q5_K, CONV_CH, HIDDEN)
            q(p + "attn_gate.weight", gw.GGML_Q4_K, INNER, HIDDEN)
            q(p + "ssm_beta.weight", gw.GGML_Q4_K, HV, HIDDEN)
            q(p + "ssm_alpha.weight", gw.GGML_Q4_K, HV, HIDDEN)
            q(p + "ssm_out.weight", gw.GGML_Q4_K, HIDDEN, INNER)
            conv = (0.3 * rng.standard_normal((CONV_CH, CONV_K))).astype(np.float32)
            t[p + "ssm_conv1d.weight"] = ((CONV_K, CONV_CH), gw.GGML_F32, conv)
            f(p + "ssm_dt.bias", 0.5 * rng.standard_normal(HV))
            f(p + "ssm_a", -(0.2 + rng.random(HV)))
            f(p + "ssm_norm.weight", norm(DK))
    return t


def write_gguf(path, model):
    meta = [("general.architecture", gw.STRING, "qwen35"),
            ("general.alignment", gw.U32, 32),
            ("qwen35.block_count", gw.U32, LAYERS),
            ("qwen35.embedding_length", gw.U32, HIDDEN),
            ("qwen35.feed_forward_length", gw.U32, FFN),
            ("qwen35.attention.head_count", gw.U32, HEADS),
            ("qwen35.attention.head_count_kv", gw.U32, KV_HEADS),
            ("qwen35.rope.freq_base", gw.F32, THETA),
            ("qwen35.attention.layer_norm_rms_epsilon", gw.F32, EPS)]
    tensors = [(name, shape, typ, data) for name, (shape, typ, data) in model.items()]
    return gw.write(path, meta, tensors)


def f16_round(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def gemm_f16(weight_f32, x, tokens):
    """run_qwen35_quant_matmul for more than 8 tokens: out [tokens][rows] =
    f16(x) [tokens][cols] times f16(W)^T, summed in float32 (f16 products are
    exact in float32)."""
    rows, cols = weight_f32.shape
    xx = f16_round(np.asarray(x, np.float32).reshape(tokens, cols))
    return (xx @ f16_round(weight_f32).T).astype(np.float32).reshape(-1)


def causal_attention_f16q(q, kc_bits, vc_bits, start, tokens, cap, heads, kv_heads, d):
    """attention_batched over cache positions 0 .. start + t for query token t,
    with the query rounded to f16 (the flash path), K/V the cache's f16 values;
    float64 softmax.  q [tokens][heads][d] -> out [tokens][heads][d]."""
    n = start + tokens
    k = kc_bits.view(np.float16).astype(np.float64).reshape(cap, kv_heads, d)[:n]
    v = vc_bits.view(np.float16).astype(np.float64).reshape(cap, kv_heads, d)[:n]
    qq = f16_round(q).astype(np.float64).reshape(tokens, heads, d)
    group = heads // kv_heads
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    mask = np.arange(n)[None, :] > (start + np.arange(tokens))[:, None]
    out = np.empty((tokens, heads, d))
    for hh in range(heads):
        s = qq[:, hh, :] @ k[:, hh // group, :].T * scale
        s[mask] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, hh, :] = (p @ v[:, hh // group, :]) / p.sum(axis=1, keepdims=True)
    return out.astype(np.float32).reshape(-1)


class OracleDecoder:
    """The oracle's greedy decode over `model`, one token per step (step), and
    its chunked prompt pass (prefill_chunk) over the same caches."""

    def __init__(self, model, capacity):
        self.m = model
        self.cap = capacity
        kv = KV_HEADS * HEAD_DIM
        self.conv = [np.zeros((CONV_K - 1) * CONV_CH, np.float32) for _ in range(LAYERS)]
        self.state = [np.zeros(HV * DK * DK, np.float32) for _ in range(LAYERS)]
        self.kc = [np.zeros(capacity * kv, np.uint16) for _ in range(LAYERS)]
        self.vc = [np.zeros(capacity * kv, np.uint16) for _ in range(LAYERS)]

    def proj(self, name, x):
        (cols, rows), typ, data = self.m[name]
        return oracle.kquant_matmul(FMT[typ], data, rows, cols, x, 1)

    def dequant(self, name):
        (cols, rows), typ, data = self.m[name]
        return oracle.kquant_dequantize(FMT[typ], data, rows * cols // 256).reshape(rows, cols)

    def proj_chunk(self, name, x, tokens):
        assert tokens > 8, "the chunk products follow the GEMM precision"
        return gemm_f16(self.dequant(name), x, tokens)

    def embed(self, token_ids):
        (_, _), typ, emb = self.m["token_embd.weight"]
        row = HIDDEN // 256 * BLOCK[typ]
        return np.concatenate([
            oracle.kquant_dequantize(FMT[typ], emb[t * row:(t + 1) * row], HIDDEN // 256)
            for t in token_ids])

    def linear_chunk(self, i, h, t):
        p = f"blk.{i}."
        n = oracle.rms_norm_batched(h, self.vec(p + "attn_norm.weight"), t, HIDDEN, EPS)
        qkv, z = self.proj_chunk(p + "attn_qkv.weight", n, t), self.proj_chunk(
            p + "attn_gate.weight", n, t)
        beta = self.proj_chunk(p + "ssm_beta.weight", n, t)
        alpha = self.proj_chunk(p + "ssm_alpha.weight", n, t)
        ci, self.conv[i] = oracle.build_ssm_conv_state(self.conv[i], qkv, CONV_K, CONV_CH, t)
        y = oracle.silu(oracle.ssm_conv(ci, self.vec(p + "ssm_conv1d.weight"), CONV_K, CONV_CH,
                                        t, 1))
        q, k, v = oracle.split_qkv_l2_norm(y, t, HK, HV, DK, EPS)
        g, b = oracle.prepare_gdn_gate_beta(alpha, beta, self.vec(p + "ssm_dt.bias"),
                                            self.vec(p + "ssm_a"), t, HV)
        o, self.state[i] = oracle.gated_delta_net(q, k, v, g, b, self.state[i], t, HK, HV, DK)
        o = oracle.norm_gated(o, self.vec(p + "ssm_norm.weight"), z, t, HV, DK, EPS)
        return self.proj_chunk(p + "ssm_out.weight", o, t)

    def full_chunk(self, i, h, start, t):
        p = f"blk.{i}."
        n = oracle.rms_norm_batched(h, self.vec(p + "attn_norm.weight"), t, HIDDEN, EPS)
        qg = self.proj_chunk(p + "attn_q.weight", n, t).reshape(t, HEADS, 2, HEAD_DIM)
        q, gate = qg[:, :, 0].ravel(), qg[:, :, 1].ravel()
        k, v = self.proj_chunk(p + "attn_k.weight", n, t), self.proj_chunk(p + "attn_v.weight",
                                                                           n, t)
        q = oracle.qk_norm_f32_batched(q, self.vec(p + "attn_q_norm.weight"), t, HEADS,
                                       HEAD_DIM, EPS)
        k = oracle.qk_norm_f32_batched(k, self.vec(p + "attn_k_norm.weight"), t, KV_HEADS,
                                       HEAD_DIM, EPS)
        positions = oracle.make_mrope_positions(start, t)
        q = oracle.mrope(q, positions, t, HEADS, HEAD_DIM, ROPE_DIMS, SECTIONS, THETA)
        k = oracle.mrope(k, positions, t, KV_HEADS, HEAD_DIM, ROPE_DIMS, SECTIONS, THETA)
        kv = KV_HEADS * HEAD_DIM
        self.kc[i][start * kv:(start + t) * kv] = oracle.f32_to_f16_bits(k)
        self.vc[i][start * kv:(start + t) * kv] = oracle.f32_to_f16_bits(v)
        a = causal_attention_f16q(q, self.kc[i], self.vc[i], start, t, self.cap, HEADS,
                                  KV_HEADS, HEAD_DIM)
        a = oracle.sigmoid_gate_mul(a, gate)
        return self.proj_chunk(p + "attn_output.weight", a, t)

    def prefill_chunk(self, token_ids, start, trace=None, rows=None):
        """Every layer over the chunk `token_ids` at positions start ..; returns
        the chunk's last hidden state [tokens][HIDDEN].  Appends, per layer,
        the hidden rows `rows` (default 0, tokens // 2, tokens - 1) to `trace`."""
        t = len(token_ids)
        rows = [0, t // 2, t - 1] if rows is None else rows
        h = self.embed(token_ids)
        for i in range(LAYERS):
            a = self.full_chunk(i, h, start, t) if full_attention(i) else self.linear_chunk(i, h, t)
            h = oracle.add(h, a)
            p = f"blk.{i}."
            n = oracle.rms_norm_batched(h, self.vec(p + "post_attention_norm.weight"), t, HIDDEN,
                                        EPS)
            up = self.proj_chunk(p + "ffn_up.weight", n, t)
            gate = self.proj_chunk(p + "ffn_gate.weight", n, t)
            h = oracle.add(h, self.proj_chunk(p + "ffn_down.weight", oracle.silu_mul(gate, up), t))
            if trace is not None:
                trace.append(h.reshape(t, HIDDEN)[rows].copy())
        return h.reshape(t, HIDDEN)

    def lm_head(self, last_row):
        """Output norm and LM head of one hidden row (fp32 GEMV): (argmax, logits)."""
        normed = self.norm(np.asarray(last_row, np.float32), "output_norm.weight")
        logits = self.proj("token_embd.weight", normed)
        return oracle.argmax(logits), logits

    def vec(self, name):
        return self.m[name][2]

    def norm(self, x, name):
        return oracle.rms_norm_batched(x, self.vec(name), 1, x.size, EPS)

    def linear(self, i, h):
        p = f"blk.{i}."
        n = self.norm(h, p + "attn_norm.weight")
        qkv, z = self.proj(p + "attn_qkv.weight", n), self.proj(p + "attn_gate.weight", n)
        beta, alpha = self.proj(p + "ssm_beta.weight", n), self.proj(p + "ssm_alpha.weight", n)
        ci, self.conv[i] = oracle.build_ssm_conv_state(self.conv[i], qkv, CONV_K, CONV_CH, 1)
        y = oracle.silu(oracle.ssm_conv(ci, self.vec(p + "ssm_conv1d.weight"), CONV_K, CONV_CH,
                                        1, 1))
        q, k, v = oracle.split_qkv_l2_norm(y, 1, HK, HV, DK, EPS)
        g, b = oracle.prepare_gdn_gate_beta(alpha, beta, self.vec(p + "ssm_dt.bias"),
                                            self.vec(p + "ssm_a"), 1, HV)
        o, self.state[i] = oracle.gated_delta_net(q, k, v, g, b, self.state[i], 1, HK, HV, DK)
        o = oracle.norm_gated(o, self.vec(p + "ssm_norm.weight"), z, 1, HV, DK, EPS)
        return self.proj(p + "ssm_out.weight", o)

    def full(self, i, h, pos):
        p = f"blk.{i}."
        n = self.norm(h, p + "attn_norm.weight")
        qg = self.proj(p + "attn_q.weight", n).reshape(HEADS, 2, HEAD_DIM)
        q, gate = qg[:, 0].ravel(), qg[:, 1].ravel()
        k, v = self.proj(p + "attn_k.weight", n), self.proj(p + "attn_v.weight", n)
        q = oracle.qk_norm_f32_batched(q, self.vec(p + "attn_q_norm.weight"), 1, HEADS,
                                       HEAD_DIM, EPS)
        k = oracle.qk_norm_f32_batched(k, self.vec(p + "attn_k_norm.weight"), 1, KV_HEADS,
                                       HEAD_DIM, EPS)
        positions = oracle.make_mrope_positions(pos, 1)
        q = oracle.mrope(q, positions, 1, HEADS, HEAD_DIM, ROPE_DIMS, SECTIONS, THETA)
        k = oracle.mrope(k, positions, 1, KV_HEADS, HEAD_DIM, ROPE_DIMS, SECTIONS, THETA)
        kv = KV_HEADS * HEAD_DIM
        self.kc[i][pos * kv:(pos + 1) * kv] = oracle.f32_to_f16_bits(k)
        self.vc[i][pos * kv:(pos + 1) * kv] = oracle.f32_to_f16_bits(v)
        a = oracle.attention_batched(q, self.kc[i], self.vc[i], 0, pos, 1, self.cap, HEADS,
                                     KV_HEADS, HEAD_DIM)
        a = oracle.sigmoid_gate_mul(a, gate)
        return self.proj(p + "attn_output.weight", a)

    def step(self, token, pos, trace=None):
        """Returns (argmax token, logits, LM-head input) for `token` at `pos`;
        appends each layer's output hidden state to `trace` when given."""
        (_, _), typ, emb = self.m["token_embd.weight"]
        row = HIDDEN // 256 * BLOCK[typ]
        h = oracle.kquant_dequantize(FMT[typ], emb[token * row:(token + 1) * row], HIDDEN // 256)
        for i in range(LAYERS):
            a = self.full(i, h, pos) if full_attention(i) else self.linear(i, h)
            h = oracle.add(h, a)
            p = f"blk.{i}."
            n = self.norm(h, p + "post_attention_norm.weight")
            up, gate = self.proj(p + "ffn_up.weight", n), self.proj(p + "ffn_gate.weight", n)
            h = oracle.add(h, self.proj(p + "ffn_down.weight", oracle.silu_mul(gate, up)))
            if trace is not None:
                trace.append(h.copy())
        normed = self.norm(h, "output_norm.weight")
        logits = self.proj("token_embd.weight", normed)
        return oracle.argmax(logits), logits, normed
