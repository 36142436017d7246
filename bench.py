"""Benchmark of the MI355X Qwen3.5 attention hot path (one GPU).

Headline (`value`): C1 decode attention -- one query token, 8 Q / 2 KV heads,
head_dim 256, F16 KV cache holding 4096 prior tokens plus the new one, output
gated by sigmoid(G) -- as algorithmic HBM GB/s:
    bytes/step = 2048 * (L + 1)  (K and V rows)  +  24 KiB (q, G, out) + 1 KiB
with the KV sets rotating over > 512 MB and 1 GiB of other data read between the
untimed and the timed replay, so every step reads from HBM, not the 256 MB
Infinity Cache ("cold"), whatever --steps is.  A step is one call of
kraken_hip_attention_f32_batched_f16_kv_gated.  The timed steps are captured in
one HIP graph on torch's stream and replayed between HIP events; inputs are
resident in HBM before the timed region starts.

`details` adds: decode at L = 1024/8192/16384 (cold and warm), flash256 prefill
(C2: T=1024 chunk after P = 0/3072/7168 prefix tokens, causal FLOP/s vs the
2.5 PFLOP/s dense fp16 MFMA peak), the GDN recurrence (C3: 1024-token chunk
prefill tok/s; single-token decode tok/s and GB/s cold over rotating state
sets) and the fused GDN layer core (conv prologue + gated recurrence), the C4 ragged block,
and the box's achievable rates (a 2 GiB copy and read, fp16 and fp32 GEMMs on the vendor BLAS)
with the hot-path results as fractions of them.

`cpu_baseline`: the CPU oracle's restatement of the same decode step
(oracle/kraken_oracle.c, one core), timed on a bounded sample.

Usage: python bench.py [--gpus 1] [--steps 1000] [--warmup 20] [--kv-len 4096]
"""
import argparse
import json
import os
import sys
import subprocess
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kraken-infer_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 (vector + MFMA)
MALL_BYTES = 256 << 20
HQ, HKV, D = 8, 2, 256
METRIC = "decode attn HBM GB/s & prefill TFLOP/s (% roofline), GDN tok/s, 1 GPU"


def progress(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_bytes(kv_len):
    return 2048 * (kv_len + 1) + 3 * HQ * D * 4 + 2 * HKV * D * 2


def prefill_flops(tokens, prefix):
    return 8192 * (tokens * prefix + tokens * (tokens + 1) // 2)


GDN_DECODE_BYTES = 2 * 16 * 128 * 128 * 4 + 3 * 16 * 128 * 4 + 2 * 16 * 4 + 16 * 128 * 4


class Runner:
    """Captures a list of step launches in one HIP graph and times replays."""

    def __init__(self, torch, ctx):
        self.torch = torch
        self.ctx = ctx
        self.flush_buf = None
        self.flush_sink = None
        self.stream = torch.cuda.Stream()
        ctx.set_stream(self.stream.cuda_stream)
        ctx.begin_graph()

    def time(self, steps, warmup, cold=False):
        """steps: list of zero-arg callables, each enqueueing one step.  Returns
        ms per step over one replay of the captured list.  cold: between the
        untimed and the timed replay, read 4x the Infinity Cache of other data,
        so the timed replay finds none of its inputs in any cache, whatever the
        number of steps."""
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for i in range(warmup):
                steps[i % len(steps)]()
            self.stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=self.stream):
                for s in steps:
                    s()
            graph.replay()  # untimed replay
            if cold:
                if self.flush_buf is None:
                    self.flush_buf = torch.ones(4 * MALL_BYTES // 4, device="cuda")
                self.flush_sink = self.flush_buf.sum()
            self.stream.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            start.record(self.stream)
            graph.replay()
            end.record(self.stream)
            end.synchronize()
            torch.cuda.synchronize()
        return start.elapsed_time(end) / len(steps), graph

    def close(self):
        self.ctx.commit_graph()
        self.ctx.set_stream(None)


def bench_decode(torch, ctx, run, kv_len, steps, warmup, cold, gen):
    """Returns dict with ms/step and GB/s for C1 decode at kv_len."""
    cap = kv_len + 1
    set_bytes = 2 * cap * HKV * D * 2
    n_sets = max(1, -(-2 * MALL_BYTES // set_bytes)) if cold else 1
    dev = "cuda"
    q = torch.randn(HQ * D, generator=gen, device=dev, dtype=torch.float32)
    g = torch.randn(HQ * D, generator=gen, device=dev, dtype=torch.float32)
    out = torch.empty(HQ * D, device=dev, dtype=torch.float32)
    ks = [torch.randn(cap * HKV * D, generator=gen, device=dev).half() for _ in range(n_sets)]
    vs = [torch.randn(cap * HKV * D, generator=gen, device=dev).half() for _ in range(n_sets)]

    def step(i):
        return lambda: ctx.attention_f32_batched_f16_kv_gated(
            q, ks[i % n_sets], vs[i % n_sets], g, 0, kv_len, 1, cap, HQ, HKV, D, out)

    ms, graph = run.time([step(i) for i in range(steps)], warmup, cold=cold)
    del graph
    gbs = decode_bytes(kv_len) / (ms * 1e-3) / 1e9
    res = {"kv_len": kv_len, "cold": cold, "kv_sets": n_sets, "ms_per_step": ms, "GB_s": gbs,
           "frac_hbm_peak": gbs / HBM_PEAK_GBS}
    del ks, vs
    torch.cuda.empty_cache()
    return res


def bench_prefill(torch, ctx, run, prefix, reps, warmup, gen):
    import kraken_hip as kh

    tokens = 1024
    cap = prefix + tokens
    dev = "cuda"
    q = torch.randn(tokens * HQ * D, generator=gen, device=dev)
    k = torch.randn(cap * HKV * D, generator=gen, device=dev)
    v = torch.randn(cap * HKV * D, generator=gen, device=dev)
    # C2 synthesis with the library's own ops: MRoPE (11,11,10,0; theta 1e7) then
    # L2 normalisation of q and k; q rounded to fp16 values, K/V stored fp16.
    pos_q = torch.arange(prefix, prefix + tokens, device=dev, dtype=torch.int32).repeat(4)
    pos_k = torch.arange(0, cap, device=dev, dtype=torch.int32).repeat(4)
    ctx.mrope_f32_in_place(q, pos_q, tokens, HQ, D, 64, 11, 11, 10, 0, 1e7)
    ctx.mrope_f32_in_place(k, pos_k, cap, HKV, D, 64, 11, 11, 10, 0, 1e7)
    ctx.l2_norm_f32_in_place(q, tokens * HQ, D, 1e-6)
    ctx.l2_norm_f32_in_place(k, cap * HKV, D, 1e-6)
    # C2's inputs are fp16: the f16-query entry reads them as they are.
    q16, kc, vc = q.half(), k.half(), v.half()
    out = torch.empty(tokens * HQ * D, device=dev)
    step = lambda: ctx.attention_f16q_batched_f16_kv(q16, kc, vc, 0, prefix, tokens, cap, HQ,
                                                     HKV, D, out)
    ms, graph = run.time([step] * reps, warmup)
    del graph
    flops = prefill_flops(tokens, prefix)
    tflops = flops / (ms * 1e-3) / 1e12
    return {"prefix": prefix, "tokens": tokens, "ms_per_chunk": ms, "TFLOP_s": tflops,
            "frac_fp16_mfma_peak": tflops / FP16_PEAK_TFLOPS, "tok_s": tokens / (ms * 1e-3),
            "gflop": flops / 1e9, "query": "f16 (kraken_hip_attention_f16q_batched_f16_kv)"}


def bench_gdn(torch, ctx, run, gen):
    hk = hv = 16
    d = 128
    dev = "cuda"
    res = {}

    def inputs(t):
        q = torch.nn.functional.normalize(torch.randn(t, hk, d, generator=gen, device=dev), dim=-1)
        k = torch.nn.functional.normalize(torch.randn(t, hk, d, generator=gen, device=dev), dim=-1)
        v = torch.randn(t, hv, d, generator=gen, device=dev)
        g = -torch.nn.functional.softplus(torch.randn(t, hv, generator=gen, device=dev))
        b = torch.sigmoid(torch.randn(t, hv, generator=gen, device=dev))
        return [x.contiguous() for x in (q, k, v, g, b)]

    # Prefill: 1024-token chunks through the recurrence.
    t = 1024
    q, k, v, g, b = inputs(t)
    state = torch.zeros(hv * d * d, device=dev)
    out = torch.empty(t * hv * d, device=dev)
    step = lambda: ctx.gated_delta_net_f32_batched_in_place_at(q, k, v, g, b, state, 0, t, hk,
                                                               hv, d, out)
    ms, graph = run.time([step] * 4, 1)
    del graph
    gflops = 1.835e6 * t / (ms * 1e-3) / 1e9
    res["prefill"] = {"tokens_per_chunk": t, "ms_per_chunk": ms, "tok_s": t / (ms * 1e-3),
                      "gflop_s_recurrent_equiv": gflops,
                      "frac_fp32_peak": gflops / (FP32_PEAK_TFLOPS * 1e3),
                      "arithmetic": "split-fp16 MFMA: each f32 operand as an f16 hi/lo pair, "
                                    "three f16 products accumulated in f32"}

    # Decode: one token per step, cold over rotating state sets (>512 MB).
    sets = 512
    q1, k1, v1, g1, b1 = inputs(1)
    states = torch.zeros(sets, hv * d * d, device=dev)
    out1 = torch.empty(hv * d, device=dev)

    def dstep(i):
        return lambda: ctx.gated_delta_net_f32_batched_in_place_at(
            q1, k1, v1, g1, b1, states[i % sets], 0, 1, hk, hv, d, out1)

    ms, graph = run.time([dstep(i) for i in range(1024)], 16, cold=True)
    del graph
    gbs = GDN_DECODE_BYTES / (ms * 1e-3) / 1e9
    res["decode"] = {"ms_per_token_layer": ms, "tok_s": 1 / (ms * 1e-3), "GB_s": gbs,
                     "frac_hbm_peak": gbs / HBM_PEAK_GBS, "state_sets": sets, "cold": True}
    del states

    # Fused layer core per decode token: conv/split/L2 prologue + gated recurrence
    # with norm-gated epilogue (4 kernels), cold over the same state sets.
    channels = (2 * hk + hv) * d
    qkv = torch.randn(channels, generator=gen, device=dev)
    w = 0.5 * torch.randn(channels * 4, generator=gen, device=dev)
    conv_states = torch.zeros(sets, channels * 3, device=dev)
    states = torch.zeros(sets, hv * d * d, device=dev)
    alpha = torch.randn(hv, generator=gen, device=dev)
    beta = torch.randn(hv, generator=gen, device=dev)
    dtb = torch.randn(hv, generator=gen, device=dev)
    ssa = -torch.rand(hv, generator=gen, device=dev)
    z = torch.randn(hv * d, generator=gen, device=dev)
    nw = torch.ones(d, device=dev)
    qb, kb, vb = (torch.empty(hk * d, device=dev), torch.empty(hk * d, device=dev),
                  torch.empty(hv * d, device=dev))

    def lstep(i):
        def f():
            ctx.qwen35_conv_split_l2_f32(qkv, conv_states[i % sets], 0, w, 4, 1, hk, hv, d, 1e-6,
                                         qb, kb, vb)
            ctx.qwen35_gdn_gated_f32(qb, kb, vb, alpha, beta, dtb, ssa, z, nw, states[i % sets],
                                     0, 1, hk, hv, d, 1e-6, out1)
        return f

    ms, graph = run.time([lstep(i) for i in range(512)], 8, cold=True)
    del graph
    res["decode_layer_core_fused"] = {"ms_per_token_layer": ms, "tok_s": 1 / (ms * 1e-3)}

    # The same layer (conv prologue, gate/beta prepare, recurrence, norm-gated epilogue) in
    # one kernel: the ragged GDN-layer entry with a single sequence, cold over the state sets.
    conv_offs = [torch.tensor([i * channels * 3], device=dev, dtype=torch.int64)
                 for i in range(sets)]
    state_offs = [torch.tensor([i * hv * d * d], device=dev, dtype=torch.int64)
                  for i in range(sets)]

    def ostep(i):
        def f():
            ctx.qwen35_gdn_layer_ragged_decode_f32(qkv, conv_states, conv_offs[i % sets], w, 4,
                                                   alpha, beta, dtb, ssa, z, nw, states,
                                                   state_offs[i % sets], 1, hk, hv, d, 1e-6,
                                                   out1)
        return f

    ms, graph = run.time([ostep(i) for i in range(512)], 8, cold=True)
    del graph
    res["decode_layer_one_kernel"] = {"ms_per_token_layer": ms, "tok_s": 1 / (ms * 1e-3),
                                      "GB_s": GDN_DECODE_BYTES / (ms * 1e-3) / 1e9}
    del states, conv_states
    torch.cuda.empty_cache()
    return res


def mt19937_64(seed):
    """64-bit Mersenne Twister (Matsumoto & Nishimura, 2004), std::mt19937_64."""
    mask = (1 << 64) - 1
    n, m = 312, 156
    mt = [seed & mask] + [0] * (n - 1)
    for i in range(1, n):
        mt[i] = (6364136223846793005 * (mt[i - 1] ^ (mt[i - 1] >> 62)) + i) & mask
    idx = n
    while True:
        if idx >= n:
            for i in range(n):
                x = (mt[i] & 0xFFFFFFFF80000000) | (mt[(i + 1) % n] & 0x7FFFFFFF)
                xa = x >> 1
                if x & 1:
                    xa ^= 0xB5026F5AA96619E9
                mt[i] = mt[(i + m) % n] ^ xa
            idx = 0
        y = mt[idx]
        idx += 1
        y ^= (y >> 29) & 0x5555555555555555
        y ^= (y << 17) & 0x71D67FFFEDA60000
        y ^= (y << 37) & 0xFFF7EEE000000000
        y ^= y >> 43
        yield y & mask


C4_SEQUENCES = 64
C4_GDN_LAYERS = 3


def c4_lengths():
    """KV lengths L_i in [512, 32768]: 512 + (mt19937_64(seed 4) output mod 32257)."""
    g = mt19937_64(4)
    return [512 + next(g) % 32257 for _ in range(C4_SEQUENCES)]


def bench_c4(torch, ctx, run, gen, steps=20):
    """C4: 64 sequences, one token each per step, each running one hybrid block of
    3 GDN layers (conv prologue, recurrence and norm-gated epilogue, one launch
    per layer) and one full-attention layer (KV append + gated attention)
    through the ragged multi-sequence entry points."""
    dev = "cuda"
    b = C4_SEQUENCES
    hk = hv = 16
    dg = 128
    ch = (2 * hk + hv) * dg
    kv_dim = HKV * D
    lengths = c4_lengths()
    # Sequence i owns rows [0, L_i + 1) of its K/V (the new token at row L_i).
    rows = [l + 1 for l in lengths]
    kv_off, cur = [], 0
    for r in rows:
        kv_off.append(cur)
        cur += r * kv_dim
    kpool = torch.randn(cur, generator=gen, device=dev).half()
    vpool = torch.randn(cur, generator=gen, device=dev).half()
    kv_off_t = torch.tensor(kv_off, dtype=torch.int64, device=dev)
    pos_t = torch.tensor(lengths, dtype=torch.int32, device=dev)
    state_elems = hv * dg * dg
    state_pool = torch.zeros(C4_GDN_LAYERS * b * state_elems, device=dev)
    conv_pool = torch.zeros(C4_GDN_LAYERS * b * ch * 3, device=dev)
    state_off = [torch.arange(b, device=dev, dtype=torch.int64) * state_elems
                 + l * b * state_elems for l in range(C4_GDN_LAYERS)]
    conv_off = [torch.arange(b, device=dev, dtype=torch.int64) * ch * 3 + l * b * ch * 3
                for l in range(C4_GDN_LAYERS)]
    qkv = [torch.randn(b * ch, generator=gen, device=dev) for _ in range(C4_GDN_LAYERS)]
    w = [0.5 * torch.randn(ch * 4, generator=gen, device=dev) for _ in range(C4_GDN_LAYERS)]
    g = [-torch.nn.functional.softplus(torch.randn(b * hv, generator=gen, device=dev))
         for _ in range(C4_GDN_LAYERS)]
    beta = [torch.sigmoid(torch.randn(b * hv, generator=gen, device=dev))
            for _ in range(C4_GDN_LAYERS)]
    z = [torch.randn(b * hv * dg, generator=gen, device=dev) for _ in range(C4_GDN_LAYERS)]
    norm_w = torch.ones(dg, device=dev)
    q = torch.empty(b * hk * dg, device=dev)
    k = torch.empty(b * hk * dg, device=dev)
    v = torch.empty(b * hv * dg, device=dev)
    y = torch.empty(b * hv * dg, device=dev)
    knew = torch.randn(b * kv_dim, generator=gen, device=dev)
    vnew = torch.randn(b * kv_dim, generator=gen, device=dev)
    aq = torch.randn(b * HQ * D, generator=gen, device=dev)
    agate = torch.randn(b * HQ * D, generator=gen, device=dev)
    aout = torch.empty(b * HQ * D, device=dev)
    maxpos = max(lengths)

    def gdn_layer(l, core_only=False):
        if core_only:
            ctx.gated_delta_net_f32_ragged_decode(q, k, v, g[l], beta[l], state_pool,
                                                  state_off[l], b, hk, hv, dg, y)
        else:
            # Conv prologue, recurrence and norm-gated epilogue in one launch.
            ctx.qwen35_gdn_layer_ragged_decode_f32(qkv[l], conv_pool, conv_off[l], w[l], 4, g[l],
                                                   beta[l], None, None, z[l], norm_w, state_pool,
                                                   state_off[l], b, hk, hv, dg, 1e-6, y)

    def attention_layer(append=True):
        if append:
            ctx.append_kv_ragged_f16(knew, vnew, kpool, vpool, kv_off_t, pos_t, b, kv_dim)
        ctx.attention_f32_ragged_f16_kv(aq, kpool, vpool, agate, kv_off_t, pos_t, b, maxpos, HQ,
                                        HKV, D, aout)

    def block():
        for l in range(C4_GDN_LAYERS):
            gdn_layer(l)
        attention_layer()

    # q/k/v inputs of the core-only timing: one conv prologue.
    ctx.qwen35_conv_split_l2_ragged_decode_f32(qkv[0], conv_pool, conv_off[0], w[0], 4, b, hk, hv,
                                               dg, 1e-6, q, k, v)
    kv_bytes = sum(2048 * r for r in rows)
    gdn_bytes = b * C4_GDN_LAYERS * GDN_DECODE_BYTES
    res = {"sequences": b, "kv_len_min": min(lengths), "kv_len_max": maxpos,
           "kv_len_mean": sum(lengths) / b, "kv_bytes_per_step": kv_bytes,
           "gdn_core_bytes_per_step": gdn_bytes,
           "lengths": "512 + mt19937_64(seed 4) mod 32257"}
    ms, graph = run.time([block] * steps, 2)
    del graph
    res["block"] = {"ms_per_step": ms, "tok_s": b / (ms * 1e-3),
                    "kv_GB_s": kv_bytes / (ms * 1e-3) / 1e9,
                    "GB_s": (kv_bytes + gdn_bytes) / (ms * 1e-3) / 1e9,
                    "frac_hbm_peak": (kv_bytes + gdn_bytes) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    ms, graph = run.time([lambda: attention_layer(False)] * steps, 2)
    del graph
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    res["attention"] = {"ms_per_step": ms, "GB_s": gbs, "frac_hbm_peak": gbs / HBM_PEAK_GBS}
    ms, graph = run.time([lambda: [gdn_layer(l, True) for l in range(C4_GDN_LAYERS)]] * steps, 2)
    del graph
    gbs = gdn_bytes / (ms * 1e-3) / 1e9
    res["gdn_core"] = {"ms_per_step": ms, "GB_s": gbs, "frac_hbm_peak": gbs / HBM_PEAK_GBS,
                       "tok_s": b * C4_GDN_LAYERS / (ms * 1e-3)}
    del kpool, vpool, state_pool, conv_pool
    torch.cuda.empty_cache()
    return res


def cpu_baseline(kv_len, budget_s):
    """Times the oracle's decode step (one core) on a bounded sample."""
    import numpy as np

    import oracle

    cap = kv_len + 1
    rng = np.random.default_rng(1)
    q = rng.standard_normal(HQ * D).astype(np.float32)
    kc = rng.standard_normal(cap * HKV * D).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(cap * HKV * D).astype(np.float16).view(np.uint16)
    gate = rng.standard_normal(HQ * D).astype(np.float32)
    oracle.lib()
    n = 0
    t0 = time.perf_counter()
    while True:
        out = oracle.attention_batched(q, kc, vc, 0, kv_len, 1, cap, HQ, HKV, D)
        oracle.sigmoid_gate_mul(out, gate)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 2000:
            break
    s_per_step = el / n
    return {"value": decode_bytes(kv_len) / s_per_step / 1e9, "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"{n} C1 decode steps at L={kv_len} (oracle_attention_batched + gate, "
                      f"double accumulation, one thread), {el:.1f} s; "
                      f"{s_per_step * 1e3:.2f} ms/step",
            "ms_per_step": s_per_step * 1e3,
            "host_threads_available": os.cpu_count()}


def host_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "cpu_count": os.cpu_count(),
            "affinity": len(os.sched_getaffinity(0))}


def cpu_baselines(budget_s):
    """The CPU oracle (oracle/kraken_oracle.c, -O3, one thread, called through ctypes) on a
    bounded sample of each configuration, about `budget_s` seconds each.  Scaled figures say
    so in their names."""
    import numpy as np

    import oracle

    oracle.lib()
    rng = np.random.default_rng(0)

    def timed(fn):
        n, t0 = 0, time.perf_counter()
        while True:
            fn(n)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                return el / n, n

    res = {"host": host_info(), "threads": 1}
    # C0: legacy attention decode steps (16 Q / 8 KV heads, head_dim 128, F32 KV) at the
    # positions of the 64 decode steps after a 512-token prefill.
    cap = 576
    kc0 = rng.standard_normal(cap * 8 * 128).astype(np.float32)
    vc0 = rng.standard_normal(cap * 8 * 128).astype(np.float32)
    q0 = rng.standard_normal(16 * 128).astype(np.float32)
    sec, n = timed(lambda i: oracle.qwen3_attention(kc0, vc0, cap, 0, 512 + i % 64, q0, 16, 8,
                                                    128))
    res["c0_decode"] = {"ms_per_step": sec * 1e3, "steps_sampled": n,
                        "sample": "oracle_qwen3_attention at positions 512..575"}
    # C2: flash256 prefill at P=7168, sampled query tokens of the chunk.
    p, t = 7168, 1024
    cap2 = p + t
    kc2 = rng.standard_normal(cap2 * HKV * D).astype(np.float16).view(np.uint16)
    vc2 = rng.standard_normal(cap2 * HKV * D).astype(np.float16).view(np.uint16)
    q2 = rng.standard_normal(HQ * D).astype(np.float32)
    toks = [0, 255, 511, 767, 1023]
    sec, n = timed(lambda i: oracle.attention_batched(q2, kc2, vc2, 0, p + toks[i % 5], 1, cap2,
                                                      HQ, HKV, D, round_query_f16=True))
    mean_keys = p + sum(toks) / len(toks) + 1
    res["c2_prefill_p7168"] = {
        "TFLOP_s": 8192 * mean_keys / sec / 1e12, "ms_per_token": sec * 1e3,
        "ms_per_chunk_scaled": sec * 1e3 * t, "tokens_sampled": n,
        "sample": "oracle_attention_batched, one query token at a time (tokens 0, 255, 511, "
                  "767, 1023 of the chunk)"}
    # C3: GDN recurrence, 16 heads, head_dim 128: a 64-token prefill and single-token decode.
    hk = hv = 16
    dk = 128
    state = np.zeros(hv * dk * dk, np.float32)
    qg = rng.standard_normal(64 * hk * dk).astype(np.float32)
    gg = -np.log1p(np.exp(rng.standard_normal(64 * hv))).astype(np.float32)
    bb = (1 / (1 + np.exp(-rng.standard_normal(64 * hv)))).astype(np.float32)
    sec, n = timed(lambda i: oracle.gated_delta_net(qg, qg, qg, gg, bb, state, 64, hk, hv, dk))
    res["c3_prefill"] = {"tok_s": 64 / sec, "ms_per_64_tokens": sec * 1e3, "calls": n}
    sec1, n1 = timed(lambda i: oracle.gated_delta_net(qg, qg, qg, gg, bb, state, 1, hk, hv, dk))
    res["c3_decode"] = {"tok_s": 1 / sec1, "ms_per_token": sec1 * 1e3, "calls": n1}
    # C4: one sequence's block step (attention decode at the mean K/V length 16872, plus three
    # GDN decode steps), scaled to 64 sequences on one thread.
    l4 = 16872
    kc4 = rng.standard_normal((l4 + 1) * HKV * D).astype(np.float16).view(np.uint16)
    vc4 = rng.standard_normal((l4 + 1) * HKV * D).astype(np.float16).view(np.uint16)

    def c4_step(i):
        oracle.attention_batched(q2, kc4, vc4, 0, l4, 1, l4 + 1, HQ, HKV, D)
        for _ in range(3):
            oracle.gated_delta_net(qg, qg, qg, gg, bb, state, 1, hk, hv, dk)

    sec4, n4 = timed(c4_step)
    res["c4_block"] = {"ms_per_sequence_step": sec4 * 1e3,
                       "tok_s_64_sequences_scaled": 1 / sec4,
                       "sequence_steps_sampled": n4,
                       "sample": "one sequence at the mean K/V length 16872: attention decode "
                                 "+ 3 GDN decode steps; 64 sequences on one thread take 64x"}
    return res


def decode_traffic():
    """HBM bytes per C1 (L=4096) decode step from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE of both dispatches, scaled by the plain-copy
    calibration), or None when it is absent."""
    path = os.path.join(ROOT, "profiles", "decode_attention_c1_l4096_counters.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("hbm_bytes_per_step:"):
                return int(line.split(":", 1)[1].strip())
    return None


MODEL_BENCH = os.path.join(ROOT, "kraken-infer_amd", "build", "qwen35_model_bench")


def model_bench(*args, timeout=300):
    """Runs kraken-infer_amd/build/qwen35_model_bench (whole-model timings on synthetic
    Qwen3.5-0.8B weights) in its own process and returns its key=value fields."""
    if not os.path.exists(MODEL_BENCH):
        raise RuntimeError(f"{MODEL_BENCH} is not built (run __graft_entry__.build())")
    out = subprocess.run([MODEL_BENCH, *map(str, args)], capture_output=True, text=True,
                         timeout=timeout)
    if out.returncode != 0:
        raise RuntimeError(f"qwen35_model_bench {args[0]} failed: " + out.stdout + out.stderr)
    line = [l for l in out.stdout.splitlines() if l.startswith(str(args[0]) + " ")][-1]
    return {k: float(v) for k, v in (kv.split("=") for kv in line.split()[1:])}


def bench_prefix():
    """Prompt prefix cache store (include/kraken/qwen35_prefix_store.hpp): commit and
    restore of 1024-token blocks of the Qwen3.5-0.8B cache."""
    vals = model_bench("prefix-store", timeout=120)
    vals["note"] = ("8 blocks of 1024 tokens: K/V rows of 6 layers, R/S of 18 layers, last "
                    "hidden row; restore = all 8 blocks' K/V rows + R/S once; payloads live in one "
                    "HBM arena allocated at the first (untimed) commit")
    return vals


KQUANT_SHAPES = [("q5_k", 6144, 1024), ("q4_k", 3584, 1024), ("q6_k", 1024, 3584),
                 ("q4_k", 1024, 2048)]
KQUANT_BLOCK = {"q4_k": 144, "q5_k": 176, "q6_k": 210}
MFMA_F16_PEAK_TFLOPS = 2500.0


def kquant_weight(torch, fmt, rows, cols, gen):
    """Random K-quant blocks with small positive f16 scales (every other byte
    pattern is a valid block), as a uint8 device tensor."""
    nb = KQUANT_BLOCK[fmt]
    blocks = rows * cols // 256
    w = torch.randint(0, 256, (blocks, nb), generator=gen, device="cuda", dtype=torch.uint8)
    d = (torch.rand(blocks, generator=gen, device="cuda") * 0.02 + 0.001).half()
    at = 208 if fmt == "q6_k" else 0
    w[:, at:at + 2] = d.view(torch.uint8).view(blocks, 2)
    if fmt != "q6_k":
        w[:, 2:4] = d.view(torch.uint8).view(blocks, 2)
    return w.reshape(-1)


def bench_kquant(torch, ctx, run, gen, shapes=(0, 1, 2, 3)):
    """The Qwen3.5-0.8B K-quant projections: one-token GEMV (weights read
    once; sets rotated over 2x the Infinity Cache so every replay reads HBM)
    and 1024-token GEMM (dequantize to fp16 + MFMA GEMM), as graph replays.
    GEMV bytes = quantized weight + f32 input + f32 output; GEMM flops =
    2 * rows * cols * tokens over the whole call (its three launches)."""
    out = []
    for fmt, rows, cols in (KQUANT_SHAPES[i] for i in shapes):
        wbytes = rows * cols // 256 * KQUANT_BLOCK[fmt]
        sets = max(1, -(-2 * MALL_BYTES // wbytes))
        ws = [kquant_weight(torch, fmt, rows, cols, gen) for _ in range(sets)]
        x = torch.randn(1024 * cols, generator=gen, device="cuda")
        y = torch.empty(1024 * rows, device="cuda")
        mv = getattr(ctx, f"matvec_{fmt}_f32_device")
        mm = getattr(ctx, f"matmul_{fmt}_f32_device")
        gemv_steps = [lambda i=i: mv(ws[i % sets], rows, cols, x, y) for i in range(2 * sets)]
        ms_gemv, graph = run.time(gemv_steps, 4, cold=True)
        del graph
        gemv_bytes = wbytes + 4 * cols + 4 * rows
        gemv_gbs = gemv_bytes / (ms_gemv * 1e-3) / 1e9
        ms_gemm, graph = run.time([lambda: mm(ws[0], rows, cols, 1024, x, y)] * 10, 2)
        del graph
        tflops = 2.0 * rows * cols * 1024 / (ms_gemm * 1e-3) / 1e12
        out.append({"format": fmt, "rows": rows, "cols": cols,
                    "gemv_us": ms_gemv * 1e3, "gemv_bytes": gemv_bytes, "gemv_GB_s": gemv_gbs,
                    "gemv_frac_hbm": gemv_gbs / HBM_PEAK_GBS, "gemv_weight_sets": sets,
                    "gemm_tokens": 1024, "gemm_us": ms_gemm * 1e3, "gemm_TFLOP_s": tflops,
                    "gemm_frac_mfma_f16": tflops / MFMA_F16_PEAK_TFLOPS})
        del ws
    return out


def bench_decode_loop(warmup=8, steps=64):
    """Greedy decode of the whole 0.8B model (synthetic K-quant weights: every
    layer's norms, projections, attention core and FFN, the tied Q6_K LM head
    with device argmax), one graph batch and one host wait per token
    (include/kraken/qwen35_decode.hpp).  weight_GB_s counts every weight byte
    read once per token."""
    res = model_bench("decode", warmup, steps)
    res["frac_hbm_peak"] = res["weight_GB_s"] / HBM_PEAK_GBS
    res["note"] = ("synthetic Qwen3.5-0.8B shapes: Q6_K token_embd/LM head 248320x1024, per layer "
                   "Q4_K/Q5_K/Q6_K projections and FFN 3584; tokens fed back greedily")
    return res


def bench_prefill_model(prompt=4096, chunk=1024):
    """Chunked prefill of the whole 0.8B model (include/kraken/qwen35_prefill.hpp):
    every layer over each 1024-token chunk (RMSNorm, K-quant GEMM projections,
    flash256 or the chunked gated delta rule, output projection, SwiGLU FFN), one
    graph batch and one host wait per chunk, then the greedy LM head of the last
    row; host clock over the whole prompt."""
    res = model_bench("prefill", prompt, chunk)
    res["note"] = ("synthetic Qwen3.5-0.8B weights; prompt of %d tokens in chunks of %d, "
                   "timed on the second pass" % (prompt, chunk))
    return res


def bench_peaks(torch, ctx, run):
    """Achievable rates on this box, next to the published peaks.  The library's probes
    (include/kraken_hip_diag.h): a nontemporal streaming read of 2 GiB and an fp16 MFMA loop
    (one wave per SIMD, four independent v_mfma_f32_32x32x16_f16 chains), both timed as graph
    replays like the hot-path kernels.  For comparison, the same box through torch: a 2 GiB
    copy and sum, and dense fp16 / fp32 GEMMs on the vendor BLAS.  The roofline fractions in the
    JSON line stay against the published peaks."""
    def timed(fn, reps=10, warm=3):
        for _ in range(warm):
            fn()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3  # seconds per call

    n = 1 << 29  # floats: 2 GiB
    src = torch.ones(n, device="cuda")
    sink = torch.empty(1 << 20, device="cuda")
    ms_probe_read, graph = run.time([lambda: ctx.diag_stream_read(src, 4 * n, sink)] * 10, 2)
    del graph
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    iters = 4000
    ms_probe_mfma, graph = run.time([lambda: ctx.diag_mfma_f16(cus, iters, sink)] * 5, 1)
    del graph
    mfma_flops = cus * 4 * iters * 8 * 32768
    dst = torch.empty_like(src)
    t_copy = timed(lambda: dst.copy_(src))
    t_read = timed(lambda: src.sum())
    del src, dst, sink
    m = 8192
    a = torch.randn(m, m, device="cuda", dtype=torch.float16)
    b = torch.randn(m, m, device="cuda", dtype=torch.float16)
    t_h = timed(lambda: torch.matmul(a, b))
    del a, b
    m32 = 4096
    a = torch.randn(m32, m32, device="cuda")
    b = torch.randn(m32, m32, device="cuda")
    t_f = timed(lambda: torch.matmul(a, b))
    del a, b
    return {"probe_read_GB_s": 4 * n / (ms_probe_read * 1e-3) / 1e9,
            "probe_mfma_f16_TFLOP_s": mfma_flops / (ms_probe_mfma * 1e-3) / 1e12,
            "torch_copy_GB_s": 2 * 4 * n / t_copy / 1e9, "torch_read_GB_s": 4 * n / t_read / 1e9,
            "fp16_gemm_TFLOP_s": 2 * m ** 3 / t_h / 1e12,
            "fp32_gemm_TFLOP_s": 2 * m32 ** 3 / t_f / 1e12,
            "note": "probes: kraken_hip_diag_stream_read over 2 GiB, kraken_hip_diag_mfma_f16 "
                    f"({cus} workgroups x {iters} iterations); torch: 2 GiB copy_ (read + "
                    "write bytes) and sum (read bytes), matmul 8192^3 fp16 and 4096^3 fp32"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kv-len", type=int, default=4096)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--quick", action="store_true", help="headline only, no details")
    ap.add_argument("--sections",
                    default="decode,prefill,gdn,c4,kquant,peaks,prefix,loop,model_prefill",
                    help="comma-separated detail sections to run after the headline "
                         "(decode, prefill, gdn, c4, kquant, peaks, prefix, loop, model_prefill)")
    ap.add_argument("--prefill-prefixes", default="0,3072,7168",
                    help="comma-separated KV prefixes of the prefill section")
    ap.add_argument("--kquant-shapes", default="0,1,2,3",
                    help="comma-separated indices into KQUANT_SHAPES for the kquant section")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run torch copies of MIB MiB (20 launches), the known-size "
                         "reference for rocprofv3 FETCH_SIZE / WRITE_SIZE scaling")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path)", file=sys.stderr)
        sys.exit(2)

    import torch

    import kraken_hip as kh

    torch.cuda.init()
    if args.copy_calibration:
        n = args.copy_calibration << 18  # floats
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        progress(f"copy calibration: 20 x {args.copy_calibration} MiB read + written")
        return
    ctx = kh.Context()
    run = Runner(torch, ctx)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1)

    # Input generation and our launches share one stream, so they stay ordered.
    with torch.cuda.stream(run.stream):
        head = bench_decode(torch, ctx, run, args.kv_len, args.steps, args.warmup, True, gen)
        progress(f"decode L={args.kv_len} cold: {head['GB_s']:.0f} GB/s")
        details = {"decode_c1": [head]}
        sections = set() if args.quick else set(args.sections.split(","))
        if "decode" in sections:
            for kv in (1024, 8192, 16384):
                details["decode_c1"].append(bench_decode(torch, ctx, run, kv, 400, 10, True, gen))
            for kv in (1024, 4096, 16384):
                details["decode_c1"].append(bench_decode(torch, ctx, run, kv, 400, 10, False,
                                                         gen))
            progress("decode details done")
        if "prefill" in sections:
            gen.manual_seed(2)
            details["prefill_c2"] = [bench_prefill(torch, ctx, run, int(p), 10, 2, gen)
                                     for p in args.prefill_prefixes.split(",")]
            progress("prefill done")
        if "gdn" in sections:
            gen.manual_seed(3)
            details["gdn_c3"] = bench_gdn(torch, ctx, run, gen)
            progress("gdn done")
        if "c4" in sections:
            gen.manual_seed(4)
            details["ragged_c4"] = bench_c4(torch, ctx, run, gen)
            progress("ragged c4 done")
        if "kquant" in sections:
            gen.manual_seed(5)
            details["kquant"] = bench_kquant(torch, ctx, run, gen,
                                             [int(i) for i in args.kquant_shapes.split(",")])
            progress("kquant: " + ", ".join(
                f"{k['format']} {k['rows']}x{k['cols']} GEMV {k['gemv_GB_s']:.0f} GB/s "
                f"GEMM {k['gemm_TFLOP_s']:.0f} TFLOP/s" for k in details["kquant"]))
        if "peaks" in sections:
            peaks = bench_peaks(torch, ctx, run)
            details["achievable_peaks"] = peaks
            # The hot-path results as fractions of what this box reaches.
            vs = {"decode_c1_vs_probe_read": head["GB_s"] / peaks["probe_read_GB_s"]}
            if "ragged_c4" in details:
                vs["c4_attention_vs_probe_read"] = (details["ragged_c4"]["attention"]["GB_s"] /
                                                    peaks["probe_read_GB_s"])
            if "prefill_c2" in details:
                vs["prefill_c2_vs_probe_mfma"] = [x["TFLOP_s"] / peaks["probe_mfma_f16_TFLOP_s"]
                                                  for x in details["prefill_c2"]]
            details["vs_achievable"] = vs
            progress(f"peaks: probe read {peaks['probe_read_GB_s']:.0f} GB/s, probe MFMA "
                     f"{peaks['probe_mfma_f16_TFLOP_s']:.0f} TFLOP/s")
    run.close()
    ctx.close()
    if "loop" in sections:
        details["decode_loop"] = bench_decode_loop()
        progress(f"decode loop: {details['decode_loop']['ms_per_token']:.3f} ms/token")
    if "model_prefill" in sections:
        details["model_prefill"] = bench_prefill_model()
        progress(f"model prefill: {details['model_prefill']['tok_s']:.0f} tok/s")
    if "prefix" in sections:
        details["prefix_store"] = bench_prefix()
        progress(f"prefix store: restore {details['prefix_store']['restore_GB_s']:.0f} GB/s")

    cpu = None if args.no_cpu else cpu_baseline(args.kv_len, args.cpu_seconds)
    if not args.no_cpu and not args.quick:
        details["cpu_baselines"] = cpu_baselines(2.0)
    progress("cpu baseline done")
    traffic = decode_traffic() if args.kv_len == 4096 else None
    line = {
        "metric": METRIC,
        "value": head["GB_s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 KV, f32 accumulate",
        "data": "synthetic (seeded N(0,1), torch generator seed 1)",
        "config": {"workload": f"C1 decode attention: 1 query token, 8 Q / 2 KV heads, "
                               f"head_dim 256, F16 KV cache of {args.kv_len} prior tokens, "
                               "sigmoid output gate fused; KV sets rotated over >512 MB (cold)",
                   "kv_len": args.kv_len, "heads": HQ, "kv_heads": HKV, "head_dim": D,
                   "batch": 1, "kv_sets": head["kv_sets"],
                   "bytes_per_step": decode_bytes(args.kv_len)},
        "roofline": {"bound": "hbm", "achieved": head["GB_s"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": head["GB_s"] / HBM_PEAK_GBS, "traffic": traffic,
                     "kernels": "attention_decode_short_kernel<4> + attention_merge "
                                "(the two dispatches of one decode step, timed together)"},
        "cpu_baseline": cpu,
        "details": details,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
