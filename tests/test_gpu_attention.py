"""GPU parity of the attention kernels against the CPU oracle.

Tolerance: fp16-KV outputs within 2e-3 relative /
1e-3 absolute of the oracle; f32-KV outputs within 1e-4.  Inputs are seeded
numpy draws (np.random.default_rng(seed)).

Cases:
  * split-K decode (T=1) at C1's shape (8 Q / 2 KV heads, D=256) for several KV
    lengths, unsplit and split, with and without the fused sigmoid gate;
  * short chunks (T<64) with causal masking, GQA group sizes 1/2/4/8,
    head_dim 64/128/256 and a generic (untuned) head_dim;
  * flash256 prefill vs the oracle (Q rounded to f16 as the reference does),
    aligned and unaligned token counts, with a KV prefix, plus C2's full shape
    through sampled tokens and through agreement with the decode kernel;
  * the reference smoke test's 64- and 65-token modular-pattern cases.
"""
import numpy as np
import pytest

import kraken_hip as kh
import oracle

RTOL, ATOL = 2e-3, 1e-3


def f16_bits(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def make_case(seed, tokens, start, cap, heads, kv_heads, d, layers=1, layer=0, scale_kv=1.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(tokens * heads * d).astype(np.float32)
    k = (rng.standard_normal(layers * cap * kv_heads * d) * scale_kv).astype(np.float32)
    v = rng.standard_normal(layers * cap * kv_heads * d).astype(np.float32)
    return q, f16_bits(k), f16_bits(v)


def run_hip(ctx, q, kc, vc, layer, start, tokens, cap, heads, kv_heads, d, gate=None):
    return kh.NumpyOps(ctx).attention_batched(q, kc, vc, layer, start, tokens, cap, heads,
                                              kv_heads, d, gate=gate)


def close(got, ref, rtol=RTOL, atol=ATOL, msg=""):
    np.testing.assert_allclose(got, ref, rtol=rtol, atol=atol, err_msg=msg)


@pytest.mark.gpu
@pytest.mark.parametrize("kv_len", [0, 31, 1024, 4096, 16384])
def test_decode_c1_shape(hip_ctx, kv_len):
    heads, kv_heads, d = 8, 2, 256
    cap = kv_len + 1
    print(f"decode C1 L={kv_len}", flush=True)
    q, kc, vc = make_case(1, 1, kv_len, cap, heads, kv_heads, d)
    got = run_hip(hip_ctx, q, kc, vc, 0, kv_len, 1, cap, heads, kv_heads, d)
    ref = oracle.attention_batched(q, kc, vc, 0, kv_len, 1, cap, heads, kv_heads, d)
    close(got, ref, msg=f"L={kv_len}")


@pytest.mark.gpu
@pytest.mark.parametrize("kernel", ["short", "mfma"])
@pytest.mark.parametrize("q_scale,atol", [(1.0, 4e-6), (8.0, 2e-5)])
def test_decode_keeps_f32_query_precision(hip_ctx, monkeypatch, kernel, q_scale, atol):
    """C1 at L=4096: the MFMA decode kernels hold the f32 query (and the f32
    probabilities) in the split fp16 form with lo scaled by 2^11, so their result
    stays within `atol` of the oracle's f32-query attention (mps_backend.mm:
    2979-2983 multiplies an f32 query).  The same attention on an f16-rounded
    query misses by more than twice `atol`, so this tolerance tells the two apart
    where the default 2e-3 / 1e-3 does not."""
    heads, kv_heads, d, kv_len = 8, 2, 256, 4096
    cap = kv_len + 1
    print(f"decode f32 query {kernel} q_scale={q_scale}", flush=True)
    q, kc, vc = make_case(1, 1, kv_len, cap, heads, kv_heads, d)
    q = (q * q_scale).astype(np.float32)
    ref = oracle.attention_batched(q, kc, vc, 0, kv_len, 1, cap, heads, kv_heads, d)
    ref_f16q = oracle.attention_batched(q, kc, vc, 0, kv_len, 1, cap, heads, kv_heads, d,
                                        round_query_f16=True)
    assert np.abs(ref_f16q - ref).max() > 2 * atol
    monkeypatch.setenv("KRAKEN_DECODE_KERNEL", kernel)
    got = run_hip(hip_ctx, q, kc, vc, 0, kv_len, 1, cap, heads, kv_heads, d)
    err = np.abs(got - ref).max()
    print(f"  max abs error {err:.3g} (f16 query: {np.abs(ref_f16q - ref).max():.3g})", flush=True)
    assert err <= atol


@pytest.mark.gpu
@pytest.mark.parametrize("kernel", ["short", "mfma", "vector"])
@pytest.mark.parametrize("keys_per_split", [None, 16384])
def test_decode_sink_over_flat_tail(hip_ctx, monkeypatch, kernel, keys_per_split):
    """L=16384: key 0 scores 10 nats above 16383 equal keys (zero K rows), for
    every query head.  In the wave that holds the sink every other weight is
    e^-10 = 4.5e-5, below the smallest normal f16, and the tail carries 43% of
    the softmax mass; a kernel that lost those weights to a denormal flush would
    miss by far more than the 2e-5 allowed here.  One split of all keys puts a
    quarter of the tail in the sink's wave."""
    heads, kv_heads, d, kv_len = 8, 2, 256, 16383
    cap = kv_len + 1
    print(f"decode sink {kernel} keys_per_split={keys_per_split}", flush=True)
    rng = np.random.default_rng(7)
    qg = rng.standard_normal((kv_heads, d)).astype(np.float32)
    q = np.repeat(qg, heads // kv_heads, axis=0).reshape(-1)  # the heads of a group agree
    k = np.zeros((cap, kv_heads, d), np.float32)
    for h in range(kv_heads):
        k[0, h] = qg[h] * (10.0 * np.sqrt(d) / float(qg[h].astype(np.float64) @ qg[h]))
    kc = f16_bits(k.reshape(-1))
    vc = f16_bits(rng.standard_normal(cap * kv_heads * d))
    ref = oracle.attention_batched(q, kc, vc, 0, kv_len, 1, cap, heads, kv_heads, d)
    v0 = np.repeat(vc.view(np.float16).astype(np.float32).reshape(cap, kv_heads, d)[0],
                   heads // kv_heads, axis=0).reshape(-1)
    assert np.abs(ref - v0).max() > 0.1  # the tail matters
    monkeypatch.setenv("KRAKEN_DECODE_KERNEL", kernel)
    if keys_per_split is not None:
        monkeypatch.setenv("KRAKEN_DECODE_KEYS_PER_SPLIT", str(keys_per_split))
    got = run_hip(hip_ctx, q, kc, vc, 0, kv_len, 1, cap, heads, kv_heads, d)
    err = np.abs(got - ref).max()
    print(f"  max abs error {err:.3g}", flush=True)
    assert err <= 2e-5


@pytest.mark.gpu
def test_decode_gated_matches_separate_gate(hip_ctx):
    heads, kv_heads, d, kv_len = 8, 2, 256, 4096
    q, kc, vc = make_case(1, 1, kv_len, kv_len + 1, heads, kv_heads, d)
    gate = np.random.default_rng(11).standard_normal(heads * d).astype(np.float32)
    got = run_hip(hip_ctx, q, kc, vc, 0, kv_len, 1, kv_len + 1, heads, kv_heads, d, gate=gate)
    ref = oracle.sigmoid_gate_mul(
        oracle.attention_batched(q, kc, vc, 0, kv_len, 1, kv_len + 1, heads, kv_heads, d), gate)
    close(got, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [
    # tokens, start, heads, kv_heads, d
    (1, 0, 8, 2, 256), (7, 100, 8, 2, 256), (33, 500, 8, 8, 256), (63, 2000, 16, 2, 128),
    (5, 300, 16, 8, 128), (9, 50, 8, 1, 128), (4, 70, 4, 4, 64), (3, 40, 6, 3, 96),
    (2, 17, 2, 1, 200), (1, 1000, 24, 4, 128),
])
def test_decode_chunk_shapes_and_layer_offset(hip_ctx, shape):
    tokens, start, heads, kv_heads, d = shape
    cap = start + tokens + 3
    print(f"decode chunk {shape}", flush=True)
    q, kc, vc = make_case(2, tokens, start, cap, heads, kv_heads, d, layers=2)
    got = run_hip(hip_ctx, q, kc, vc, 1, start, tokens, cap, heads, kv_heads, d)
    ref = oracle.attention_batched(q, kc, vc, 1, start, tokens, cap, heads, kv_heads, d)
    close(got, ref, msg=str(shape))


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [
    # tokens, start, heads, kv_heads (head_dim 256, f16 cache: the MFMA decode kernel)
    (1, 4096, 8, 2), (1, 0, 8, 2), (1, 15, 8, 2), (1, 16, 8, 2), (1, 2047, 4, 2),
    (7, 100, 8, 2), (33, 500, 4, 4), (5, 20, 2, 1), (1, 30000, 8, 2),
])
@pytest.mark.parametrize("q_scale", [1.0, 12.0])
def test_decode_mfma_matches_vector_kernel_and_oracle(hip_ctx, monkeypatch, shape, q_scale):
    """The MFMA decode kernel (head_dim 256, f16 KV, up to 4 query heads per KV
    head; forced with KRAKEN_DECODE_KERNEL=mfma, since by default it takes only
    splits of 512 keys or more) against the oracle and against the vector
    kernel (KRAKEN_DECODE_KERNEL=vector), including keys that are not a
    multiple of its 16-key tiles, GQA groups 1/2/4 and a sharp softmax (q
    scaled by 12)."""
    tokens, start, heads, kv_heads = shape
    d = 256
    cap = start + tokens + 2
    print(f"decode mfma {shape} q_scale={q_scale}", flush=True)
    q, kc, vc = make_case(6, tokens, start, cap, heads, kv_heads, d, layers=2)
    q = (q * q_scale).astype(np.float32)
    ref = oracle.attention_batched(q, kc, vc, 1, start, tokens, cap, heads, kv_heads, d)
    monkeypatch.setenv("KRAKEN_DECODE_KERNEL", "mfma")
    got = run_hip(hip_ctx, q, kc, vc, 1, start, tokens, cap, heads, kv_heads, d)
    close(got, ref, msg=f"mfma {shape}")
    monkeypatch.setenv("KRAKEN_DECODE_KERNEL", "vector")
    vec = run_hip(hip_ctx, q, kc, vc, 1, start, tokens, cap, heads, kv_heads, d)
    close(vec, ref, msg=f"vector {shape}")
    close(got, vec, rtol=1e-3, atol=5e-4, msg=f"mfma vs vector {shape}")
    monkeypatch.setenv("KRAKEN_DECODE_KERNEL", "short")
    short = run_hip(hip_ctx, q, kc, vc, 1, start, tokens, cap, heads, kv_heads, d)
    close(short, ref, msg=f"short {shape}")
    close(short, vec, rtol=1e-3, atol=5e-4, msg=f"short vs vector {shape}")


@pytest.mark.gpu
@pytest.mark.parametrize("keys_per_split", ["16", "33", "100", "300"])
@pytest.mark.parametrize("shape", [(1, 4096, 8, 2), (1, 30000, 8, 2), (7, 100, 8, 2),
                                   (3, 2000, 2, 1), (1, 5000, 4, 2)])
def test_decode_short_kernel_split_sizes(hip_ctx, monkeypatch, keys_per_split, shape):
    """The short-split decode kernel (the batch-1 default) with splits of one
    tile, of several tiles per wave (its next-tile loads overlap the current
    tile's math) and with a partial last tile, GQA groups 1/2/4, sharp softmax
    (q scaled by 8), against the oracle."""
    tokens, start, heads, kv_heads = shape
    d = 256
    cap = start + tokens + 1
    print(f"decode short {shape} kps={keys_per_split}", flush=True)
    q, kc, vc = make_case(13, tokens, start, cap, heads, kv_heads, d)
    q = (q * 8.0).astype(np.float32)
    ref = oracle.attention_batched(q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d)
    monkeypatch.setenv("KRAKEN_DECODE_KERNEL", "short")
    monkeypatch.setenv("KRAKEN_DECODE_KEYS_PER_SPLIT", keys_per_split)
    got = run_hip(hip_ctx, q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d)
    close(got, ref, msg=f"short {shape} kps={keys_per_split}")


@pytest.mark.gpu
def test_decode_graph_replays(hip_ctx):
    """Batch-1 decode as bench.py runs it: three steps (two KV sets, two
    lengths) captured in one HIP graph on a torch stream and replayed three
    times, with eager work between the replays (the query changes in place);
    every replay matches the oracle."""
    torch = pytest.importorskip("torch")
    heads, kv_heads, d = 8, 2, 256
    lens = [4096, 1000, 4096]
    cap = 4097
    rng = np.random.default_rng(24)
    kcs = [f16_bits(rng.standard_normal(cap * kv_heads * d)) for _ in range(2)]
    vcs = [f16_bits(rng.standard_normal(cap * kv_heads * d)) for _ in range(2)]
    gate = rng.standard_normal(heads * d).astype(np.float32)
    dev = "cuda"
    kt = [torch.from_numpy(k.view(np.float16)).to(dev) for k in kcs]
    vt = [torch.from_numpy(v.view(np.float16)).to(dev) for v in vcs]
    gt = torch.from_numpy(gate).to(dev)
    qt = torch.zeros(heads * d, device=dev, dtype=torch.float32)
    outs = [torch.zeros(heads * d, device=dev, dtype=torch.float32) for _ in lens]
    stream = torch.cuda.Stream()
    hip_ctx.set_stream(stream.cuda_stream)
    hip_ctx.begin_graph()
    def steps():
        for i, n in enumerate(lens):
            hip_ctx.attention_f32_batched_f16_kv_gated(
                qt, kt[i % 2], vt[i % 2], gt, 0, n, 1, cap, heads, kv_heads, d, outs[i])

    try:
        with torch.cuda.stream(stream):
            # One eager pass first: the context sizes its workspace outside the
            # capture (a capturing stream cannot wait for a resize).
            steps()
            stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                steps()
            for replay in range(3):
                q = rng.standard_normal(heads * d).astype(np.float32) * (1.0 + 4.0 * replay)
                qt.copy_(torch.from_numpy(q).to(dev))
                torch.cuda.synchronize()
                graph.replay()
                stream.synchronize()
                for i, n in enumerate(lens):
                    ref = oracle.sigmoid_gate_mul(
                        oracle.attention_batched(q, kcs[i % 2], vcs[i % 2], 0, n, 1, cap, heads,
                                                 kv_heads, d), gate)
                    close(outs[i].cpu().numpy(), ref, msg=f"replay {replay} step {i}")
                    outs[i].zero_()
            del graph
    finally:
        hip_ctx.commit_graph()
        hip_ctx.set_stream(None)


@pytest.mark.gpu
def test_flash_graph_replays(hip_ctx):
    """Two split flash prefill calls (flash launch, then the merge launch) captured
    in one HIP graph and replayed three times with a new query before each replay
    and eager calls in between: every replay gives the eager call's bits."""
    torch = pytest.importorskip("torch")
    heads, kv_heads, d = 8, 2, 256
    calls = [(128, 1000), (1024, 3072)]  # tokens, start
    cap = 4096
    rng = np.random.default_rng(52)
    dev = "cuda"
    kt = torch.from_numpy(f16_bits(rng.standard_normal(cap * kv_heads * d)).view(np.float16)).to(dev)
    vt = torch.from_numpy(f16_bits(rng.standard_normal(cap * kv_heads * d)).view(np.float16)).to(dev)
    qts = [torch.zeros(t * heads * d, device=dev) for t, _ in calls]
    outs = [torch.zeros(t * heads * d, device=dev) for t, _ in calls]
    eager = [torch.zeros(t * heads * d, device=dev) for t, _ in calls]
    stream = torch.cuda.Stream()
    hip_ctx.set_stream(stream.cuda_stream)

    def steps(dst):
        for i, (t, start) in enumerate(calls):
            hip_ctx.attention_f32_batched_f16_kv(qts[i], kt, vt, 0, start, t, cap, heads,
                                                 kv_heads, d, dst[i])

    try:
        with torch.cuda.stream(stream):
            steps(eager)
            stream.synchronize()
            hip_ctx.begin_graph()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                steps(outs)
            hip_ctx.commit_graph()
            for replay in range(3):
                for i, (t, _) in enumerate(calls):
                    q = rng.standard_normal(t * heads * d).astype(np.float32) * (1.0 + replay)
                    qts[i].copy_(torch.from_numpy(q).to(dev))
                torch.cuda.synchronize()
                graph.replay()
                stream.synchronize()
                steps(eager)
                stream.synchronize()
                for i in range(len(calls)):
                    got, want = outs[i].cpu().numpy(), eager[i].cpu().numpy()
                    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
                        f"replay {replay} call {i}"
                    outs[i].zero_()
            del graph
    finally:
        hip_ctx.commit_graph()
        hip_ctx.set_stream(None)


@pytest.mark.gpu
def test_workspace_growth_between_replays(hip_ctx):
    """A graph captured while the context's workspace was small keeps replaying
    correctly after an eager call has grown the workspace: the outgrown
    workspace stays allocated (the graph holds its address) until the context
    is destroyed.  Decode step at L=4096 captured; a C2-sized flash prefill
    (T=1024 after 3072 cached tokens, 34 MB of split partials) grows the
    workspace between replays, and the context is used again afterwards."""
    torch = pytest.importorskip("torch")
    heads, kv_heads, d, n = 8, 2, 256, 4096
    cap = 4096 + 1024
    rng = np.random.default_rng(31)
    kc = f16_bits(rng.standard_normal(cap * kv_heads * d))
    vc = f16_bits(rng.standard_normal(cap * kv_heads * d))
    gate = rng.standard_normal(heads * d).astype(np.float32)
    dev = "cuda"
    kt = torch.from_numpy(kc.view(np.float16)).to(dev)
    vt = torch.from_numpy(vc.view(np.float16)).to(dev)
    gt = torch.from_numpy(gate).to(dev)
    qt = torch.zeros(heads * d, device=dev, dtype=torch.float32)
    out = torch.zeros(heads * d, device=dev, dtype=torch.float32)
    stream = torch.cuda.Stream()
    hip_ctx.set_stream(stream.cuda_stream)
    hip_ctx.begin_graph()

    def step():
        hip_ctx.attention_f32_batched_f16_kv_gated(qt, kt, vt, gt, 0, n, 1, cap, heads,
                                                   kv_heads, d, out)

    def check(q, what):
        ref = oracle.sigmoid_gate_mul(
            oracle.attention_batched(q, kc, vc, 0, n, 1, cap, heads, kv_heads, d), gate)
        close(out.cpu().numpy(), ref, msg=what)
        out.zero_()

    try:
        with torch.cuda.stream(stream):
            step()
            stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                step()
            for replay in range(3):
                q = rng.standard_normal(heads * d).astype(np.float32)
                qt.copy_(torch.from_numpy(q).to(dev))
                torch.cuda.synchronize()
                graph.replay()
                stream.synchronize()
                check(q, f"replay {replay}")
                if replay == 0:
                    # Eager prefill chunk that needs a larger workspace.
                    t, start = 1024, 3072
                    qp = rng.standard_normal(t * heads * d).astype(np.float32)
                    qpt = torch.from_numpy(qp).to(dev)
                    op = torch.zeros(t * heads * d, device=dev, dtype=torch.float32)
                    hip_ctx.attention_f32_batched_f16_kv(qpt, kt, vt, 0, start, t, cap, heads,
                                                         kv_heads, d, op)
                    stream.synchronize()
                    sample = [0, 511, 1023]
                    got = op.cpu().numpy().reshape(t, heads * d)[sample]
                    for i, tok in enumerate(sample):
                        qs = qp.reshape(t, heads * d)[tok]
                        ref = oracle.attention_batched(qs, kc, vc, 0, start + tok, 1, cap, heads,
                                                       kv_heads, d, round_query_f16=True)
                        close(got[i], ref, msg=f"prefill token {tok}")
            del graph
            step()  # eager again, on the grown workspace
            stream.synchronize()
            check(q, "eager after growth")
    finally:
        hip_ctx.commit_graph()
        hip_ctx.set_stream(None)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(1, 300, 16, 8, 128), (8, 64, 8, 2, 256), (3, 9, 4, 1, 64)])
def test_f32_kv_twin(hip_ctx, shape):
    tokens, start, heads, kv_heads, d = shape
    cap = start + tokens
    rng = np.random.default_rng(3)
    q = rng.standard_normal(tokens * heads * d).astype(np.float32)
    kc = rng.standard_normal(cap * kv_heads * d).astype(np.float32)
    vc = rng.standard_normal(cap * kv_heads * d).astype(np.float32)
    got = run_hip(hip_ctx, q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d)
    ref = oracle.attention_batched(q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d)
    close(got, ref, rtol=1e-4, atol=1e-4)


@pytest.mark.gpu
def test_decode_uniform_average_closed_form(hip_ctx):
    """q = 0 gives the uniform mean of V over the causal prefix (smoke_test.cpp:1688-1725)."""
    heads, kv_heads, d, tokens, start = 8, 2, 256, 5, 3000
    cap = start + tokens
    rng = np.random.default_rng(4)
    v = rng.standard_normal(cap * kv_heads * d).astype(np.float32)
    vb = f16_bits(v)
    vf = vb.view(np.float16).astype(np.float64).reshape(cap, kv_heads, d)
    q = np.zeros(tokens * heads * d, np.float32)
    kb = f16_bits(rng.standard_normal(cap * kv_heads * d))
    got = run_hip(hip_ctx, q, kb, vb, 0, start, tokens, cap, heads, kv_heads, d)
    got = got.reshape(tokens, heads, d)
    for t in range(tokens):
        mean = vf[:start + t + 1].mean(axis=0)
        for h in range(heads):
            close(got[t, h], mean[h // 4], rtol=1e-4, atol=1e-5)


# ------------------------------------------------------------------ flash ----

def mrope_l2_inputs(seed, tokens, prefix, heads=8, kv_heads=2, d=256):
    """C2 inputs: q,k ~ N(0,1) with MRoPE (sections 11,11,10,0; theta 1e7; pos = P+i)
    then L2-normalised per head; v ~ N(0,1); all fp16-representable."""
    rng = np.random.default_rng(seed)
    cap = prefix + tokens
    q = rng.standard_normal(tokens * heads * d).astype(np.float32)
    k = rng.standard_normal(cap * kv_heads * d).astype(np.float32)
    v = rng.standard_normal(cap * kv_heads * d).astype(np.float32)
    qpos = oracle.make_mrope_positions(prefix, tokens)
    kpos = oracle.make_mrope_positions(0, cap)
    q = oracle.mrope(q, qpos, tokens, heads, d, 64, (11, 11, 10, 0), 1e7)
    k = oracle.mrope(k, kpos, cap, kv_heads, d, 64, (11, 11, 10, 0), 1e7)
    q = oracle.l2_norm(q, tokens * heads, d, 1e-6)
    k = oracle.l2_norm(k, cap * kv_heads, d, 1e-6)
    q = q.astype(np.float16).astype(np.float32)
    return q, f16_bits(k), f16_bits(v)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [
    # tokens, start, heads, kv_heads
    (64, 0, 8, 2), (65, 0, 2, 1), (128, 0, 8, 2), (100, 37, 8, 2), (256, 1000, 8, 2),
    (96, 7, 8, 8), (70, 3, 4, 2), (64, 64, 8, 1),
])
def test_flash_prefill_vs_oracle(hip_ctx, shape):
    tokens, start, heads, kv_heads = shape
    d = 256
    cap = start + tokens + 5
    print(f"flash {shape}", flush=True)
    q, kc, vc = make_case(5, tokens, start, cap, heads, kv_heads, d)
    got = run_hip(hip_ctx, q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d)
    ref = oracle.attention_batched(q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d,
                                   round_query_f16=True)
    close(got, ref, msg=str(shape))


@pytest.mark.gpu
@pytest.mark.parametrize("q_scale,splits", [(8.0, None), (30.0, None), (8.0, "1"), (8.0, "3")])
def test_flash_sharp_softmax_and_split_counts(hip_ctx, q_scale, splits, monkeypatch):
    """Scaled queries make the running max jump by far more than the lazy-rescale
    slack many times along the key axis; forced split counts move the split
    boundaries (KRAKEN_FLASH_SPLITS)."""
    tokens, start, heads, kv_heads, d = 160, 300, 8, 2, 256
    cap = start + tokens
    if splits is not None:
        monkeypatch.setenv("KRAKEN_FLASH_SPLITS", splits)
    print(f"flash sharp q_scale={q_scale} splits={splits}", flush=True)
    q, kc, vc = make_case(21, tokens, start, cap, heads, kv_heads, d)
    q = (q * q_scale).astype(np.float16).astype(np.float32)
    got = run_hip(hip_ctx, q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d)
    ref = oracle.attention_batched(q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d,
                                   round_query_f16=True)
    close(got, ref, msg=f"q_scale={q_scale} splits={splits}")


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [
    # tokens, start, heads, kv_heads: flash at C2's P=3072 and unaligned, then
    # the decode kernels (short chunk, single token)
    (1024, 3072, 8, 2), (100, 37, 8, 2), (7, 300, 8, 2), (1, 4096, 8, 2),
])
def test_f16_query_entry_equals_f32_entry(hip_ctx, shape):
    """kraken_hip_attention_f16q_batched_f16_kv on f16 query values gives the f32
    entry's output bit for bit on the same (f16-representable) values: the flash
    kernel reads the f16 row instead of rounding the f32 one, the decode kernels
    read the exact widening."""
    tokens, start, heads, kv_heads = shape
    d = 256
    cap = start + tokens
    print(f"f16 query entry {shape}", flush=True)
    q, kc, vc = make_case(31, tokens, start, cap, heads, kv_heads, d)
    q16 = q.astype(np.float16)
    want = run_hip(hip_ctx, q16.astype(np.float32), kc, vc, 0, start, tokens, cap, heads,
                   kv_heads, d)
    qb = hip_ctx.buffer(q16.view(np.uint16), dtype=np.uint16)
    kb, vb = hip_ctx.buffer(kc, dtype=np.uint16), hip_ctx.buffer(vc, dtype=np.uint16)
    out = hip_ctx.buffer(byte_size=4 * tokens * heads * d)
    hip_ctx.attention_f16q_batched_f16_kv(qb, kb, vb, 0, start, tokens, cap, heads, kv_heads,
                                          d, out)
    got = out.download(tokens * heads * d)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), shape


@pytest.mark.gpu
def test_flash_gated(hip_ctx):
    tokens, start, heads, kv_heads, d = 128, 200, 8, 2, 256
    cap = start + tokens
    q, kc, vc = make_case(6, tokens, start, cap, heads, kv_heads, d)
    gate = np.random.default_rng(12).standard_normal(tokens * heads * d).astype(np.float32)
    got = run_hip(hip_ctx, q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d, gate=gate)
    ref = oracle.sigmoid_gate_mul(oracle.attention_batched(
        q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d, round_query_f16=True), gate)
    close(got, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("prefix", [0, 3072, 7168])
def test_flash_c2_full_shape_sampled_tokens(hip_ctx, prefix):
    """C2 at full size (T=1024, P in {0,3072,7168}); the oracle checks 12 sampled
    query tokens (first, last, tile edges, random) of every head."""
    tokens, heads, kv_heads, d = 1024, 8, 2, 256
    cap = prefix + tokens
    print(f"flash C2 P={prefix}", flush=True)
    q, kc, vc = mrope_l2_inputs(2, tokens, prefix)
    got = run_hip(hip_ctx, q, kc, vc, 0, prefix, tokens, cap, heads, kv_heads, d)
    got = got.reshape(tokens, heads * d)
    rng = np.random.default_rng(7)
    sample = sorted({0, 31, 32, 63, 64, 511, 1022, 1023, *rng.integers(0, tokens, 4).tolist()})
    for t in sample:
        ref = oracle.attention_batched(q[t * heads * d:(t + 1) * heads * d], kc, vc, 0,
                                       prefix + t, 1, cap, heads, kv_heads, d,
                                       round_query_f16=True)
        close(got[t], ref, msg=f"P={prefix} t={t}")


@pytest.mark.gpu
@pytest.mark.parametrize("prefix", [0, 3072, 7168])
def test_flash_agrees_with_split_decode_unnormalised(hip_ctx, prefix, monkeypatch):
    """Two independent kernels (MFMA flash and VALU split-K) agree on every
    output at C2's shape with un-normalised N(0,1) q/k (a sharper softmax than
    the L2-normalised C2 inputs)."""
    tokens, heads, kv_heads, d = 1024, 8, 2, 256
    cap = prefix + tokens
    q, kc, vc = make_case(8, tokens, prefix, cap, heads, kv_heads, d)
    q = q.astype(np.float16).astype(np.float32)  # flash rounds Q; give both the same Q
    flash = run_hip(hip_ctx, q, kc, vc, 0, prefix, tokens, cap, heads, kv_heads, d)
    monkeypatch.setenv("KRAKEN_QWEN35_FLASH_ATTENTION", "0")
    split = run_hip(hip_ctx, q, kc, vc, 0, prefix, tokens, cap, heads, kv_heads, d)
    close(flash, split)


def smoke_pattern_case(tokens, heads, kv_heads, d, qa, qm, qo, qs, ka, km, ko, ks, va, vm, vo, vs):
    """The reference smoke test's modular input patterns (smoke_test.cpp:1744-1753, 1832-1841)."""
    qv = tokens * heads * d
    kv = tokens * kv_heads * d
    i = np.arange(qv)
    q = (((i * qa) % qm) - qo).astype(np.float32) * np.float32(qs)
    j = np.arange(kv)
    k = (((j * ka) % km) - ko).astype(np.float32) * np.float32(ks)
    v = (((j * va) % vm) - vo).astype(np.float32) * np.float32(vs)
    return q, k, v


@pytest.mark.gpu
def test_reference_smoke_64_token_flash_equivalence(hip_ctx, monkeypatch):
    """smoke_test.cpp:1727-1812: 64 tokens, 8/2/256; flash vs default within 1e-5 on f32 KV.
    Here: F16 flash vs the oracle on the f16-rounded cache, and F32 decode vs oracle."""
    tokens, heads, kv_heads, d = 64, 8, 2, 256
    q, k, v = smoke_pattern_case(tokens, heads, kv_heads, d, 13, 31, 15, 0.015, 7, 29, 14,
                                 0.012, 11, 37, 18, 0.025)
    ref32 = oracle.attention_batched(q, k, v, 0, 0, tokens, tokens, heads, kv_heads, d)
    got32 = run_hip(hip_ctx, q, k, v, 0, 0, tokens, tokens, heads, kv_heads, d)
    close(got32, ref32, rtol=1e-5, atol=1e-5)
    kb, vb = f16_bits(k), f16_bits(v)
    got16 = run_hip(hip_ctx, q, kb, vb, 0, 0, tokens, tokens, heads, kv_heads, d)
    close(got16, ref32, rtol=0, atol=5e-3)
    ref16 = oracle.attention_batched(q, kb, vb, 0, 0, tokens, tokens, heads, kv_heads, d,
                                     round_query_f16=True)
    close(got16, ref16)


@pytest.mark.gpu
def test_reference_smoke_65_token_unaligned(hip_ctx, monkeypatch):
    """smoke_test.cpp:1814-1972: 65 tokens, 2/1/256, F16 flash vs F32 default within 5e-3,
    and F16 flash vs F16 default (forced by KRAKEN_QWEN35_FLASH_ATTENTION) within 5e-3."""
    tokens, heads, kv_heads, d = 65, 2, 1, 256
    q, k, v = smoke_pattern_case(tokens, heads, kv_heads, d, 17, 43, 21, 0.01, 5, 41, 20,
                                 0.011, 19, 47, 23, 0.017)
    ref32 = oracle.attention_batched(q, k, v, 0, 0, tokens, tokens, heads, kv_heads, d)
    kb, vb = f16_bits(k), f16_bits(v)
    monkeypatch.setenv("KRAKEN_QWEN35_FLASH_ATTENTION", "1")
    flash16 = run_hip(hip_ctx, q, kb, vb, 0, 0, tokens, tokens, heads, kv_heads, d)
    monkeypatch.setenv("KRAKEN_QWEN35_FLASH_ATTENTION", "0")
    default16 = run_hip(hip_ctx, q, kb, vb, 0, 0, tokens, tokens, heads, kv_heads, d)
    close(flash16, ref32, rtol=0, atol=5e-3)
    close(flash16, default16, rtol=0, atol=5e-3)


@pytest.mark.gpu
def test_gqa_heads_with_equal_query_agree(hip_ctx):
    heads, kv_heads, d, kv_len = 8, 2, 256, 2048
    rng = np.random.default_rng(9)
    qh = rng.standard_normal(d).astype(np.float32)
    q = np.tile(qh, heads)
    kc = f16_bits(rng.standard_normal((kv_len + 1) * kv_heads * d))
    vc = f16_bits(rng.standard_normal((kv_len + 1) * kv_heads * d))
    out = run_hip(hip_ctx, q, kc, vc, 0, kv_len, 1, kv_len + 1, heads, kv_heads, d)
    out = out.reshape(heads, d)
    for h in range(heads):
        np.testing.assert_array_equal(out[h], out[(h // 4) * 4])
