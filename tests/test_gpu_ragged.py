"""Ragged multi-sequence decode on the GPU against the CPU oracle, sequence by
sequence.

Each sequence contributes one token.  Its result must equal the single-sequence
op's on its own data:
- attention: oracle_attention_batched with tokens = 1, start = position, f16 KV
  (mps_backend.mm:2943-3008), then sigmoid(G) when gated
  (qwen35_runtime.cpp:3347-3355);
- GDN: oracle_gated_delta_net with tokens = 1 (mps_backend.mm:2307-2374);
- conv prologue: oracle build_ssm_conv_state + ssm_conv + SiLU + split/L2
  (mps_backend.mm:2097-2153, 2376-2457).
Pools hold the sequences at scattered offsets with gaps.  Out-of-pool and
misaligned offsets must leave memory untouched or read zeros, never fault.
Tolerances: 2e-3 rel / 1e-3 abs (f16 KV); 1e-4 abs on f32 GDN state and
outputs; 1e-5 on the conv prologue.
"""
import numpy as np
import pytest

import kraken_hip as kh
import oracle

pytestmark = pytest.mark.gpu


def scattered_offsets(rng, rows, row_elems, align=8):
    """Element offsets of sequences with `rows[i]` rows each, in order, with random
    aligned gaps; returns (offsets, total elements)."""
    offsets, cur = [], 0
    for r in rows:
        cur += int(rng.integers(0, 4)) * align
        offsets.append(cur)
        cur += r * row_elems
        cur = (cur + align - 1) // align * align
    return np.array(offsets, np.uint64), cur + 4 * align


def attention_reference(q, kpool, vpool, offsets, positions, heads, kv_heads, d, gate=None):
    kv_dim = kv_heads * d
    out = []
    for b, (off, pos) in enumerate(zip(offsets, positions)):
        rows = int(pos) + 1
        kc = kpool[int(off):int(off) + rows * kv_dim].view(np.uint16)
        vc = vpool[int(off):int(off) + rows * kv_dim].view(np.uint16)
        qb = q[b * heads * d:(b + 1) * heads * d]
        r = oracle.attention_batched(qb, kc, vc, 0, int(pos), 1, rows, heads, kv_heads, d)
        if gate is not None:
            r = oracle.sigmoid_gate_mul(r, gate[b * heads * d:(b + 1) * heads * d])
        out.append(r)
    return np.concatenate(out)


@pytest.mark.parametrize("d,heads,kv_heads,kernel", [
    (256, 8, 2, None), (256, 8, 2, "vector"), (256, 4, 4, None), (128, 8, 4, None),
    (64, 16, 2, None)])
@pytest.mark.parametrize("gated", [False, True])
def test_ragged_attention_matches_oracle(hip_ctx, monkeypatch, d, heads, kv_heads, kernel, gated):
    """Head_dim 256 with an f16 pool takes the MFMA decode kernel by default (1024-key
    splits); kernel "vector" forces the vector kernel on the same case."""
    if kernel is None:
        monkeypatch.delenv("KRAKEN_DECODE_KERNEL", raising=False)
    else:
        monkeypatch.setenv("KRAKEN_DECODE_KERNEL", kernel)
    rng = np.random.default_rng(40 + d + heads)
    # Positions around the 1024-key split boundary, tiny and long ones.
    positions = np.array([0, 1, 31, 1023, 1024, 1025, 2047, 3000, 5], np.uint32)
    b = len(positions)
    kv_dim = kv_heads * d
    offsets, total = scattered_offsets(rng, positions.astype(np.int64) + 1, kv_dim)
    kpool = rng.standard_normal(total).astype(np.float16)
    vpool = rng.standard_normal(total).astype(np.float16)
    q = rng.standard_normal(b * heads * d).astype(np.float32)
    gate = rng.standard_normal(b * heads * d).astype(np.float32) if gated else None
    ctx = hip_ctx
    kb, vb = ctx.buffer(kpool.view(np.uint16)), ctx.buffer(vpool.view(np.uint16))
    qb, ob = ctx.buffer(q), ctx.buffer(byte_size=4 * q.size)
    gb = ctx.buffer(gate) if gated else None
    ctx.attention_f32_ragged_f16_kv(qb, kb, vb, gb, ctx.buffer(offsets), ctx.buffer(positions),
                                    b, int(positions.max()), heads, kv_heads, d, ob)
    got = ob.download()
    ref = attention_reference(q, kpool, vpool, offsets, positions, heads, kv_heads, d, gate)
    np.testing.assert_allclose(got, ref, rtol=2e-3, atol=1e-3)


def test_ragged_attention_bad_offsets_read_zeros(hip_ctx):
    """An offset outside the pool, or not a whole 16-byte chunk, reads zeros: the
    output is the uniform mean of zero values (0); other sequences are unaffected."""
    rng = np.random.default_rng(7)
    heads, kv_heads, d = 8, 2, 256
    kv_dim = kv_heads * d
    positions = np.array([100, 200, 300, 50], np.uint32)
    offsets, total = scattered_offsets(rng, positions.astype(np.int64) + 1, kv_dim)
    good = offsets.copy()
    offsets[1] = np.uint64(total + 1024)          # past the pool
    offsets[3] = np.uint64(int(offsets[3]) + 3)   # misaligned rows
    kpool = rng.standard_normal(total).astype(np.float16)
    vpool = rng.standard_normal(total).astype(np.float16)
    q = rng.standard_normal(4 * heads * d).astype(np.float32)
    ctx = hip_ctx
    ob = ctx.buffer(byte_size=4 * q.size)
    ctx.attention_f32_ragged_f16_kv(ctx.buffer(q), ctx.buffer(kpool.view(np.uint16)),
                                    ctx.buffer(vpool.view(np.uint16)), None,
                                    ctx.buffer(offsets), ctx.buffer(positions), 4, 300, heads,
                                    kv_heads, d, ob)
    got = ob.download().reshape(4, heads * d)
    ref = attention_reference(q, kpool, vpool, good, positions, heads, kv_heads, d)
    ref = ref.reshape(4, heads * d)
    np.testing.assert_array_equal(got[1], 0.0)
    np.testing.assert_array_equal(got[3], 0.0)
    np.testing.assert_allclose(got[[0, 2]], ref[[0, 2]], rtol=2e-3, atol=1e-3)


def test_ragged_kv_append(hip_ctx):
    rng = np.random.default_rng(8)
    kv_dim = 512
    positions = np.array([0, 7, 1500, 3], np.uint32)
    offsets, total = scattered_offsets(rng, positions.astype(np.int64) + 1, kv_dim)
    kpool = rng.standard_normal(total).astype(np.float16)
    vpool = rng.standard_normal(total).astype(np.float16)
    krows = rng.standard_normal(4 * kv_dim).astype(np.float32)
    vrows = rng.standard_normal(4 * kv_dim).astype(np.float32)
    ctx = hip_ctx
    kb, vb = ctx.buffer(kpool.view(np.uint16)), ctx.buffer(vpool.view(np.uint16))
    ctx.append_kv_ragged_f16(ctx.buffer(krows), ctx.buffer(vrows), kb, vb, ctx.buffer(offsets),
                             ctx.buffer(positions), 4, kv_dim)
    ek, ev = kpool.copy(), vpool.copy()
    for b in range(4):
        row = int(offsets[b]) + int(positions[b]) * kv_dim
        ek[row:row + kv_dim] = krows[b * kv_dim:(b + 1) * kv_dim].astype(np.float16)
        ev[row:row + kv_dim] = vrows[b * kv_dim:(b + 1) * kv_dim].astype(np.float16)
    np.testing.assert_array_equal(kb.download(dtype=np.uint16), ek.view(np.uint16))
    np.testing.assert_array_equal(vb.download(dtype=np.uint16), ev.view(np.uint16))


def gdn_inputs(rng, b, hk, hv, dd):
    def unit(n):
        x = rng.standard_normal((n, dd)).astype(np.float32)
        return (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32).ravel()
    q, k = unit(b * hk), unit(b * hk)
    v = rng.standard_normal(b * hv * dd).astype(np.float32)
    g = (-np.logaddexp(0, rng.standard_normal(b * hv))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal(b * hv)))).astype(np.float32)
    return q, k, v, g, beta


def test_ragged_gdn_decode_matches_oracle(hip_ctx):
    rng = np.random.default_rng(9)
    b, hk, hv, dd = 6, 16, 16, 128
    state_elems = hv * dd * dd
    offsets, total = scattered_offsets(rng, [1] * b, state_elems, align=dd)
    offsets[4] = np.uint64(total + 7)  # outside the pool: skipped, nothing touched
    pool = (0.1 * rng.standard_normal(total)).astype(np.float32)
    q, k, v, g, beta = gdn_inputs(rng, b, hk, hv, dd)
    ctx = hip_ctx
    sb = ctx.buffer(pool)
    sentinel = np.full(b * hv * dd, 7.0, np.float32)
    ob = ctx.buffer(sentinel)
    ctx.gated_delta_net_f32_ragged_decode(ctx.buffer(q), ctx.buffer(k), ctx.buffer(v),
                                          ctx.buffer(g), ctx.buffer(beta), sb,
                                          ctx.buffer(offsets), b, hk, hv, dd, ob)
    got_out = ob.download().reshape(b, hv * dd)
    got_pool = sb.download()
    exp_pool = pool.copy()
    for i in range(b):
        if i == 4:
            np.testing.assert_array_equal(got_out[i], 7.0)
            continue
        off = int(offsets[i])
        s = pool[off:off + state_elems].copy()
        sl = slice(i * hk * dd, (i + 1) * hk * dd)
        vl = slice(i * hv * dd, (i + 1) * hv * dd)
        gl = slice(i * hv, (i + 1) * hv)
        out, st = oracle.gated_delta_net(q[sl], k[sl], v[vl], g[gl], beta[gl], s, 1, hk, hv, dd)
        np.testing.assert_allclose(got_out[i], out, rtol=0, atol=1e-4)
        exp_pool[off:off + state_elems] = st
    np.testing.assert_allclose(got_pool, exp_pool, rtol=0, atol=1e-4)


def test_ragged_conv_split_matches_oracle(hip_ctx):
    rng = np.random.default_rng(10)
    b, hk, hv, dd, kk = 5, 16, 16, 128, 4
    ch = (2 * hk + hv) * dd
    state_elems = ch * (kk - 1)
    offsets, total = scattered_offsets(rng, [1] * b, state_elems, align=64)
    pool = rng.standard_normal(total).astype(np.float32)
    x = rng.standard_normal(b * ch).astype(np.float32)
    w = (0.5 * rng.standard_normal(ch * kk)).astype(np.float32)
    ctx = hip_ctx
    pb = ctx.buffer(pool)
    qb, kb = ctx.buffer(byte_size=4 * b * hk * dd), ctx.buffer(byte_size=4 * b * hk * dd)
    vb = ctx.buffer(byte_size=4 * b * hv * dd)
    ctx.qwen35_conv_split_l2_ragged_decode_f32(ctx.buffer(x), pb, ctx.buffer(offsets),
                                               ctx.buffer(w), kk, b, hk, hv, dd, 1e-6, qb, kb,
                                               vb)
    gq, gk, gv = qb.download(), kb.download(), vb.download()
    got_pool = pb.download()
    exp_pool = pool.copy()
    for i in range(b):
        off = int(offsets[i])
        st = pool[off:off + state_elems].copy()
        xi = x[i * ch:(i + 1) * ch]
        ci, new_state = oracle.build_ssm_conv_state(st, xi, kk, ch, 1)
        y = oracle.silu(oracle.ssm_conv(ci, w, kk, ch, 1, 1))
        rq, rk, rv = oracle.split_qkv_l2_norm(y, 1, hk, hv, dd, 1e-6)
        np.testing.assert_allclose(gq[i * hk * dd:(i + 1) * hk * dd], rq, rtol=0, atol=1e-5)
        np.testing.assert_allclose(gk[i * hk * dd:(i + 1) * hk * dd], rk, rtol=0, atol=1e-5)
        np.testing.assert_allclose(gv[i * hv * dd:(i + 1) * hv * dd], rv, rtol=0, atol=1e-5)
        exp_pool[off:off + state_elems] = new_state
    np.testing.assert_array_equal(got_pool, exp_pool)


def test_ragged_attention_c4_shape_sampled(hip_ctx):
    """C4 attention layer shape: 64 sequences, lengths in [512, 32768]; eight
    sequences (shortest, longest and six others) checked against the oracle."""
    rng = np.random.default_rng(4)
    heads, kv_heads, d = 8, 2, 256
    kv_dim = kv_heads * d
    b = 64
    positions = rng.integers(512, 32769, b).astype(np.uint32)
    offsets, total = scattered_offsets(rng, positions.astype(np.int64) + 1, kv_dim)
    # ~1 GB per pool: a random 1M-element block repeated (period ~2048 rows).
    block = 1 << 20
    kpool = np.resize(rng.standard_normal(block).astype(np.float16), total)
    vpool = np.resize(rng.standard_normal(block + 8).astype(np.float16), total)
    q = rng.standard_normal(b * heads * d).astype(np.float32)
    gate = rng.standard_normal(b * heads * d).astype(np.float32)
    ctx = hip_ctx
    ob = ctx.buffer(byte_size=4 * q.size)
    ctx.attention_f32_ragged_f16_kv(ctx.buffer(q), ctx.buffer(kpool.view(np.uint16)),
                                    ctx.buffer(vpool.view(np.uint16)), ctx.buffer(gate),
                                    ctx.buffer(offsets), ctx.buffer(positions), b,
                                    int(positions.max()), heads, kv_heads, d, ob)
    got = ob.download().reshape(b, heads * d)
    pick = sorted({int(np.argmin(positions)), int(np.argmax(positions)), 3, 17, 29, 40, 51, 63})
    for i in pick:
        sl = slice(i * heads * d, (i + 1) * heads * d)
        ref = attention_reference(q[sl], kpool, vpool, offsets[i:i + 1], positions[i:i + 1],
                                  heads, kv_heads, d, gate[sl])
        np.testing.assert_allclose(got[i], ref, rtol=2e-3, atol=1e-3, err_msg=f"sequence {i}")


def _gdn_layer_case(rng, b, hk, hv, dd, kk, prepare):
    ch = (2 * hk + hv) * dd
    conv_elems = ch * (kk - 1)
    state_elems = hv * dd * dd
    coffs, ctotal = scattered_offsets(rng, [1] * b, conv_elems, align=64)
    soffs, stotal = scattered_offsets(rng, [1] * b, state_elems, align=dd)
    c = dict(
        qkv=rng.standard_normal(b * ch).astype(np.float32),
        conv_pool=rng.standard_normal(ctotal).astype(np.float32),
        w=(0.5 * rng.standard_normal(ch * kk)).astype(np.float32),
        gate=rng.standard_normal(b * hv).astype(np.float32),
        beta=rng.standard_normal(b * hv).astype(np.float32),
        z=rng.standard_normal(b * hv * dd).astype(np.float32),
        nw=(1 + 0.1 * rng.standard_normal(dd)).astype(np.float32),
        state_pool=(0.1 * rng.standard_normal(stotal)).astype(np.float32),
        coffs=coffs, soffs=soffs)
    if prepare:
        c["dtb"] = rng.standard_normal(hv).astype(np.float32)
        c["ssa"] = (-rng.random(hv)).astype(np.float32)
    else:
        c["gate"] = (-np.logaddexp(0, c["gate"])).astype(np.float32)
        c["beta"] = (1 / (1 + np.exp(-c["beta"]))).astype(np.float32)
    return c


def _run_gdn_layer(ctx, c, b, hk, hv, dd, kk):
    cp, sp = ctx.buffer(c["conv_pool"]), ctx.buffer(c["state_pool"])
    ob = ctx.buffer(np.full(b * hv * dd, 7.0, np.float32))
    dtb = ctx.buffer(c["dtb"]) if "dtb" in c else None
    ssa = ctx.buffer(c["ssa"]) if "ssa" in c else None
    ctx.qwen35_gdn_layer_ragged_decode_f32(
        ctx.buffer(c["qkv"]), cp, ctx.buffer(c["coffs"]), ctx.buffer(c["w"]), kk,
        ctx.buffer(c["gate"]), ctx.buffer(c["beta"]), dtb, ssa, ctx.buffer(c["z"]),
        ctx.buffer(c["nw"]), sp, ctx.buffer(c["soffs"]), b, hk, hv, dd, 1e-6, ob)
    return ob.download(), cp.download(), sp.download()


def _run_gdn_chain(ctx, c, b, hk, hv, dd, kk):
    """The same step as the separate ragged ops (gate/beta prepared on the device)."""
    cp, sp = ctx.buffer(c["conv_pool"]), ctx.buffer(c["state_pool"])
    qb, kb = ctx.buffer(byte_size=4 * b * hk * dd), ctx.buffer(byte_size=4 * b * hk * dd)
    vb = ctx.buffer(byte_size=4 * b * hv * dd)
    ctx.qwen35_conv_split_l2_ragged_decode_f32(ctx.buffer(c["qkv"]), cp, ctx.buffer(c["coffs"]),
                                               ctx.buffer(c["w"]), kk, b, hk, hv, dd, 1e-6, qb,
                                               kb, vb)
    gb, bb = ctx.buffer(c["gate"]), ctx.buffer(c["beta"])
    if "dtb" in c:
        ctx.prepare_qwen35_gdn_gate_beta_f32(gb, bb, ctx.buffer(c["dtb"]), ctx.buffer(c["ssa"]),
                                             b, hv)
    ob = ctx.buffer(byte_size=4 * b * hv * dd)
    ctx.gated_delta_net_f32_ragged_decode(qb, kb, vb, gb, bb, sp, ctx.buffer(c["soffs"]), b, hk,
                                          hv, dd, ob)
    ctx.qwen35_norm_gated_f32_in_place(ob, ctx.buffer(c["nw"]), ctx.buffer(c["z"]), b, hv, dd,
                                       1e-6)
    return ob.download(), cp.download(), sp.download()


@pytest.mark.parametrize("shape,prepare", [
    ((7, 16, 16, 128, 4), True), ((7, 16, 16, 128, 4), False),  # one kernel
    ((1, 16, 16, 128, 4), True), ((4, 16, 16, 128, 4), False),  # one kernel, few sequences
    ((5, 2, 4, 64, 3), True), ((3, 4, 4, 96, 4), False),         # three-kernel chain
])
def test_ragged_gdn_layer_matches_chain_and_oracle(hip_ctx, shape, prepare):
    """kraken_hip_qwen35_gdn_layer_ragged_decode_f32 against the three ragged ops
    it replaces (equal bit for bit for the one-kernel shapes, among them a single
    sequence; the chain shapes are that chain) and against the oracle's conv,
    prepare, recurrence and norm-gated steps per sequence (1e-4 absolute).  The
    layer runs twice on the same inputs and gives the same result both times."""
    b, hk, hv, dd, kk = shape
    print(f"gdn layer {shape} prepare={prepare}", flush=True)
    rng = np.random.default_rng(50 + b + hk)
    c = _gdn_layer_case(rng, b, hk, hv, dd, kk, prepare)
    out, cpool, spool = _run_gdn_layer(hip_ctx, c, b, hk, hv, dd, kk)
    again = _run_gdn_layer(hip_ctx, c, b, hk, hv, dd, kk)
    for x, y in zip((out, cpool, spool), again):
        np.testing.assert_array_equal(x, y)
    ref_out, ref_cpool, ref_spool = _run_gdn_chain(hip_ctx, c, b, hk, hv, dd, kk)
    np.testing.assert_array_equal(out, ref_out)
    np.testing.assert_array_equal(cpool, ref_cpool)
    np.testing.assert_array_equal(spool, ref_spool)
    ch = (2 * hk + hv) * dd
    conv_elems, state_elems = ch * (kk - 1), hv * dd * dd
    g, beta = c["gate"], c["beta"]
    if prepare:
        g, beta = oracle.prepare_gdn_gate_beta(g, beta, c["dtb"], c["ssa"], b, hv)
    for i in range(b):
        co, so = int(c["coffs"][i]), int(c["soffs"][i])
        ci, new_conv = oracle.build_ssm_conv_state(c["conv_pool"][co:co + conv_elems],
                                                   c["qkv"][i * ch:(i + 1) * ch], kk, ch, 1)
        y = oracle.silu(oracle.ssm_conv(ci, c["w"], kk, ch, 1, 1))
        q, k, v = oracle.split_qkv_l2_norm(y, 1, hk, hv, dd, 1e-6)
        gl = slice(i * hv, (i + 1) * hv)
        yo, st = oracle.gated_delta_net(q, k, v, g[gl], beta[gl],
                                        c["state_pool"][so:so + state_elems], 1, hk, hv, dd)
        yo = oracle.norm_gated(yo, c["nw"], c["z"][i * hv * dd:(i + 1) * hv * dd], 1, hv, dd,
                               1e-6)
        np.testing.assert_allclose(out[i * hv * dd:(i + 1) * hv * dd], yo, rtol=0, atol=1e-4)
        np.testing.assert_array_equal(cpool[co:co + conv_elems], new_conv)
        np.testing.assert_allclose(spool[so:so + state_elems], st, rtol=0, atol=1e-4)


def test_ragged_gdn_layer_skips_out_of_pool_sequence(hip_ctx):
    """A sequence whose state offset is outside its pool is skipped by the one
    kernel: its output, conv state and state are untouched; the others match."""
    b, hk, hv, dd, kk = 4, 16, 16, 128, 4
    rng = np.random.default_rng(61)
    c = _gdn_layer_case(rng, b, hk, hv, dd, kk, True)
    good = dict(c)
    c["soffs"] = c["soffs"].copy()
    c["soffs"][2] = np.uint64(len(c["state_pool"]) + 5)
    out, cpool, spool = _run_gdn_layer(hip_ctx, c, b, hk, hv, dd, kk)
    ref_out, _, ref_spool = _run_gdn_layer(hip_ctx, good, b, hk, hv, dd, kk)
    d = hv * dd
    np.testing.assert_array_equal(out[2 * d:3 * d], 7.0)
    co = int(c["coffs"][2])
    conv_elems = (2 * hk + hv) * dd * (kk - 1)
    np.testing.assert_array_equal(cpool[co:co + conv_elems], c["conv_pool"][co:co + conv_elems])
    for i in (0, 1, 3):
        np.testing.assert_array_equal(out[i * d:(i + 1) * d], ref_out[i * d:(i + 1) * d])


def test_c4_block_two_steps_sampled_against_oracle(hip_ctx):
    """The C4 hybrid block as bench.py runs it: 64 sequences with the bench's KV
    lengths (512 + mt19937_64(4) mod 32257), each step three GDN layers (one
    launch each: conv prologue, prepared gate/beta, recurrence, norm-gated
    epilogue with a non-unit weight) and one full-attention layer (ragged K/V
    append, gated attention).  Two steps, so the second reads the conv and
    recurrent states and the K/V rows the first wrote.  Eight sequences
    (shortest, longest, six others) are replayed through the oracle chain and
    compared after every step: GDN outputs and states 1e-4, conv states and
    appended K/V rows exactly, attention 2e-3 rel / 1e-3 abs."""
    import bench

    rng = np.random.default_rng(44)
    b, layers, steps = 64, 3, 2
    hk = hv = 16
    dd, kk = 128, 4
    heads, kv_heads, d = 8, 2, 256
    ch = (2 * hk + hv) * dd
    kv_dim = kv_heads * d
    conv_elems, state_elems = ch * (kk - 1), hv * dd * dd
    lengths = np.array(bench.c4_lengths(), np.int64)
    kv_offsets, kv_total = scattered_offsets(rng, lengths + steps, kv_dim)
    block = 1 << 20
    kpool = np.resize(rng.standard_normal(block).astype(np.float16), kv_total)
    vpool = np.resize(rng.standard_normal(block + 8).astype(np.float16), kv_total)
    ctx = hip_ctx
    kb, vb = ctx.buffer(kpool.view(np.uint16)), ctx.buffer(vpool.view(np.uint16))
    kvo = ctx.buffer(kv_offsets)
    lay = []
    for l in range(layers):
        coffs, ctotal = scattered_offsets(rng, [1] * b, conv_elems, align=64)
        soffs, stotal = scattered_offsets(rng, [1] * b, state_elems, align=dd)
        c = dict(conv=rng.standard_normal(ctotal).astype(np.float32),
                 state=(0.1 * rng.standard_normal(stotal)).astype(np.float32),
                 w=(0.5 * rng.standard_normal(ch * kk)).astype(np.float32),
                 nw=(1 + 0.1 * rng.standard_normal(dd)).astype(np.float32),
                 dtb=rng.standard_normal(hv).astype(np.float32),
                 ssa=(-rng.random(hv)).astype(np.float32), coffs=coffs, soffs=soffs)
        c["dev"] = {k: ctx.buffer(c[k]) for k in ("conv", "state", "w", "nw", "dtb", "ssa",
                                                   "coffs", "soffs")}
        lay.append(c)
    pick = sorted({int(np.argmin(lengths)), int(np.argmax(lengths)), 5, 19, 33, 42, 57, 62})
    # Host copies the oracle advances for the sampled sequences.
    conv_ref = {(l, i): lay[l]["conv"][int(lay[l]["coffs"][i]):][:conv_elems].copy()
                for l in range(layers) for i in pick}
    state_ref = {(l, i): lay[l]["state"][int(lay[l]["soffs"][i]):][:state_elems].copy()
                 for l in range(layers) for i in pick}
    kv_rows = {i: (kpool[int(kv_offsets[i]):][:(int(lengths[i]) + steps) * kv_dim].copy(),
                   vpool[int(kv_offsets[i]):][:(int(lengths[i]) + steps) * kv_dim].copy())
               for i in pick}
    for s in range(steps):
        print(f"c4 block step {s}", flush=True)
        pos = (lengths + s).astype(np.uint32)
        inp = [dict(qkv=rng.standard_normal(b * ch).astype(np.float32),
                    gate=rng.standard_normal(b * hv).astype(np.float32),
                    beta=rng.standard_normal(b * hv).astype(np.float32),
                    z=rng.standard_normal(b * hv * dd).astype(np.float32))
               for _ in range(layers)]
        knew = rng.standard_normal(b * kv_dim).astype(np.float32)
        vnew = rng.standard_normal(b * kv_dim).astype(np.float32)
        aq = rng.standard_normal(b * heads * d).astype(np.float32)
        agate = rng.standard_normal(b * heads * d).astype(np.float32)
        outs = [ctx.buffer(byte_size=4 * b * hv * dd) for _ in range(layers)]
        aout = ctx.buffer(byte_size=4 * b * heads * d)
        posb = ctx.buffer(pos)
        dev_in = [{k: ctx.buffer(v) for k, v in x.items()} for x in inp]
        knb, vnb, aqb, agb = (ctx.buffer(x) for x in (knew, vnew, aq, agate))
        ctx.begin_graph()  # the block as one batch: one host wait per step
        for l in range(layers):
            dv, di = lay[l]["dev"], dev_in[l]
            ctx.qwen35_gdn_layer_ragged_decode_f32(
                di["qkv"], dv["conv"], dv["coffs"], dv["w"], kk, di["gate"], di["beta"],
                dv["dtb"], dv["ssa"], di["z"], dv["nw"], dv["state"], dv["soffs"], b, hk, hv, dd,
                1e-6, outs[l])
        ctx.append_kv_ragged_f16(knb, vnb, kb, vb, kvo, posb, b, kv_dim)
        ctx.attention_f32_ragged_f16_kv(aqb, kb, vb, agb, kvo, posb, b, int(pos.max()), heads,
                                        kv_heads, d, aout)
        ctx.commit_graph()
        got_out = [o.download() for o in outs]
        got_conv = [lay[l]["dev"]["conv"].download() for l in range(layers)]
        got_state = [lay[l]["dev"]["state"].download() for l in range(layers)]
        got_att = aout.download()
        for i in pick:
            for l in range(layers):
                g, be = oracle.prepare_gdn_gate_beta(inp[l]["gate"][i * hv:(i + 1) * hv],
                                                     inp[l]["beta"][i * hv:(i + 1) * hv],
                                                     lay[l]["dtb"], lay[l]["ssa"], 1, hv)
                ci, conv_ref[(l, i)] = oracle.build_ssm_conv_state(
                    conv_ref[(l, i)], inp[l]["qkv"][i * ch:(i + 1) * ch], kk, ch, 1)
                y = oracle.silu(oracle.ssm_conv(ci, lay[l]["w"], kk, ch, 1, 1))
                q, k, v = oracle.split_qkv_l2_norm(y, 1, hk, hv, dd, 1e-6)
                yo, state_ref[(l, i)] = oracle.gated_delta_net(q, k, v, g, be, state_ref[(l, i)],
                                                               1, hk, hv, dd)
                yo = oracle.norm_gated(yo, lay[l]["nw"], inp[l]["z"][i * hv * dd:][:hv * dd],
                                       1, hv, dd, 1e-6)
                msg = f"step {s} layer {l} sequence {i}"
                np.testing.assert_allclose(got_out[l][i * hv * dd:][:hv * dd], yo, rtol=0,
                                           atol=1e-4, err_msg=msg)
                co, so = int(lay[l]["coffs"][i]), int(lay[l]["soffs"][i])
                np.testing.assert_array_equal(got_conv[l][co:co + conv_elems], conv_ref[(l, i)],
                                              err_msg=msg)
                np.testing.assert_allclose(got_state[l][so:so + state_elems], state_ref[(l, i)],
                                           rtol=0, atol=1e-4, err_msg=msg)
            kc, vc = kv_rows[i]
            row = int(pos[i])
            kc[row * kv_dim:(row + 1) * kv_dim] = knew[i * kv_dim:(i + 1) * kv_dim]
            vc[row * kv_dim:(row + 1) * kv_dim] = vnew[i * kv_dim:(i + 1) * kv_dim]
            off = 2 * (int(kv_offsets[i]) + row * kv_dim)
            np.testing.assert_array_equal(kb.download(kv_dim, np.uint16, off), kc[
                row * kv_dim:(row + 1) * kv_dim].view(np.uint16))
            np.testing.assert_array_equal(vb.download(kv_dim, np.uint16, off), vc[
                row * kv_dim:(row + 1) * kv_dim].view(np.uint16))
            sl = slice(i * heads * d, (i + 1) * heads * d)
            ref = oracle.attention_batched(aq[sl], kc[:(row + 1) * kv_dim].view(np.uint16),
                                           vc[:(row + 1) * kv_dim].view(np.uint16), 0, row, 1,
                                           row + 1, heads, kv_heads, d)
            ref = oracle.sigmoid_gate_mul(ref, agate[sl])
            np.testing.assert_allclose(got_att[sl], ref, rtol=2e-3, atol=1e-3,
                                       err_msg=f"step {s} attention sequence {i}")
