"""GPU parity of the K-quant projections, dequantization and argmax against
the CPU oracle (oracle/kquant_oracle.c, pinned in test_oracle_kquant.py).

Bars:
  * dequantize_row / dequantize_rows: bit-exact (the reference's arithmetic,
    operation for operation); row ids outside [0, rows) give zero rows.
  * matvec and matmul: within TOL * sum_k |w_k x_k| of the oracle's
    float64-accumulated product on the same operands, where the operands are
    what the reference multiplies for that token count: fp32 weights and
    inputs for 1-3 tokens (q*_k_matvec / q*_k_matmul, mps_backend.mm:
    284-460), fp16-rounded weights with fp32 inputs for 4-8 tokens
    (k_quant_mul_mv_ext_body, :889-960), fp16 weights and inputs for more
    (k_quant_mul_mm_simd_body, :1096-1230).  TOL = 1e-5 bounds fp32
    accumulation over the K <= 3584 products these shapes sum (about 70
    sequential roundings per lane plus a 6-level tree in the GEMV; 224 MFMA
    K-steps in the GEMM).
  * argmax: the index exactly; the probability within 1e-5 relative.

Weights are random blocks: packed from random fields (kquant_cases.pack) for
the small exact cases, random bytes with small positive f16 scales for the
Qwen3.5-0.8B projection shapes (every byte pattern is a valid block).
"""
import numpy as np
import pytest

import kquant_cases as kc
import kraken_hip as kh
import oracle

GOLD = kc.load()
FORMATS = ("q4_k", "q5_k", "q6_k")
TOL = 1e-5
# (format, rows, cols) of the Qwen3.5-0.8B projections this path serves.
QWEN = [("q5_k", 6144, 1024), ("q4_k", 3584, 1024), ("q6_k", 1024, 3584),
        ("q4_k", 1024, 2048)]


@pytest.fixture(scope="module")
def ops(hip_ctx):
    return kh.NumpyOps(hip_ctx)


def operands(tokens):
    """(weight_f16, input_f16) as the reference rounds them for `tokens`."""
    if tokens <= 3:
        return False, False
    if tokens <= 8:
        return True, False
    return True, True


def oracle_projection(fmt, w, rows, cols, x, tokens):
    """Oracle output [tokens * rows] and the bound scale sum |w x| per entry.
    Small products call oracle.kquant_matmul itself; large ones use the
    oracle's dequantization and a float64 product, which the oracle tests pin
    as equal to it (test_matmul_equals_numpy_over_dequantized_rows)."""
    wf16, xf16 = operands(tokens)
    dense = oracle.kquant_dequantize(fmt, w, rows * cols // 256).reshape(rows, cols)
    if wf16:
        dense = dense.astype(np.float16).astype(np.float32)
    xs = np.asarray(x, np.float32).reshape(tokens, cols)
    if xf16:
        xs = xs.astype(np.float16).astype(np.float32)
    if rows * tokens * cols <= 64 * 2**20:
        want = oracle.kquant_matmul(fmt, w, rows, cols, x, tokens, weight_f16=wf16,
                                    input_f16=xf16)
    else:
        want = (xs.astype(np.float64) @ dense.astype(np.float64).T).reshape(-1)
    scale = (np.abs(xs).astype(np.float64) @ np.abs(dense).astype(np.float64).T).reshape(-1)
    return want, scale


def check_projection(got, want, scale, msg):
    err = np.abs(got.astype(np.float64) - want)
    bound = TOL * scale + 1e-6
    worst = int(np.argmax(err / bound))
    assert np.all(err <= bound), (
        f"{msg}: index {worst} got {got[worst]} want {want[worst]} bound {bound[worst]}")


# ------------------------------------------------------------ known answers ----

@pytest.mark.gpu
@pytest.mark.parametrize("case", GOLD["cases"], ids=[c["name"] for c in GOLD["cases"]])
def test_smoke_known_answers(ops, case):
    """The reference smoke test's K-quant and argmax cases (smoke_test.cpp:
    875-1149, 1614-1638), on the device."""
    print(f"kquant known answer {case['name']}", flush=True)
    kc.run_case(ops, case, GOLD)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", FORMATS)
def test_smoke_dequantize_row_entry(ops, fmt):
    case = next(c for c in GOLD["cases"] if c["name"] == f"{fmt}_dequantize_row")
    got = ops.kquant_dequantize_row(fmt, kc.case_weight(case), 0, 256)
    for index, value in case["expected_at"].items():
        assert abs(got[int(index)] - value) <= GOLD["atol"]


# -------------------------------------------------------------- dequantize ----

@pytest.mark.gpu
@pytest.mark.parametrize("fmt", FORMATS)
def test_dequantize_rows_bit_exact(hip_ctx, ops, fmt):
    rows, cols = 37, 768  # 3 blocks per row: Q6_K rows start 2-byte aligned
    print(f"dequantize {fmt} {rows}x{cols}", flush=True)
    w = kc.random_weight(fmt, rows, cols, seed=11)
    dense = oracle.kquant_dequantize(fmt, w, rows * cols // 256).reshape(rows, cols)
    ids = np.array([5, 0, 36, -1, 37, 1000, 17, 5, 36], np.int32)
    wb = hip_ctx.buffer(w)
    idb = hip_ctx.buffer(ids)
    out = hip_ctx.buffer(byte_size=4 * ids.size * cols)
    getattr(hip_ctx, f"dequantize_rows_{fmt}_f32")(wb, rows, idb, ids.size, cols, out)
    got = out.download(ids.size * cols).reshape(ids.size, cols)
    for t, r in enumerate(ids):
        want = dense[r] if 0 <= r < rows else np.zeros(cols, np.float32)
        np.testing.assert_array_equal(got[t].view(np.uint32), want.view(np.uint32),
                                      err_msg=f"token {t} row {r}")
    for r in (0, 17, 36):
        row = ops.kquant_dequantize_row(fmt, w, r, cols)
        np.testing.assert_array_equal(row.view(np.uint32), dense[r].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("fmt,rows,cols", QWEN)
def test_dequantize_qwen_shapes_bit_exact(ops, fmt, rows, cols):
    w = kc.random_weight_fast(fmt, rows, cols, seed=rows + cols)
    got = ops.kquant_dequantize(fmt, w, rows * cols // 256)
    want = oracle.kquant_dequantize(fmt, w, rows * cols // 256)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------- projections ----

@pytest.mark.gpu
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("tokens", [1, 2, 3, 4, 5, 7, 8, 9, 33, 130])
def test_projection_token_counts(ops, fmt, tokens):
    """Every GEMV token grouping (1, 2, 4, 8 and their sums) and GEMM edge
    tiles (rows and tokens not multiples of 128) on packer-made blocks."""
    rows, cols = 77, 512
    print(f"projection {fmt} rows={rows} cols={cols} tokens={tokens}", flush=True)
    w = kc.random_weight(fmt, rows, cols, seed=tokens)
    x = np.random.default_rng(tokens).standard_normal(tokens * cols).astype(np.float32)
    got = ops.kquant_matmul(fmt, w, rows, cols, x, tokens)
    want, scale = oracle_projection(fmt, w, rows, cols, x, tokens)
    check_projection(got, want, scale, f"{fmt} T={tokens}")


@pytest.mark.gpu
@pytest.mark.parametrize("fmt,rows,cols", QWEN)
@pytest.mark.parametrize("tokens", [1, 8, 1024])
def test_projection_qwen_shapes(ops, fmt, rows, cols, tokens):
    print(f"projection {fmt} {rows}x{cols} T={tokens}", flush=True)
    w = kc.random_weight_fast(fmt, rows, cols, seed=rows + cols)
    x = np.random.default_rng(tokens + 5).standard_normal(tokens * cols).astype(np.float32)
    got = ops.kquant_matmul(fmt, w, rows, cols, x, tokens)
    want, scale = oracle_projection(fmt, w, rows, cols, x, tokens)
    check_projection(got, want, scale, f"{fmt} {rows}x{cols} T={tokens}")


@pytest.mark.gpu
def test_matvec_and_one_token_matmul_agree(hip_ctx, ops):
    """matvec_*_device and matmul_*_device at T=1 run the same kernel."""
    fmt, rows, cols = "q5_k", 6144, 1024
    w = kc.random_weight_fast(fmt, rows, cols, seed=3)
    x = np.random.default_rng(4).standard_normal(cols).astype(np.float32)
    a = ops.kquant_matmul(fmt, w, rows, cols, x, 1)
    wb, xb = hip_ctx.buffer(w), hip_ctx.buffer(x)
    out = hip_ctx.buffer(byte_size=4 * rows)
    hip_ctx.matmul_q5_k_f32_device(wb, rows, cols, 1, xb, out)
    np.testing.assert_array_equal(out.download(rows), a)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt,rows,cols,tokens", [q + (1024,) for q in QWEN] + [
    ("q4_k", 77, 512, 130), ("q5_k", 200, 768, 9), ("q6_k", 130, 1280, 257),
    ("q6_k", 16, 1024, 1024)])
def test_fused_gemm_equals_two_pass_gemm(ops, monkeypatch, fmt, rows, cols, tokens):
    """The GEMM that decodes the weights into its B tile (KRAKEN_KQUANT_GEMM=fused;
    the default for Q4_K) against the two-pass form (=unfused: an fp16 weight
    matrix written by the exact dequantization, then the fp16 GEMM; the default
    for Q5_K and Q6_K): the same fp16 weights and the same MFMA order over K, so
    the outputs are bit-identical; partial row and token tiles, odd block counts
    per row and 16-row tensors included."""
    print(f"fused gemm {fmt} {rows}x{cols} tokens={tokens}", flush=True)
    w = kc.random_weight_fast(fmt, rows, cols, seed=rows * 7 + cols)
    x = np.random.default_rng(tokens).standard_normal(tokens * cols).astype(np.float32)
    monkeypatch.setenv("KRAKEN_KQUANT_GEMM", "fused")
    fused = ops.kquant_matmul(fmt, w, rows, cols, x, tokens)
    monkeypatch.setenv("KRAKEN_KQUANT_GEMM", "unfused")
    two_pass = ops.kquant_matmul(fmt, w, rows, cols, x, tokens)
    np.testing.assert_array_equal(fused, two_pass)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt,rows,cols,tokens", [
    ("q5_k", 6144, 1024, 1024),   # 128 x 256 tiles
    ("q6_k", 6000, 1280, 1000),   # 128 x 256 tiles, partial row and token tiles
    ("q6_k", 1024, 3584, 1024),   # 128 x 128 tiles, four K splits of 14 steps
    ("q4_k", 1024, 2048, 1024),   # four K splits of 8 steps
    ("q5_k", 300, 256, 300),      # four K steps, fewer than the stages
    ("q4_k", 77, 512, 130), ("q5_k", 200, 768, 9)])
def test_pipelined_gemm_equals_plain_gemm(ops, monkeypatch, fmt, rows, cols, tokens):
    """The two-pass form's fp16 GEMM with direct-to-LDS copies through three or
    four stages (the default) against the kernel that prefetches one step into
    registers (KRAKEN_GEMM_F16=plain): same LDS layout and MFMA order over K,
    so bit-identical outputs."""
    print(f"pipelined gemm {fmt} {rows}x{cols} tokens={tokens}", flush=True)
    w = kc.random_weight_fast(fmt, rows, cols, seed=rows * 5 + cols)
    x = np.random.default_rng(tokens + 1).standard_normal(tokens * cols).astype(np.float32)
    monkeypatch.setenv("KRAKEN_KQUANT_GEMM", "unfused")
    piped = ops.kquant_matmul(fmt, w, rows, cols, x, tokens)
    monkeypatch.setenv("KRAKEN_GEMM_F16", "plain")
    plain = ops.kquant_matmul(fmt, w, rows, cols, x, tokens)
    np.testing.assert_array_equal(piped, plain)
    assert np.isfinite(piped).all()


# --------------------------------------------------------- grouped matmul ----
GGML = {"q4_k": 12, "q5_k": 13, "q6_k": 14}


@pytest.mark.gpu
@pytest.mark.parametrize("group,tokens", [
    ((("q4_k", 2048), ("q4_k", 16), ("q4_k", 16)), 1024),   # prefill z, beta, alpha
    ((("q4_k", 2048), ("q4_k", 16), ("q4_k", 16)), 9),
    ((("q4_k", 3584), ("q4_k", 3584)), 1024),                # FFN up, gate
    ((("q4_k", 130), ("q4_k", 300), ("q4_k", 16), ("q4_k", 1)), 200),  # ragged tiles
    ((("q5_k", 6144), ("q4_k", 2048)), 1024),                # mixed types: one call each
])
def test_multi_matmul_equals_single_matmuls(hip_ctx, ops, group, tokens):
    """kraken_hip_kquant_matmul_multi_f32 against each matrix's own matmul
    entry on the same input: bit-identical where the single call runs without a
    K split (the grouped launch never splits), else within TOL of the oracle
    like the single call (K split into planes sums in another order)."""
    print(f"multi matmul {group} tokens={tokens}", flush=True)
    cols = 1024
    x = np.random.default_rng(tokens).standard_normal(tokens * cols).astype(np.float32)
    ws = [kc.random_weight_fast(f, r, cols, seed=31 * i + r) for i, (f, r) in enumerate(group)]
    xb = hip_ctx.buffer(x)
    outs = [hip_ctx.buffer(byte_size=4 * tokens * r) for _, r in group]
    hip_ctx.kquant_matmul_multi([GGML[f] for f, _ in group], [hip_ctx.buffer(w) for w in ws],
                                [r for _, r in group], cols, tokens, xb, outs)
    for (f, r), w, ob in zip(group, ws, outs):
        got = ob.download(tokens * r)
        single = ops.kquant_matmul(f, w, r, cols, x, tokens)
        tiles = -(-r // 128) * -(-tokens // 128)
        if f == "q4_k" and tiles < 128 and tokens > 8:
            want, scale = oracle_projection(f, w, r, cols, x, tokens)
            check_projection(got, want, scale, f"{f} {r} rows")
        else:
            np.testing.assert_array_equal(got, single, err_msg=f"{f} {r} rows")


# ----------------------------------------------------------- fused matmul ----
@pytest.mark.gpu
@pytest.mark.parametrize("fmt,rows,cols", [("q6_k", 1024, 3584), ("q4_k", 1024, 2048),
                                           ("q4_k", 3584, 1024), ("q5_k", 6144, 1024)])
@pytest.mark.parametrize("tokens", [9, 1024])
def test_fused_matmul_equals_separate_ops(hip_ctx, fmt, rows, cols, tokens):
    """kraken_hip_kquant_matmul_fused_f32 against the ops it folds:
    silu_mul_f32_in_place(gate, up), the matmul entry, add_f32_in_place(residual,
    out).  Bit-identical with SwiGLU, with the residual (given as the output
    buffer itself, and as a separate buffer), with both and with neither, with
    and without K splits, in both GEMM forms."""
    print(f"fused matmul {fmt} {rows}x{cols} tokens={tokens}", flush=True)
    rng = np.random.default_rng(rows + tokens)
    w = hip_ctx.buffer(kc.random_weight_fast(fmt, rows, cols, seed=rows + cols))
    gate = rng.standard_normal(tokens * cols).astype(np.float32)
    up = rng.standard_normal(tokens * cols).astype(np.float32)
    res = rng.standard_normal(tokens * rows).astype(np.float32)
    ty = GGML[fmt]
    none = None
    for swiglu in (False, True):
        # The separate ops.
        g = hip_ctx.buffer(gate)
        if swiglu:
            hip_ctx.silu_mul_f32_in_place(g, hip_ctx.buffer(up), tokens * cols)
        plain = hip_ctx.buffer(byte_size=4 * tokens * rows)
        getattr(hip_ctx, f"matmul_{fmt}_f32_device")(w, rows, cols, tokens, g, plain)
        want_plain = plain.download(tokens * rows)
        summed = hip_ctx.buffer(res)
        hip_ctx.add_f32_in_place(summed, plain, tokens * rows)
        want_res = summed.download(tokens * rows)
        ub = hip_ctx.buffer(up) if swiglu else none
        # Folded: no residual; the residual as the output; a separate residual.
        out = hip_ctx.buffer(byte_size=4 * tokens * rows)
        hip_ctx.kquant_matmul_fused_f32(ty, w, rows, cols, tokens, hip_ctx.buffer(gate), ub, none,
                                        out)
        np.testing.assert_array_equal(out.download(tokens * rows).view(np.uint32),
                                      want_plain.view(np.uint32), err_msg=f"swiglu={swiglu}")
        inplace = hip_ctx.buffer(res)
        hip_ctx.kquant_matmul_fused_f32(ty, w, rows, cols, tokens, hip_ctx.buffer(gate), ub,
                                        inplace, inplace)
        np.testing.assert_array_equal(inplace.download(tokens * rows).view(np.uint32),
                                      want_res.view(np.uint32), err_msg=f"in place {swiglu}")
        out2 = hip_ctx.buffer(byte_size=4 * tokens * rows)
        hip_ctx.kquant_matmul_fused_f32(ty, w, rows, cols, tokens, hip_ctx.buffer(gate), ub,
                                        hip_ctx.buffer(res), out2)
        np.testing.assert_array_equal(out2.download(tokens * rows).view(np.uint32),
                                      want_res.view(np.uint32), err_msg=f"separate {swiglu}")


# ------------------------------------------------------------------ top1 ----

def planted_logit_weight(fmt, rows, cols, winner, seed):
    """Random blocks, with row `winner` made the clear maximum for an
    all-positive input: its blocks get a large scale and quants near the top."""
    w = kc.random_weight_fast(fmt, rows, cols, seed).reshape(rows, -1)
    nb = kc.BLOCK_BYTES[fmt]
    row = w[winner].reshape(-1, nb)
    if fmt == "q6_k":
        row[:, 0:128] = 0xFF          # low nibbles 15
        row[:, 128:192] = 0xFF        # high bits 3 -> q = 63
        row[:, 192:208] = 100         # int8 scales
        row[:, 208:210] = np.array([1.0], np.float16).view(np.uint8)
    else:
        row[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
        row[:, 2:4] = 0               # dmin 0
        row[:, 4:16] = 0x3F           # scales 63 (and the packed high bits)
        row[:, 16:nb] = 0xFF
    w[winner] = row.reshape(-1)
    return w.reshape(-1)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", FORMATS)
def test_top1_planted_winner_full_vocabulary(ops, fmt):
    """248320 rows (the Qwen3.5 vocabulary) x 1024: the planted row's logit
    exceeds every other row's by construction (>= 225 * 0.5 * 1024 against at
    most 0.02 * 127 * 31 * 1024), so the index is known without an oracle."""
    rows, cols = 248320, 1024
    winner = rows * 3 // 5
    print(f"top1 planted {fmt}", flush=True)
    w = planted_logit_weight(fmt, rows, cols, winner, seed=rows)
    x = np.random.default_rng(1).uniform(0.5, 1.0, cols).astype(np.float32)
    assert ops.kquant_top1(fmt, w, rows, cols, x) == winner
    idx, p = ops.kquant_top1(fmt, w, rows, cols, x, probability=True)
    assert idx == winner and p == 1.0


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows,cols", [(5, 256), (1000, 4096), (32768, 1024)])
def test_top1_random_logits(ops, fmt, rows, cols):
    """Random weights and input: the returned row's oracle logit is within
    the projection bound of the oracle maximum, and the probability within
    what that bound allows (p scales by at most exp(2 * bound))."""
    print(f"top1 random {fmt} rows={rows} cols={cols}", flush=True)
    w = kc.random_weight_fast(fmt, rows, cols, seed=rows + 1)
    x = np.random.default_rng(rows).standard_normal(cols).astype(np.float32)
    want, scale = oracle_projection(fmt, w, rows, cols, x, 1)
    bound = TOL * scale + 1e-6
    o_idx, o_p = oracle.argmax(want.astype(np.float32), probability=True)
    idx = ops.kquant_top1(fmt, w, rows, cols, x)
    idx2, p = ops.kquant_top1(fmt, w, rows, cols, x, probability=True)
    assert idx == idx2
    assert want[idx] >= want[o_idx] - bound[idx] - bound[o_idx], (idx, o_idx)
    slack = np.expm1(2.0 * bound.max()) + 1e-5
    assert abs(p - o_p) <= slack * o_p, (p, o_p)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows", [1000, 32768])
def test_top1_without_a_finite_logit_returns_row_zero(ops, fmt, rows):
    """When no logit exceeds -inf (an all-NaN input; or -inf in the input against
    all-positive weights, which gives -inf or NaN logits) the K-quant top-1 and
    argmax return token 0 with probability 0, as the reference's reduction does:
    it starts from index 0 at -inf and only a larger value or a smaller index at
    an equal value replaces it (mps_backend.mm:692-750, 1652-1690).  One pass
    (1000 rows) and two passes (32768 rows)."""
    cols = 256
    print(f"top1 no finite logit {fmt} rows={rows}", flush=True)
    w = np.concatenate([planted_logit_weight(fmt, 1, cols, 0, seed=rows)] * rows)
    for name, x in (("nan", np.full(cols, np.nan, np.float32)),
                    ("-inf", np.concatenate([[-np.inf], np.zeros(cols - 1)]).astype(np.float32))):
        assert ops.kquant_top1(fmt, w, rows, cols, x) == 0, name
        assert ops.kquant_top1(fmt, w, rows, cols, x, probability=True) == (0, 0.0), name


# ------------------------------------------------------------------ argmax ----

ARGMAX_SIZES = [3, 255, 16384, 16385, 248320]


@pytest.mark.gpu
@pytest.mark.parametrize("size", ARGMAX_SIZES)
def test_argmax_random(ops, size):
    v = np.random.default_rng(size).standard_normal(size).astype(np.float32) * 4
    assert ops.argmax(v) == oracle.argmax(v)
    idx, p = ops.argmax(v, probability=True)
    o_idx, o_p = oracle.argmax(v, probability=True)
    assert idx == o_idx
    assert abs(p - o_p) <= 1e-5 * o_p


@pytest.mark.gpu
@pytest.mark.parametrize("size", ARGMAX_SIZES)
def test_argmax_ties_nan_and_inf(ops, size):
    rng = np.random.default_rng(size + 1)
    v = rng.standard_normal(size).astype(np.float32)
    top = np.float32(9.0)
    ties = sorted(rng.choice(size, size=min(3, size), replace=False))
    v[ties] = top                                  # first of equal maxima wins
    cases = {"ties": v.copy()}
    w = v.copy()
    w[ties[0]] = np.nan                            # a NaN never wins
    cases["nan_at_max"] = w
    w = np.full(size, -np.inf, np.float32)          # all -inf: index 0
    cases["all_-inf"] = w
    w = np.full(size, np.nan, np.float32)           # no candidate: index = size
    cases["all_nan"] = w
    w = v.copy()
    w[: size // 2 + 1] = -np.inf                    # long -inf runs (masked vocab)
    w[-1] = 20.0
    cases["masked"] = w
    for name, values in cases.items():
        print(f"argmax {name} size={size}", flush=True)
        assert ops.argmax(values) == oracle.argmax(values), name
        idx, p = ops.argmax(values, probability=True)
        o_idx, o_p = oracle.argmax(values, probability=True)
        assert idx == o_idx, name
        assert abs(p - o_p) <= 1e-5 * abs(o_p) + 1e-12, (name, p, o_p)


# ------------------------------------------------------------ fused GEMV ----

GGML = {"q4_k": 12, "q5_k": 13, "q6_k": 14}


@pytest.mark.gpu
@pytest.mark.parametrize("fmt,rows,cols", QWEN + [("q4_k", 16, 1024), ("q6_k", 77, 256)])
@pytest.mark.parametrize("mode", ["norm", "swiglu", "plain"])
@pytest.mark.parametrize("residual", [False, True])
def test_fused_matvec_against_oracle_chain(hip_ctx, fmt, rows, cols, mode, residual):
    """kraken_hip_kquant_matvec_fused_f32 against the oracle's separate ops: the
    batched RMSNorm (or SwiGLU) of the input, the fp32 projection, the residual
    add; the bound is the projection's, on the transformed input."""
    rng = np.random.default_rng(rows + cols + len(mode) + residual)
    w = kc.random_weight_fast(fmt, rows, cols, seed=rows)
    x = (2 * rng.standard_normal(cols)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    up = rng.standard_normal(cols).astype(np.float32)
    res = rng.standard_normal(rows).astype(np.float32)
    xt = {"norm": lambda: oracle.rms_norm_batched(x, nw, 1, cols, 1e-6),
          "swiglu": lambda: oracle.silu_mul(x, up), "plain": lambda: x}[mode]()
    want, scale = oracle_projection(fmt, w, rows, cols, xt, 1)
    if residual:
        want = want + res
    none = None
    out = hip_ctx.buffer(res) if residual else hip_ctx.buffer(byte_size=4 * rows)
    hip_ctx.kquant_matvec_fused_f32(
        GGML[fmt], hip_ctx.buffer(w), rows, cols, hip_ctx.buffer(x),
        hip_ctx.buffer(nw) if mode == "norm" else none, 1e-6,
        hip_ctx.buffer(up) if mode == "swiglu" else none, out if residual else none, out)
    # The norm's scale is a float32 sum in another order: allow 1e-6 relative on it.
    check_projection(out.download(rows), want, scale * (1 + 2e-6 / TOL), f"{fmt} {mode}")


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", FORMATS)
def test_fused_top1_with_output_norm(hip_ctx, fmt):
    rows, cols = 32768, 1024
    rng = np.random.default_rng(9)
    w = kc.random_weight_fast(fmt, rows, cols, seed=rows + 2)
    x = (3 * rng.standard_normal(cols)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    xt = oracle.rms_norm_batched(x, nw, 1, cols, 1e-6)
    want, scale = oracle_projection(fmt, w, rows, cols, xt, 1)
    bound = TOL * scale + 1e-6
    tok = hip_ctx.buffer(np.array([-1], np.int32))
    prob = hip_ctx.buffer(np.array([-1], np.float32))
    hip_ctx.kquant_top1_fused_f32(GGML[fmt], hip_ctx.buffer(w), rows, cols, hip_ctx.buffer(x),
                                  hip_ctx.buffer(nw), 1e-6, tok, prob)
    idx = int(tok.download(1)[0])
    o_idx, o_p = oracle.argmax(want.astype(np.float32), probability=True)
    assert want[idx] >= want[o_idx] - bound[idx] - bound[o_idx]
    assert abs(float(prob.download(1)[0]) - o_p) <= (np.expm1(2 * bound.max()) + 1e-5) * o_p


@pytest.mark.gpu
@pytest.mark.parametrize("shapes", [
    [("q5_k", 6144), ("q4_k", 2048), ("q4_k", 16), ("q4_k", 16)],   # qkv, z, beta, alpha
    [("q4_k", 4096), ("q4_k", 512), ("q6_k", 512)],                 # q+gate, k, v
    [("q4_k", 3584), ("q4_k", 3584)],                               # ffn up, gate
    [("q6_k", 77)]])
@pytest.mark.parametrize("mode", ["norm", "swiglu"])
def test_multi_matvec_against_oracle_chain(hip_ctx, shapes, mode):
    """kraken_hip_kquant_matvec_multi_f32: each matrix of one launch against the
    oracle's transform and fp32 projection; the first matrix also adds a
    residual.  A bad count or width is rejected before launch."""
    cols = 1024
    rng = np.random.default_rng(len(shapes) + len(mode))
    x = (2 * rng.standard_normal(cols)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    up = rng.standard_normal(cols).astype(np.float32)
    xt = (oracle.rms_norm_batched(x, nw, 1, cols, 1e-6) if mode == "norm"
          else oracle.silu_mul(x, up))
    ws = [kc.random_weight_fast(f, r, cols, seed=r + i) for i, (f, r) in enumerate(shapes)]
    res = rng.standard_normal(shapes[0][1]).astype(np.float32)
    outs = [hip_ctx.buffer(res)] + [hip_ctx.buffer(byte_size=4 * r) for _, r in shapes[1:]]
    residuals = [outs[0]] + [None] * (len(shapes) - 1)
    none = None
    print(f"multi matvec {shapes} {mode}", flush=True)
    hip_ctx.kquant_matvec_multi(
        [GGML[f] for f, _ in shapes], [hip_ctx.buffer(w) for w in ws], [r for _, r in shapes],
        cols, hip_ctx.buffer(x), hip_ctx.buffer(nw) if mode == "norm" else none, 1e-6,
        hip_ctx.buffer(up) if mode == "swiglu" else none, residuals, outs)
    for i, ((f, r), w) in enumerate(zip(shapes, ws)):
        want, scale = oracle_projection(f, w, r, cols, xt, 1)
        if i == 0:
            want = want + res
        check_projection(outs[i].download(r), want, scale * (1 + 2e-6 / TOL), f"{f} {r} #{i}")


@pytest.mark.gpu
def test_multi_matvec_rejections(hip_ctx):
    w = hip_ctx.buffer(kc.random_weight_fast("q4_k", 16, 8192, seed=1))
    x = hip_ctx.buffer(np.ones(8192, np.float32))
    out = hip_ctx.buffer(byte_size=64)
    none = None
    with pytest.raises(kh.KrakenError, match="cols exceeds 4096"):
        hip_ctx.kquant_matvec_multi([12], [w], [16], 8192, x, none, 1e-6, none, [None], [out])
    with pytest.raises(kh.KrakenError, match="1 to 4 matrices"):
        hip_ctx.kquant_matvec_multi([12] * 5, [w] * 5, [16] * 5, 1024, x, none, 1e-6, none,
                                    [None] * 5, [out] * 5)
