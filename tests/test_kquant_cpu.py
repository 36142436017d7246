"""CPU tests of the K-quant and argmax entry points' argument checks, in the
reference's order and wording ("HIP" for "MPS"): make_q*_k_matvec_layout and
make_k_quant_matmul_layout (mps_backend.mm:4038-4189), the matvec / top1 /
argmax / matmul methods (:6134-6450 for Q4_K; Q5_K and Q6_K repeat them),
dequantize_row(s) (:7217-7380) and argmax_f32_i32 / argmax_prob_f32_i32
(:10004-10090).  The validation-only context runs every check and answers
`unavailable` instead of launching.
"""
import pytest

import kraken_hip as kh

ACCEPTED = "validation-only context: arguments accepted"
BLOCK = {"q4_k": 144, "q5_k": 176, "q6_k": 210}
NAME = {"q4_k": "Q4_K", "q5_k": "Q5_K", "q6_k": "Q6_K"}
FORMATS = tuple(BLOCK)


@pytest.fixture()
def vctx():
    ctx = kh.Context(validation_only=True)
    yield ctx
    ctx.close()


def fake(nbytes, address=0x1000):
    return kh.KrakenBuffer(address, nbytes)


def null(nbytes=0):
    return kh.KrakenBuffer(0, nbytes)


def status(ctx, name, *args):
    return ctx.status(name, *args), kh.last_error()


def wbytes(fmt, rows, cols):
    return rows * (cols // 256) * BLOCK[fmt]


def invalid(msg):
    return (kh.INVALID_ARGUMENT, msg)


# The Qwen3.5-0.8B projection shapes named for this row (rows x cols).
QWEN_SHAPES = [("q5_k", 6144, 1024), ("q4_k", 3584, 1024), ("q6_k", 1024, 3584),
               ("q4_k", 1024, 2048)]


@pytest.mark.parametrize("fmt,rows,cols", QWEN_SHAPES)
@pytest.mark.parametrize("tokens", [1, 4, 8, 9, 1024])
def test_matmul_accepts_qwen_shapes(vctx, fmt, rows, cols, tokens):
    args = (fake(wbytes(fmt, rows, cols)), rows, cols, tokens, fake(4 * tokens * cols),
            fake(4 * tokens * rows))
    assert status(vctx, f"matmul_{fmt}_f32_device", *args) == (kh.UNAVAILABLE, ACCEPTED)
    if tokens == 1:
        args = (fake(wbytes(fmt, rows, cols)), rows, cols, fake(4 * cols), fake(4 * rows))
        assert status(vctx, f"matvec_{fmt}_f32_device", *args) == (kh.UNAVAILABLE, ACCEPTED)


@pytest.mark.parametrize("fmt", FORMATS)
def test_matvec_check_order(vctx, fmt):
    n = NAME[fmt]
    op = f"matvec_{fmt}_f32_device"
    rows, cols = 32, 512
    w, x, y = fake(wbytes(fmt, rows, cols)), fake(4 * cols), fake(4 * rows)
    assert status(vctx, op, null(), rows, cols, x, y) == invalid(
        f"HIP {n} weight buffer is not initialized")
    assert status(vctx, op, w, 0, cols, x, y) == invalid(
        f"HIP {n} matvec rows and cols must be greater than zero")
    assert status(vctx, op, w, rows, 300, x, y) == invalid(
        f"HIP {n} matvec cols must be divisible by 256")
    assert status(vctx, op, w, rows, 256 << 32, x, y) == invalid(
        f"HIP {n} matvec cols exceeds uint32 range")
    assert status(vctx, op, w, 1 << 63, cols, x, y) == invalid(
        f"HIP {n} matvec block count overflow")
    assert status(vctx, op, fake(wbytes(fmt, rows, cols) - 1), rows, cols, x, y) == invalid(
        f"HIP {n} weight buffer is too small")
    code, msg = status(vctx, op, w, rows, cols, fake(4 * cols - 4), y)
    assert code == kh.INVALID_ARGUMENT and f"{n} matvec input" in msg
    code, msg = status(vctx, op, w, rows, cols, x, fake(4 * rows - 4))
    assert code == kh.INVALID_ARGUMENT and f"{n} matvec output" in msg
    # Beyond the reference: the device loads need aligned weights and inputs.
    code, msg = status(vctx, op, fake(wbytes(fmt, rows, cols) + 8, 0x1001), rows, cols, x, y)
    assert code == kh.INVALID_ARGUMENT and "aligned" in msg
    code, msg = status(vctx, op, w, rows, cols, fake(4 * cols, 0x1004), y)
    assert code == kh.INVALID_ARGUMENT and "16-byte aligned" in msg
    assert status(vctx, op, w, rows, cols, x, y) == (kh.UNAVAILABLE, ACCEPTED)


def test_q6_k_weight_needs_only_two_byte_alignment(vctx):
    rows, cols = 3, 256
    args = (fake(wbytes("q6_k", rows, cols), 0x1002), rows, cols, fake(4 * cols),
            fake(4 * rows))
    assert status(vctx, "matvec_q6_k_f32_device", *args) == (kh.UNAVAILABLE, ACCEPTED)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("kind", ["top1", "argmax"])
def test_top1_and_argmax_check_order(vctx, fmt, kind):
    n = NAME[fmt]
    op = f"matvec_{fmt}_f32_{kind}"
    rows, cols = 248320, 1024
    w, x, tok, prob = fake(wbytes(fmt, rows, cols)), fake(4 * cols), fake(4), fake(4)
    outs = (tok, prob) if kind == "top1" else (tok,)
    assert status(vctx, op, null(), rows, cols, x, *outs) == invalid(
        f"HIP {n} {kind} weight buffer is not initialized")
    assert status(vctx, op, w, rows, 100, x, *outs) == invalid(
        f"HIP {n} matvec cols must be divisible by 256")
    big = fake(wbytes(fmt, rows, 4352))
    assert status(vctx, op, big, rows, 4352, fake(4 * 4352), *outs) == invalid(
        f"HIP {n} {kind} block count exceeds kernel limit")
    assert status(vctx, op, fake(10), rows, cols, x, *outs) == invalid(
        f"HIP {n} {kind} weight buffer is too small")
    code, msg = status(vctx, op, w, rows, cols, fake(8), *outs)
    assert code == kh.INVALID_ARGUMENT and f"{n} {kind} input" in msg
    bad_tok = (null(), prob) if kind == "top1" else (null(),)
    code, msg = status(vctx, op, w, rows, cols, x, *bad_tok)
    assert code == kh.INVALID_ARGUMENT and f"{n} {kind} token output" in msg
    if kind == "top1":
        code, msg = status(vctx, op, w, rows, cols, x, tok, fake(2))
        assert code == kh.INVALID_ARGUMENT and f"{n} top1 probability output" in msg
    assert status(vctx, op, w, rows, cols, x, *outs) == (kh.UNAVAILABLE, ACCEPTED)
    # 4096 columns (16 blocks) is the largest row the top1 kernels take.
    assert status(vctx, op, fake(wbytes(fmt, 8, 4096)), 8, 4096, fake(4 * 4096),
                  *outs) == (kh.UNAVAILABLE, ACCEPTED)


@pytest.mark.parametrize("fmt", FORMATS)
def test_matmul_check_order(vctx, fmt):
    n = NAME[fmt]
    op = f"matmul_{fmt}_f32_device"
    rows, cols, tokens = 64, 512, 33
    w, x, y = fake(wbytes(fmt, rows, cols)), fake(4 * tokens * cols), fake(4 * tokens * rows)
    assert status(vctx, op, null(), rows, cols, tokens, x, y) == invalid(
        f"HIP {n} weight buffer is not initialized")
    assert status(vctx, op, w, rows, cols, 0, x, y) == invalid(
        f"HIP {n} matmul rows, cols and tokens must be greater than zero")
    assert status(vctx, op, w, rows, 257, tokens, x, y) == invalid(
        f"HIP {n} matmul cols must be divisible by 256")
    assert status(vctx, op, w, 1 << 33, cols, tokens, x, y) == invalid(
        f"HIP {n} matmul dimensions exceed uint32 range")
    assert status(vctx, op, w, rows, cols, 1 << 60, x, y) == invalid(
        f"HIP {n} matmul dimensions exceed uint32 range")
    assert status(vctx, op, fake(100), rows, cols, tokens, x, y) == invalid(
        f"HIP {n} matmul weight buffer is too small")
    code, msg = status(vctx, op, w, rows, cols, tokens, fake(4 * cols), y)
    assert code == kh.INVALID_ARGUMENT and f"{n} matmul input" in msg
    code, msg = status(vctx, op, w, rows, cols, tokens, x, fake(4 * rows))
    assert code == kh.INVALID_ARGUMENT and f"{n} matmul output" in msg
    assert status(vctx, op, w, rows, cols, tokens, x, y) == (kh.UNAVAILABLE, ACCEPTED)


@pytest.mark.parametrize("fmt", FORMATS)
def test_get_row_check_order(vctx, fmt):
    n = NAME[fmt]
    op = f"dequantize_row_{fmt}_f32"
    cols = 1024
    w, y = fake(wbytes(fmt, 10, cols)), fake(4 * cols)
    assert status(vctx, op, null(), 3, cols, y) == invalid(
        f"HIP {n} get-row weight buffer is not initialized")
    assert status(vctx, op, w, 3, 0, y) == invalid(
        f"HIP {n} get-row cols must be positive and divisible by 256")
    assert status(vctx, op, w, 2**64 - 1, cols, y) == invalid(
        f"HIP {n} get-row weight byte count overflow")
    assert status(vctx, op, w, 10, cols, y) == invalid(
        f"HIP {n} get-row weight buffer is too small")
    code, msg = status(vctx, op, w, 9, cols, fake(4))
    assert code == kh.INVALID_ARGUMENT and f"{n} get-row output" in msg
    assert status(vctx, op, w, 9, cols, y) == (kh.UNAVAILABLE, ACCEPTED)


@pytest.mark.parametrize("fmt", FORMATS)
def test_get_rows_check_order(vctx, fmt):
    n = NAME[fmt]
    op = f"dequantize_rows_{fmt}_f32"
    rows, tokens, cols = 10, 5, 512
    w, ids, y = fake(wbytes(fmt, rows, cols)), fake(4 * tokens), fake(4 * tokens * cols)
    assert status(vctx, op, null(), rows, ids, tokens, cols, y) == invalid(
        f"HIP {n} get-rows weight buffer is not initialized")
    assert status(vctx, op, w, rows, ids, 0, cols, y) == invalid(
        f"HIP {n} get-rows rows, tokens and cols must be positive and cols divisible by 256")
    assert status(vctx, op, w, 2**62, ids, tokens, cols, y) == invalid(
        f"HIP {n} get-rows weight byte count overflow")
    assert status(vctx, op, fake(20), rows, ids, tokens, cols, y) == invalid(
        f"HIP {n} get-rows weight buffer is too small")
    code, msg = status(vctx, op, w, rows, fake(4), tokens, cols, y)
    assert code == kh.INVALID_ARGUMENT and f"{n} get-rows row ids" in msg
    code, msg = status(vctx, op, w, rows, ids, tokens, cols, fake(16))
    assert code == kh.INVALID_ARGUMENT and f"{n} get-rows output" in msg
    assert status(vctx, op, w, rows, ids, tokens, cols, y) == (kh.UNAVAILABLE, ACCEPTED)


def test_argmax_check_order(vctx):
    v, tok, prob = fake(4 * 100), fake(4), fake(4)
    assert status(vctx, "argmax_f32_i32", v, 0, tok) == invalid("HIP argmax size must be positive")
    code, msg = status(vctx, "argmax_f32_i32", v, 1 << 33, tok)
    assert code == kh.INVALID_ARGUMENT and "argmax size" in msg
    code, msg = status(vctx, "argmax_f32_i32", fake(8), 100, tok)
    assert code == kh.INVALID_ARGUMENT and "argmax values" in msg
    assert status(vctx, "argmax_f32_i32", v, 100, null()) == invalid(
        "HIP argmax output buffer is not initialized")
    assert status(vctx, "argmax_f32_i32", v, 100, fake(2)) == invalid(
        "HIP argmax output buffer is too small")
    assert status(vctx, "argmax_f32_i32", v, 100, tok) == (kh.UNAVAILABLE, ACCEPTED)

    op = "argmax_prob_f32_i32"
    assert status(vctx, op, v, 0, tok, prob) == invalid(
        "HIP argmax probability size must be positive")
    code, msg = status(vctx, op, fake(8), 100, tok, prob)
    assert code == kh.INVALID_ARGUMENT and "argmax probability values" in msg
    assert status(vctx, op, v, 100, null(), prob) == invalid(
        "HIP argmax probability token output buffer is not initialized")
    assert status(vctx, op, v, 100, fake(3), prob) == invalid(
        "HIP argmax probability token output buffer is too small")
    code, msg = status(vctx, op, v, 100, tok, null())
    assert code == kh.INVALID_ARGUMENT and "argmax probability output" in msg
    assert status(vctx, op, v, 100, tok, prob) == (kh.UNAVAILABLE, ACCEPTED)
    # Vocabulary-sized inputs take the two-pass path (context workspace).
    assert status(vctx, op, fake(4 * 248320), 248320, tok, prob) == (kh.UNAVAILABLE, ACCEPTED)


# ------------------------------------------------------------ grouped matmul --
# kraken_hip_kquant_matmul_multi_f32: 1..4 matmuls sharing input, cols and
# tokens, each checked as its own matmul entry.
def _multi_matmul(vctx, types, rows, cols, tokens, outputs=None, weights=None):
    import ctypes
    n = len(types)
    fmts = {12: "q4_k", 13: "q5_k", 14: "q6_k"}
    t = (ctypes.c_uint32 * n)(*types)
    ws = (kh.KrakenBuffer * n)(*(weights or [fake(wbytes(fmts.get(ty, "q4_k"), r, cols))
                                             for ty, r in zip(types, rows)]))
    rs = (ctypes.c_size_t * n)(*rows)
    outs = (kh.KrakenBuffer * n)(*(outputs or [fake(4 * tokens * r) for r in rows]))
    return status(vctx, "kquant_matmul_multi_f32", n, t, ws, rs, cols, tokens,
                  fake(4 * tokens * cols), outs)


def test_multi_matmul_accepts_group_and_mixed_types(vctx):
    # The prefill's z / beta / alpha and FFN up / gate groups, and a mixed group.
    for types, rows in (([12, 12, 12], [2048, 16, 16]), ([12, 12], [3584, 3584]),
                        ([13, 12, 14], [6144, 2048, 16])):
        for tokens in (1, 8, 9, 1024):
            assert _multi_matmul(vctx, types, rows, 1024, tokens) == (kh.UNAVAILABLE, ACCEPTED)


def test_multi_matmul_checks(vctx):
    import ctypes
    assert _multi_matmul(vctx, [], [], 1024, 64) == invalid(
        "HIP K-quant multi matmul takes 1 to 4 matrices")
    assert _multi_matmul(vctx, [12] * 5, [16] * 5, 1024, 64) == invalid(
        "HIP K-quant multi matmul takes 1 to 4 matrices")
    assert status(vctx, "kquant_matmul_multi_f32", 1, None, None, None, 1024, 64,
                  fake(4 * 64 * 1024), None) == invalid(
        "HIP K-quant multi matmul array argument is null")
    assert _multi_matmul(vctx, [12, 2], [16, 16], 1024, 64) == invalid(
        "HIP K-quant multi matmul type must be Q4_K, Q5_K or Q6_K")
    # Each matrix's own matmul checks, in its own wording.
    code, msg = _multi_matmul(vctx, [12, 12], [16, 32], 1024, 64,
                              outputs=[fake(4 * 64 * 16), fake(4 * 64 * 16)])
    assert code == kh.INVALID_ARGUMENT and "Q4_K matmul output" in msg
    assert _multi_matmul(vctx, [12, 14], [16, 16], 1024, 64,
                         weights=[fake(wbytes("q4_k", 16, 1024)), fake(100)]) == invalid(
        "HIP Q6_K matmul weight buffer is too small")
    assert _multi_matmul(vctx, [12], [16], 1000, 64) == invalid(
        "HIP Q4_K matmul cols must be divisible by 256")


# -------------------------------------------------------------- fused matmul --
# kraken_hip_kquant_matmul_fused_f32: the matmul entry's checks, then its own.
def _fused(vctx, fmt="q6_k", rows=1024, cols=3584, tokens=64, up=True, residual=True, **over):
    w = over.get("w", fake(wbytes(fmt, rows, cols)))
    x = over.get("x", fake(4 * tokens * cols))
    u = over.get("upbuf", fake(4 * tokens * cols, 0x100000) if up else null())
    out = over.get("out", fake(4 * tokens * rows, 0x200000))
    r = over.get("resbuf", fake(4 * tokens * rows, 0x10000000) if residual else null())
    return status(vctx, "kquant_matmul_fused_f32", {"q4_k": 12, "q5_k": 13, "q6_k": 14}[fmt], w,
                  rows, cols, tokens, x, u, r, out)


def test_fused_matmul_accepts(vctx):
    for kw in ({}, dict(up=False), dict(residual=False), dict(up=False, residual=False),
               dict(fmt="q4_k", rows=1024, cols=2048), dict(fmt="q5_k", rows=6144, cols=1024),
               dict(tokens=9), dict(tokens=1024)):
        assert _fused(vctx, **kw) == (kh.UNAVAILABLE, ACCEPTED), kw
    # The residual may be the output itself.
    out = fake(4 * 64 * 1024, 0x200000)
    assert _fused(vctx, out=out, resbuf=out) == (kh.UNAVAILABLE, ACCEPTED)


def test_fused_matmul_checks(vctx):
    assert status(vctx, "kquant_matmul_fused_f32", 2, fake(100), 16, 256, 64, fake(4 * 64 * 256),
                  null(), null(), fake(4 * 64 * 16)) == invalid(
        "HIP K-quant fused matmul type must be Q4_K, Q5_K or Q6_K")
    assert _fused(vctx, w=fake(100)) == invalid("HIP Q6_K matmul weight buffer is too small")
    assert _fused(vctx, tokens=8) == invalid("HIP K-quant fused matmul needs more than 8 tokens")
    code, msg = _fused(vctx, upbuf=fake(4 * 64 * 3584 - 4, 0x100000))
    assert code == kh.INVALID_ARGUMENT and "K-quant fused matmul up" in msg
    assert _fused(vctx, upbuf=fake(4 * 64 * 3584, 0x100004)) == invalid(
        "HIP K-quant fused matmul up buffer must be 16-byte aligned")
    code, msg = _fused(vctx, resbuf=fake(4 * 64 * 1024 - 4, 0x10000000))
    assert code == kh.INVALID_ARGUMENT and "K-quant fused matmul residual" in msg
    assert _fused(vctx, resbuf=fake(4 * 64 * 1024, 0x10000004)) == invalid(
        "HIP K-quant fused matmul residual buffer must be 16-byte aligned")
    assert _fused(vctx, resbuf=fake(4 * 64 * 1024, 0x200000 + 4096)) == invalid(
        "HIP K-quant fused matmul residual overlaps the output")
