"""Shared helpers for the K-quant tests: building the reference smoke test's
blocks from the golden fixture (tests/golden/kquant_known_answers.json), an
independent packer that writes GGUF K-quant blocks from chosen fields, and
random block generation."""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "kquant_known_answers.json")
BLOCK_BYTES = {"q4_k": 144, "q5_k": 176, "q6_k": 210}


def load():
    with open(GOLDEN) as f:
        return json.load(f)


def block_bytes(spec):
    b = np.zeros(spec["bytes"], np.uint8)
    for start, end, value in spec["fills"]:
        b[start:end] = value
    return b


def case_weight(case):
    """The case's weight: its block repeated over rows (one block per row)."""
    return np.tile(block_bytes(case["block"]), case["args"]["rows"])


def case_input(case):
    a = case["args"]
    fills = case["input"]["fill_per_token"]
    return np.repeat(np.asarray(fills, np.float32), a["cols"])


# ------------------------------------------------------------- packer ----
# Written from GGUF's k-quant layout as ggml's quantizers emit it (the inverse
# of the reads in oracle/kquant_oracle.c): it takes the fields a quantizer
# chooses and lays them out in bytes.

def _f16(x):
    return np.array([x], np.float16).view(np.uint8)


def pack_q4_q5(d, dmin, sc, m, q, five_bit):
    """d, dmin: floats (stored as f16); sc, m: 8 six-bit values per sub-block;
    q: 256 quants (0..15, or 0..31 with five_bit)."""
    s = np.zeros(12, np.uint8)
    for j in range(8):
        ls, lm = int(sc[j]), int(m[j])
        if j < 4:
            s[j] = ls
            s[j + 4] = lm
        else:
            s[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4)
            s[j - 4] |= (ls >> 4) << 6
            s[j] |= (lm >> 4) << 6
    qs = np.zeros(128, np.uint8)
    qh = np.zeros(32, np.uint8)
    m1, m2 = 1, 2
    for n in range(0, 256, 64):
        for j in range(32):
            l1, l2 = int(q[n + j]), int(q[n + j + 32])
            if five_bit:
                if l1 > 15:
                    l1 -= 16
                    qh[j] |= m1
                if l2 > 15:
                    l2 -= 16
                    qh[j] |= m2
            qs[n // 2 + j] = l1 | (l2 << 4)
        m1 <<= 2
        m2 <<= 2
    head = np.concatenate([_f16(d), _f16(dmin), s])
    return np.concatenate([head, qh, qs]) if five_bit else np.concatenate([head, qs])


def pack_q6(d, scales, q):
    """d: float (f16); scales: 16 int8; q: 256 quants 0..63 (value = q - 32)."""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for h in range(2):
        base = 128 * h
        for l in range(32):
            q1, q2 = int(q[base + l]), int(q[base + l + 32])
            q3, q4 = int(q[base + l + 64]), int(q[base + l + 96])
            ql[64 * h + l] = (q1 & 0xF) | ((q3 & 0xF) << 4)
            ql[64 * h + l + 32] = (q2 & 0xF) | ((q4 & 0xF) << 4)
            qh[32 * h + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    return np.concatenate([ql, qh, np.asarray(scales, np.int8).view(np.uint8), _f16(d)])


def expected_q4_q5(d, dmin, sc, m, q):
    """The values the fields stand for, in float32 with the reference's order
    of operations: (d * sc) * q - dmin * m."""
    f = np.float32
    out = np.empty(256, np.float32)
    dd, dm = f(np.float16(d)), f(np.float16(dmin))
    for i in range(256):
        sub = i // 32
        out[i] = f(f(dd * f(sc[sub])) * f(q[i])) - f(dm * f(m[sub]))
    return out


def expected_q6(d, scales, q):
    f = np.float32
    dd = f(np.float16(d))
    out = np.empty(256, np.float32)
    for i in range(256):
        out[i] = f(f(dd * f(scales[i // 16])) * f(int(q[i]) - 32))
    return out


def random_fields(fmt, rng):
    if fmt == "q6_k":
        return {"d": float(rng.uniform(0.001, 0.05)),
                "scales": rng.integers(-128, 128, 16), "q": rng.integers(0, 64, 256)}
    return {"d": float(rng.uniform(0.001, 0.05)), "dmin": float(rng.uniform(0.0, 0.05)),
            "sc": rng.integers(0, 64, 8), "m": rng.integers(0, 64, 8),
            "q": rng.integers(0, 32 if fmt == "q5_k" else 16, 256)}


def pack(fmt, fields):
    if fmt == "q6_k":
        return pack_q6(fields["d"], fields["scales"], fields["q"])
    return pack_q4_q5(fields["d"], fields["dmin"], fields["sc"], fields["m"], fields["q"],
                      fmt == "q5_k")


def expected(fmt, fields):
    if fmt == "q6_k":
        return expected_q6(fields["d"], fields["scales"], fields["q"])
    return expected_q4_q5(fields["d"], fields["dmin"], fields["sc"], fields["m"], fields["q"])


def random_weight(fmt, rows, cols, seed):
    """rows x cols weights: random blocks packed from random fields."""
    rng = np.random.default_rng(seed)
    blocks = rows * (cols // 256)
    return np.concatenate([pack(fmt, random_fields(fmt, rng)) for _ in range(blocks)])


def random_weight_fast(fmt, rows, cols, seed):
    """Large weights: random bytes with the f16 scale fields set to small
    positive values (every bit pattern of the other bytes is a valid block)."""
    rng = np.random.default_rng(seed)
    nb = BLOCK_BYTES[fmt]
    blocks = rows * (cols // 256)
    w = rng.integers(0, 256, size=(blocks, nb), dtype=np.uint8)
    d = rng.uniform(0.001, 0.02, size=blocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    if fmt == "q6_k":
        w[:, 208:210] = d
    else:
        w[:, 0:2] = d
        dm = rng.uniform(0.0, 0.02, size=blocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
        w[:, 2:4] = dm
    return w.reshape(-1)


def run_case(impl, case, gold):
    """Runs one known-answer case through `impl` (the oracle module or a device
    front end with the same function names) and checks it."""
    a = case.get("args", {})
    op = case["op"]
    if op in ("argmax", "argmax_prob"):
        if op == "argmax":
            assert impl.argmax(case["values"]) == case["expected_index"]
        else:
            idx, p = impl.argmax(case["values"], probability=True)
            assert idx == case["expected_index"]
            assert abs(p - case["expected_probability"]) < case["probability_atol"]
        return
    fmt = case["format"]
    w = case_weight(case)
    if op == "dequantize_row":
        got = impl.kquant_dequantize(fmt, w, a["cols"] // 256)
    elif op == "dequantize_rows":
        row_bytes = (a["cols"] // 256) * BLOCK_BYTES[fmt]
        got = np.concatenate([impl.kquant_dequantize(fmt, w[r * row_bytes:(r + 1) * row_bytes],
                                                     a["cols"] // 256) for r in a["row_ids"]])
    else:
        got = impl.kquant_matmul(fmt, w, a["rows"], a["cols"], case_input(case), a["tokens"])
    if "expected" in case:
        np.testing.assert_allclose(got, case["expected"], rtol=0, atol=gold["atol"])
    for index, value in case["expected_at"].items() if "expected_at" in case else []:
        assert abs(got[int(index)] - value) <= gold["atol"], (case["name"], index)
