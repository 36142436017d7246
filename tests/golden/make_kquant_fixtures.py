"""Writes tests/golden/kquant_known_answers.json.

The cases are the K-quant and argmax known-answer checks of the reference's
smoke test, restated as data: the block bytes the test builds (as byte fills),
the call arguments and the values it asserts (tests/smoke_test.cpp:875-1149 for
Q4_K/Q5_K/Q6_K matvec, dequantize_row, two-token matmul, dequantize_rows and
the 65-row batched matmuls; :1614-1638 for argmax_f32_i32 and
argmax_prob_f32_i32).  The reference is not imported or run; the expected
values are the literals the test asserts (e.g. 384, 4480, -8192 and their
per-token multiples).  Tolerance: the test's assert_close, 1e-5 absolute
(smoke_test.cpp:432-438); the argmax probability uses the test's own 1e-4.

Run: python tests/golden/make_kquant_fixtures.py
"""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))

# One block of each format (smoke_test.cpp:875-880, 896-901, 918-921): byte
# ranges [start, end) and their value; everything else is zero.
BLOCKS = {
    "q4_k": {"bytes": 144, "fills": [[1, 2, 0x3C], [4, 16, 1], [16, 144, 0x21]]},
    "q5_k": {"bytes": 176, "fills": [[1, 2, 0x3C], [4, 16, 1], [16, 48, 0xFF], [48, 176, 0x21]]},
    "q6_k": {"bytes": 210, "fills": [[192, 208, 1], [209, 210, 0x3C]]},
}
BASE = {"q4_k": 384.0, "q5_k": 4480.0, "q6_k": -8192.0}
ROW = {  # dequantize_row: index -> value (smoke_test.cpp:890-894, 911-915, 931-935)
    "q4_k": {"0": 1.0, "31": 1.0, "32": 2.0, "255": 2.0},
    "q5_k": {"0": 17.0, "31": 17.0, "32": 18.0, "255": 18.0},
    "q6_k": {"0": -32.0, "127": -32.0, "128": -32.0, "255": -32.0},
}
ROWS2 = {  # dequantize_rows with row ids {1, 0} over two equal rows (:1022-1039)
    "q4_k": {"0": 1.0, "32": 2.0, "256": 1.0, "288": 2.0},
    "q5_k": {"0": 17.0, "32": 18.0, "256": 17.0, "288": 18.0},
    "q6_k": {"0": -32.0, "127": -32.0, "256": -32.0, "511": -32.0},
}


def main():
    cases = []
    for fmt in ("q4_k", "q5_k", "q6_k"):
        cases.append({"name": f"{fmt}_dequantize_row", "cite": "smoke_test.cpp:875-935",
                      "op": "dequantize_row", "format": fmt, "block": BLOCKS[fmt],
                      "args": {"rows": 1, "row": 0, "cols": 256}, "expected_at": ROW[fmt]})
        cases.append({"name": f"{fmt}_matvec", "cite": "smoke_test.cpp:886-929",
                      "op": "matvec", "format": fmt, "block": BLOCKS[fmt],
                      "args": {"rows": 1, "cols": 256, "tokens": 1},
                      "input": {"fill_per_token": [1.0]}, "expected": [BASE[fmt]]})
        cases.append({"name": f"{fmt}_matmul_two_tokens", "cite": "smoke_test.cpp:937-1021",
                      "op": "matmul", "format": fmt, "block": BLOCKS[fmt],
                      "args": {"rows": 1, "cols": 256, "tokens": 2},
                      "input": {"fill_per_token": [1.0, 2.0]},
                      "expected": [BASE[fmt], 2 * BASE[fmt]]})
        cases.append({"name": f"{fmt}_dequantize_rows_swapped", "cite": "smoke_test.cpp:981-1039",
                      "op": "dequantize_rows", "format": fmt, "block": BLOCKS[fmt],
                      "args": {"rows": 2, "tokens": 2, "cols": 256, "row_ids": [1, 0]},
                      "expected_at": ROWS2[fmt]})
        # 65 rows of the same block; token t's input is (t % 7) + 1 everywhere.
        for tokens, checked in ((4, [0, 3]), (5, [0, 4]), (6, [0, 5]), (33, [0, 31, 32])):
            expected_at = {}
            for t in checked:
                scale = float(t % 7 + 1)
                for r in (0, 63, 64):
                    expected_at[str(t * 65 + r)] = BASE[fmt] * scale
            cases.append({"name": f"{fmt}_matmul_65_rows_{tokens}_tokens",
                          "cite": "smoke_test.cpp:1041-1149", "op": "matmul", "format": fmt,
                          "block": BLOCKS[fmt],
                          "args": {"rows": 65, "cols": 256, "tokens": tokens},
                          "input": {"fill_per_token": [float(t % 7 + 1) for t in range(tokens)]},
                          "expected_at": expected_at})
    cases.append({"name": "argmax_f32_i32", "cite": "smoke_test.cpp:1614-1621",
                  "op": "argmax", "values": [-1.0, 5.0, 2.0], "expected_index": 1})
    cases.append({"name": "argmax_prob_f32_i32", "cite": "smoke_test.cpp:1622-1638",
                  "op": "argmax_prob", "values": [-1.0, 5.0, 2.0], "expected_index": 1,
                  "expected_probability": 0.950330, "probability_atol": 1e-4})
    out = {"source": "reference tests/smoke_test.cpp K-quant and argmax known answers, "
                     "transcribed", "atol": 1e-5, "cases": cases}
    with open(os.path.join(HERE, "kquant_known_answers.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
