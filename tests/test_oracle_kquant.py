"""The CPU oracle's K-quant dequantization, projections and argmax, pinned
before it judges the HIP kernels.

  * Known answers: the reference smoke test's blocks and asserted values
    (tests/golden/kquant_known_answers.json, smoke_test.cpp:875-1149, 1614-1638).
  * Round trip: blocks written by an independent packer (tests/kquant_cases.py,
    the layout as GGUF quantizers emit it) from random fields decode to exactly
    the values the fields stand for, bit for bit, so every scale/min bit field,
    nibble, high bit and sign is exercised.
  * Position: a block with a single non-zero quant decodes to a single
    non-trivial value at the documented index.
  * Projection: the oracle's matmul equals float64 numpy W @ x over the
    oracle's own dequantization, and with f16 rounding of both operands equals
    numpy on the rounded arrays.
  * argmax: first index of the maximum, NaN skipped, -inf selectable, empty
    candidate set -> size; probability = 1 / sum exp(v - max).
"""
import numpy as np
import pytest

import kquant_cases as kc
import oracle

GOLD = kc.load()
FORMATS = ("q4_k", "q5_k", "q6_k")


@pytest.mark.parametrize("case", GOLD["cases"], ids=[c["name"] for c in GOLD["cases"]])
def test_oracle_matches_smoke_known_answer(case):
    kc.run_case(oracle, case, GOLD)


def test_planted_nibble_swap_is_caught():
    """An oracle reading the high nibble first must fail the Q4_K known answer."""

    class Broken:
        @staticmethod
        def kquant_dequantize(fmt, data, blocks):
            y = oracle.kquant_dequantize(fmt, data, blocks).reshape(-1, 4, 2, 32)
            return y[:, :, ::-1, :].reshape(-1)

    case = next(c for c in GOLD["cases"] if c["name"] == "q4_k_dequantize_row")
    with pytest.raises(AssertionError):
        kc.run_case(Broken, case, GOLD)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("seed", range(6))
def test_round_trip_through_independent_packer(fmt, seed):
    rng = np.random.default_rng(100 + seed)
    fields = [kc.random_fields(fmt, rng) for _ in range(3)]
    data = np.concatenate([kc.pack(fmt, f) for f in fields])
    assert data.size == 3 * kc.BLOCK_BYTES[fmt]
    got = oracle.kquant_dequantize(fmt, data, 3)
    want = np.concatenate([kc.expected(fmt, f) for f in fields])
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("index", [0, 17, 31, 32, 63, 64, 100, 127, 128, 160, 191, 200, 255])
def test_single_quant_lands_at_its_index(fmt, index):
    """All quants at the zero point except one: only `index` differs."""
    if fmt == "q6_k":
        q = np.full(256, 32)
        q[index] = 32 + 5
        fields = {"d": 1.0, "scales": np.ones(16, np.int64), "q": q}
    else:
        q = np.zeros(256, np.int64)
        q[index] = 5 if fmt == "q4_k" else 21
        fields = {"d": 1.0, "dmin": 0.0, "sc": np.ones(8, np.int64), "m": np.zeros(8, np.int64),
                  "q": q}
    y = oracle.kquant_dequantize(fmt, kc.pack(fmt, fields), 1)
    nz = np.flatnonzero(y)
    assert nz.tolist() == [index]
    assert y[index] == (5 if fmt != "q5_k" else 21)


@pytest.mark.parametrize("fmt", FORMATS)
def test_matmul_equals_numpy_over_dequantized_rows(fmt):
    rows, cols, tokens = 5, 512, 3
    w = kc.random_weight(fmt, rows, cols, seed=7)
    x = np.random.default_rng(8).standard_normal(tokens * cols).astype(np.float32)
    dense = oracle.kquant_dequantize(fmt, w, rows * cols // 256).reshape(rows, cols)
    got = oracle.kquant_matmul(fmt, w, rows, cols, x, tokens).reshape(tokens, rows)
    want = x.reshape(tokens, cols).astype(np.float64) @ dense.astype(np.float64).T
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-5)
    got16 = oracle.kquant_matmul(fmt, w, rows, cols, x, tokens, weight_f16=True,
                                 input_f16=True).reshape(tokens, rows)
    want16 = (x.reshape(tokens, cols).astype(np.float16).astype(np.float64) @
              dense.astype(np.float16).astype(np.float64).T)
    np.testing.assert_allclose(got16, want16, rtol=1e-6, atol=1e-5)


def brute_argmax(v):
    best, best_v = len(v), -np.inf
    for i, x in enumerate(v):
        if x > best_v or (x == best_v and i < best):
            best, best_v = i, x
    return best


@pytest.mark.parametrize("values", [
    [3.0, 7.0, 7.0, 1.0],                      # tie: first index
    [np.nan, 2.0, np.nan, 2.0],                # NaN skipped
    [-np.inf, -np.inf],                        # -inf selectable: index 0
    [np.nan, np.nan],                          # no candidate: index = size
    [1e30, -1e30, 1e30],
    list(np.random.default_rng(0).standard_normal(1000)),
])
def test_argmax_rules(values):
    v = np.asarray(values, np.float32)
    assert oracle.argmax(v) == brute_argmax(v)
    idx, p = oracle.argmax(v, probability=True)
    assert idx == brute_argmax(v)
    finite = v[np.isfinite(v)]
    if np.isnan(v).any() or not np.isfinite(v).any():
        assert p == 0.0
    elif finite.size == v.size:
        want = 1.0 / np.exp(v.astype(np.float64) - v.max()).sum()
        assert abs(p - want) < 1e-6
