"""Writes tests/golden/smoke_known_answers.json.

The cases are the known-answer checks of the reference's smoke test for the
hot-path operators (tests/smoke_test.cpp:1211-1725 of the reference), restated
as data: the inputs the test feeds, the call arguments, and the expected values
the test asserts, evaluated here from the same closed-form expressions the test
writes (e.g. `3.0F * norm_scale_34 * 2.0F`).  The reference is not imported or
run; this script only evaluates those expressions.  Tolerances are the test's
own (`assert_close` uses 1e-5 absolute, smoke_test.cpp:432-438; the
head_dim-128 GDN case uses 5e-5, smoke_test.cpp:1510-1517).

Run: python tests/golden/make_smoke_fixtures.py
"""
import json
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f32(x):
    return float(np.float32(x))


def sig(x):
    return 1.0 / (1.0 + math.exp(-x))


def silu(x):
    return x / (1.0 + math.exp(-x))


def gdn_d128_case():
    # smoke_test.cpp:1447-1517: inputs and the test's own fp32 CPU loop.
    tokens, d = 2, 128
    q = np.array([0.001 * (1 + i % 13) for i in range(tokens * d)], np.float32)
    k = np.array([0.0007 * (1 + i % 17) for i in range(tokens * d)], np.float32)
    v = np.array([0.01 * (1 + i % 19) for i in range(tokens * d)], np.float32)
    gate = np.zeros(tokens, np.float32)
    beta = np.array([0.75, 0.5], np.float32)
    state = np.array([0.0002 * (1 + i % 23) for i in range(d * d)], np.float32)
    s = state.copy()
    out = np.zeros(tokens * d, np.float32)
    one = np.float32(1.0)
    for t in range(tokens):
        ge = np.float32(math.exp(float(gate[t])))
        for r in range(d):
            sk = np.float32(0.0)
            for c in range(d):
                s[r * d + c] = np.float32(s[r * d + c] * ge)
                sk = np.float32(sk + s[r * d + c] * k[t * d + c])
            delta = np.float32((v[t * d + r] - sk) * beta[t])
            y = np.float32(0.0)
            for c in range(d):
                s[r * d + c] = np.float32(s[r * d + c] + k[t * d + c] * delta)
                y = np.float32(y + s[r * d + c] * q[t * d + c])
            out[t * d + r] = np.float32(y / np.float32(math.sqrt(d)) * one)
    # Arrays of this case are large, so they live in a compact .npz beside the JSON.
    np.savez_compressed(os.path.join(HERE, "gdn_head_dim_128.npz"), query=q, key=k, value=v,
                        gate=gate, beta=beta, state=state, expected_output=out,
                        expected_state=s)
    return {
        "name": "gdn_batched_head_dim_128",
        "cite": "smoke_test.cpp:1447-1517",
        "op": "gated_delta_net",
        "args": {"tokens": tokens, "key_heads": 1, "value_heads": 1, "head_dim": d},
        "npz": "gdn_head_dim_128.npz",
        "atol": 5e-5,
    }


def main():
    s34 = 1.0 / math.sqrt(12.5)
    cases = [
        {
            "name": "qk_norm_batched", "cite": "smoke_test.cpp:1211-1232",
            "op": "qk_norm_f32_batched",
            "args": {"tokens": 2, "heads": 1, "head_dim": 2, "eps": 0.0},
            "inputs": {"values": [1, 1, 3, 4], "weight": [2, 3]},
            "expected": {"values": [2, 3, 3 * s34 * 2, 4 * s34 * 3]},
        },
        {
            "name": "norm_gated", "cite": "smoke_test.cpp:1234-1246",
            "op": "norm_gated",
            "args": {"tokens": 2, "heads": 1, "head_dim": 2, "eps": 0.0},
            "inputs": {"values": [1, 1, 3, 4], "weight": [2, 3], "gate": [0, 1, -1, 2]},
            "expected": {"values": [0.0, 3 * silu(1.0), 3 * s34 * 2 * silu(-1.0),
                                    4 * s34 * 3 * silu(2.0)]},
        },
        {
            "name": "mrope_sections_1111", "cite": "smoke_test.cpp:1255-1273",
            "op": "mrope",
            "args": {"tokens": 1, "heads": 1, "head_dim": 8, "n_dims": 8,
                     "sections": [1, 1, 1, 1], "theta": 10000.0},
            "inputs": {"values": [1, 1, 1, 1, 0, 0, 0, 0], "positions": [1, 2, 3, 4]},
            "expected": {"values": [math.cos(1.0), math.cos(0.2), math.cos(0.03),
                                    math.cos(0.004), math.sin(1.0), math.sin(0.2),
                                    math.sin(0.03), math.sin(0.004)]},
        },
        {
            "name": "l2_norm", "cite": "smoke_test.cpp:1281-1287", "op": "l2_norm",
            "args": {"rows": 2, "row_size": 2, "eps": 0.0},
            "inputs": {"values": [3, 4, 0, 2]},
            "expected": {"values": [0.6, 0.8, 0.0, 1.0]},
        },
        {
            "name": "split_qkv_l2_norm", "cite": "smoke_test.cpp:1289-1328",
            "op": "split_qkv_l2_norm",
            "args": {"tokens": 2, "key_heads": 2, "value_heads": 2, "head_dim": 2, "eps": 0.0},
            "inputs": {"source": [3, 4, 0, 2, 5, 12, 8, 15, 1, 2, 3, 4,
                                  1, 0, 2, 0, 0, 6, 7, 24, 9, 10, 11, 12]},
            "expected": {"query": [0.6, 0.8, 0.0, 1.0, 1.0, 0.0, 1.0, 0.0],
                         "key": [5 / 13, 12 / 13, 8 / 17, 15 / 17, 0.0, 1.0, 7 / 25, 24 / 25],
                         "value": [1, 2, 3, 4, 9, 10, 11, 12]},
        },
        {
            "name": "ssm_conv", "cite": "smoke_test.cpp:1330-1342", "op": "ssm_conv",
            "args": {"conv_kernel": 4, "channels": 2, "tokens": 3, "sequences": 1},
            "inputs": {"input": [1, 2, 3, 4, 5, 6, 10, 20, 30, 40, 50, 60],
                       "kernel": [1, 0, 0, 0, 0, 1, 0, 0]},
            "expected": {"output": [1, 20, 2, 30, 3, 40]},
        },
        {
            "name": "ssm_conv1_stateful", "cite": "smoke_test.cpp:1344-1362",
            "op": "ssm_conv1_stateful",
            "args": {"conv_kernel": 4, "channels": 2},
            "inputs": {"state": [1, 2, 3, 10, 20, 30], "input": [4, 40],
                       "kernel": [1, 1, 1, 1, 0, 1, 0, 1]},
            "expected": {"output": [10, 60], "state": [2, 3, 4, 20, 30, 40]},
        },
        {
            "name": "build_ssm_conv_state_then_conv", "cite": "smoke_test.cpp:1364-1400",
            "op": "build_ssm_conv_state_then_conv",
            "args": {"conv_kernel": 4, "channels": 2, "tokens": 2},
            "inputs": {"state": [10, 20, 30, 40, 50, 60], "input": [1, 2, 3, 4],
                       "kernel": [1] * 8},
            "expected": {"conv_input": [10, 20, 30, 1, 3, 40, 50, 60, 2, 4],
                         "state": [30, 1, 3, 60, 2, 4],
                         "output": [61, 152, 54, 116]},
        },
        {
            "name": "gdn_single_token", "cite": "smoke_test.cpp:1402-1420",
            "op": "gated_delta_net",
            "args": {"tokens": 1, "key_heads": 1, "value_heads": 1, "head_dim": 2},
            "inputs": {"query": [1, 0], "key": [0.5, 0.25], "value": [10, 20], "gate": [0],
                       "beta": [1], "state": [1, 2, 3, 4]},
            "expected": {"output": [5.5 / math.sqrt(2), 11.75 / math.sqrt(2)],
                         "state": [5.5, 4.25, 11.75, 8.375]},
        },
        {
            "name": "gdn_batched_two_tokens", "cite": "smoke_test.cpp:1422-1445",
            "op": "gated_delta_net",
            "args": {"tokens": 2, "key_heads": 1, "value_heads": 1, "head_dim": 2},
            "inputs": {"query": [1, 0, 0, 1], "key": [0.5, 0.25, 0.25, 0.5],
                       "value": [10, 20, 1, 2], "gate": [0, 0], "beta": [1, 0.5],
                       "state": [1, 2, 3, 4]},
            "expected": {"output": [5.5 / math.sqrt(2), 11.75 / math.sqrt(2),
                                    3.625 / math.sqrt(2), 7.09375 / math.sqrt(2)],
                         "state": [5.1875, 3.625, 11.109375, 7.09375]},
        },
        gdn_d128_case(),
        {
            "name": "sigmoid", "cite": "smoke_test.cpp:1547-1551", "op": "sigmoid",
            "args": {}, "inputs": {"values": [-1, 0]},
            "expected": {"values": [1 / (1 + math.exp(1)), 0.5]},
        },
        {
            "name": "softplus", "cite": "smoke_test.cpp:1553-1557", "op": "softplus",
            "args": {}, "inputs": {"values": [0, 2]},
            "expected": {"values": [math.log(2.0), math.log(1 + math.exp(2.0))]},
        },
        {
            "name": "prepare_gdn_gate_beta", "cite": "smoke_test.cpp:1559-1576",
            "op": "prepare_gdn_gate_beta", "args": {"rows": 2, "row_size": 2},
            "inputs": {"gate": [0, 2, -1, 1], "beta": [-1, 0, 1, 2], "gate_bias": [0.5, -0.5],
                       "gate_scale": [2, -3]},
            "expected": {"gate": [math.log(1 + math.exp(0.5)) * 2, math.log(1 + math.exp(1.5)) * -3,
                                  math.log(1 + math.exp(-0.5)) * 2, math.log(1 + math.exp(0.5)) * -3],
                         "beta": [sig(-1), 0.5, sig(1), sig(2)]},
        },
        {
            "name": "silu", "cite": "smoke_test.cpp:1578-1582", "op": "silu", "args": {},
            "inputs": {"values": [0, 1]}, "expected": {"values": [0.0, sig(1.0)]},
        },
        {
            "name": "mul", "cite": "smoke_test.cpp:1526-1531", "op": "mul", "args": {},
            "inputs": {"target": [2, 3], "rhs": [4, 5]}, "expected": {"target": [8, 15]},
        },
        {
            "name": "copy_f32_rows", "cite": "smoke_test.cpp:1598-1612", "op": "copy_f32_rows",
            "args": {"rows": 3, "row_size": 2, "source_stride": 4, "source_offset": 1,
                     "destination_stride": 3, "destination_offset": 0},
            "inputs": {"source": list(range(12)), "destination": [-1] * 9},
            "expected": {"destination": [1, 2, -1, 5, 6, -1, 9, 10, -1]},
        },
        {
            "name": "attention_single_key", "cite": "smoke_test.cpp:1640-1649",
            "op": "attention", "kv": "f32",
            "args": {"layer": 0, "start_position": 0, "tokens": 1, "capacity_tokens": 1,
                     "heads": 1, "kv_heads": 1, "head_dim": 2},
            "inputs": {"query": [1, 0], "key_cache": [1, 0], "value_cache": [5, 6]},
            "expected": {"output": [5, 6]},
        },
        {
            "name": "attention_f16_kv_single_key", "cite": "smoke_test.cpp:1651-1666",
            "op": "attention", "kv": "f16",
            "args": {"layer": 0, "start_position": 0, "tokens": 1, "capacity_tokens": 1,
                     "heads": 1, "kv_heads": 1, "head_dim": 2},
            "inputs": {"query": [1, 0], "key_cache": [1, 0], "value_cache": [5, 6]},
            "expected": {"output": [5, 6]},
        },
        {
            "name": "attention_batched_causal_2x3", "cite": "smoke_test.cpp:1668-1686",
            "op": "attention", "kv": "f32",
            "args": {"layer": 0, "start_position": 1, "tokens": 2, "capacity_tokens": 3,
                     "heads": 1, "kv_heads": 1, "head_dim": 2},
            "inputs": {"query": [0, 0, 0, 0], "key_cache": [1, 0, 0, 1, 1, 1],
                       "value_cache": [5, 6, 7, 8, 9, 10]},
            "expected": {"output": [6, 7, 7, 8]},
        },
        {
            "name": "attention_zero_query_uniform_average", "cite": "smoke_test.cpp:1688-1725",
            "op": "attention", "kv": "f32",
            "args": {"layer": 0, "start_position": 0, "tokens": 16, "capacity_tokens": 16,
                     "heads": 1, "kv_heads": 1, "head_dim": 2},
            "inputs": {"query": [0] * 32, "key_cache": [0] * 32,
                       "value_cache": [x for t in range(16) for x in (t, t + 1)]},
            # The test asserts rows 0, 14 and 15; the closed form t/2, t/2+1 covers all rows.
            "expected": {"output": [x for t in range(16) for x in (t / 2, t / 2 + 1)]},
        },
    ]
    for case in cases:
        case.setdefault("atol", 1e-5)
    path = os.path.join(HERE, "smoke_known_answers.json")
    with open(path, "w") as f:
        json.dump({"source": "reference tests/smoke_test.cpp known answers, transcribed",
                   "cases": cases}, f, indent=1)
    print(f"wrote {len(cases)} cases to {path}")


if __name__ == "__main__":
    main()
