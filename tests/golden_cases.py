"""Loads the transcribed smoke-test known answers and runs them on a backend.

A backend is any object with the numpy-level functions of oracle/oracle.py
(`qk_norm_f32_batched`, `gated_delta_net`, `attention_batched`, ...).  The CPU
oracle and the HIP library's numpy front end (kraken_hip.NumpyOps) both
qualify, so the same cases pin the oracle on the CPU and check the HIP kernels
on the GPU.
"""
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_cases():
    with open(os.path.join(GOLDEN, "smoke_known_answers.json")) as f:
        cases = json.load(f)["cases"]
    for case in cases:
        if "npz" in case:
            data = np.load(os.path.join(GOLDEN, case["npz"]))
            case["inputs"] = {k: data[k] for k in data.files if not k.startswith("expected_")}
            case["expected"] = {k[len("expected_"):]: data[k] for k in data.files
                                if k.startswith("expected_")}
    return cases


def f16_bits(values):
    return np.asarray(values, np.float32).astype(np.float16).view(np.uint16)


def run_case(backend, case):
    """Returns {name: np.ndarray} for every key of case['expected']."""
    op, a, x = case["op"], case["args"], case["inputs"]
    if op == "qk_norm_f32_batched":
        return {"values": backend.qk_norm_f32_batched(x["values"], x["weight"], a["tokens"],
                                                      a["heads"], a["head_dim"], a["eps"])}
    if op == "norm_gated":
        return {"values": backend.norm_gated(x["values"], x["weight"], x["gate"], a["tokens"],
                                             a["heads"], a["head_dim"], a["eps"])}
    if op == "mrope":
        return {"values": backend.mrope(x["values"], x["positions"], a["tokens"], a["heads"],
                                        a["head_dim"], a["n_dims"], a["sections"], a["theta"])}
    if op == "l2_norm":
        return {"values": backend.l2_norm(x["values"], a["rows"], a["row_size"], a["eps"])}
    if op == "split_qkv_l2_norm":
        q, k, v = backend.split_qkv_l2_norm(x["source"], a["tokens"], a["key_heads"],
                                            a["value_heads"], a["head_dim"], a["eps"])
        return {"query": q, "key": k, "value": v}
    if op == "ssm_conv":
        return {"output": backend.ssm_conv(x["input"], x["kernel"], a["conv_kernel"],
                                           a["channels"], a["tokens"], a["sequences"])}
    if op == "ssm_conv1_stateful":
        out, st = backend.ssm_conv1_stateful(x["state"], x["input"], x["kernel"],
                                             a["conv_kernel"], a["channels"])
        return {"output": out, "state": st}
    if op == "build_ssm_conv_state_then_conv":
        ci, st = backend.build_ssm_conv_state(x["state"], x["input"], a["conv_kernel"],
                                              a["channels"], a["tokens"])
        out = backend.ssm_conv(ci, x["kernel"], a["conv_kernel"], a["channels"], a["tokens"], 1)
        return {"conv_input": ci, "state": st, "output": out}
    if op == "gated_delta_net":
        out, st = backend.gated_delta_net(x["query"], x["key"], x["value"], x["gate"],
                                          x["beta"], x["state"], a["tokens"], a["key_heads"],
                                          a["value_heads"], a["head_dim"])
        return {"output": out, "state": st}
    if op == "sigmoid":
        return {"values": backend.sigmoid(x["values"])}
    if op == "softplus":
        return {"values": backend.softplus(x["values"])}
    if op == "silu":
        return {"values": backend.silu(x["values"])}
    if op == "mul":
        return {"target": backend.mul(x["target"], x["rhs"])}
    if op == "prepare_gdn_gate_beta":
        g, b = backend.prepare_gdn_gate_beta(x["gate"], x["beta"], x["gate_bias"],
                                             x["gate_scale"], a["rows"], a["row_size"])
        return {"gate": g, "beta": b}
    if op == "copy_f32_rows":
        return {"destination": backend.copy_f32_rows(
            x["source"], x["destination"], a["rows"], a["row_size"], a["source_stride"],
            a["source_offset"], a["destination_stride"], a["destination_offset"])}
    if op == "attention":
        if case["kv"] == "f16":
            kc, vc = f16_bits(x["key_cache"]), f16_bits(x["value_cache"])
        else:
            kc = np.asarray(x["key_cache"], np.float32)
            vc = np.asarray(x["value_cache"], np.float32)
        return {"output": backend.attention_batched(
            x["query"], kc, vc, a["layer"], a["start_position"], a["tokens"],
            a["capacity_tokens"], a["heads"], a["kv_heads"], a["head_dim"])}
    raise KeyError(f"unknown golden op {op}")


def check_case(backend, case, atol=None):
    got = run_case(backend, case)
    tol = case["atol"] if atol is None else atol
    for key, expected in case["expected"].items():
        np.testing.assert_allclose(np.asarray(got[key], np.float64),
                                   np.asarray(expected, np.float64), rtol=0, atol=tol,
                                   err_msg=f"{case['name']}:{key} ({case['cite']})")
