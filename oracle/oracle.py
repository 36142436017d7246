"""ctypes front end of the CPU oracle (oracle/kraken_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker.  Product code never imports it.

Every wrapper takes and returns numpy arrays in the reference's layouts and
mirrors one function of kraken_oracle.h (whose comments cite the reference
file:line each one restates).  Wrappers copy their inputs, so in-place
reference ops become "return the updated array" here.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "libkraken_oracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_sz = ctypes.c_size_t


def build() -> str:
    """Compile the oracle with its Makefile (plain gcc); returns the .so path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(l):
    l.oracle_f32_to_f16.restype = ctypes.c_uint16
    l.oracle_f32_to_f16.argtypes = [ctypes.c_float]
    l.oracle_f16_to_f32.restype = ctypes.c_float
    l.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    l.oracle_f32_to_f16_array.argtypes = [_f32p, _u16p, _sz]
    l.oracle_f16_to_f32_array.argtypes = [_u16p, _f32p, _sz]
    l.oracle_qk_norm_f32_batched.argtypes = [_f32p, _f32p, _sz, _sz, _sz, ctypes.c_float]
    l.oracle_norm_gated_f32.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz, ctypes.c_float]
    l.oracle_l2_norm_f32.argtypes = [_f32p, _sz, _sz, ctypes.c_float]
    l.oracle_split_qkv_l2_norm.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz,
                                           ctypes.c_float]
    l.oracle_gated_delta_net.argtypes = [_f32p] * 6 + [_sz] * 4 + [_f32p]
    l.oracle_ssm_conv.argtypes = [_f32p, _f32p, _sz, _sz, _sz, _sz, _f32p]
    l.oracle_ssm_conv1_stateful.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _f32p]
    l.oracle_build_ssm_conv_state.argtypes = [_f32p, _f32p, _sz, _sz, _sz, _f32p]
    l.oracle_mrope_f32.argtypes = [_f32p, _i32p] + [_sz] * 8 + [ctypes.c_float]
    l.oracle_make_mrope_positions.argtypes = [_i32p, _sz, _sz]
    for name in ("oracle_sigmoid_f32", "oracle_softplus_f32", "oracle_silu_f32"):
        getattr(l, name).argtypes = [_f32p, _sz]
    l.oracle_mul_f32.argtypes = [_f32p, _f32p, _sz]
    l.oracle_add_f32.argtypes = [_f32p, _f32p, _sz]
    l.oracle_silu_mul_f32.argtypes = [_f32p, _f32p, _sz]
    l.oracle_prepare_gdn_gate_beta.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz]
    l.oracle_copy_f32_rows.argtypes = [_f32p, _f32p] + [_sz] * 6
    l.oracle_copy_f32_rows_to_f16.argtypes = [_f32p, _u16p] + [_sz] * 6
    l.oracle_attention_batched.argtypes = [_f32p, ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_int] + [_sz] * 7 + [ctypes.c_int, _f32p]
    l.oracle_sigmoid_gate_mul.argtypes = [_f32p, _f32p, _sz]
    l.oracle_qwen3_qk_norm.argtypes = [_f32p, _sz, _sz, _f32p, ctypes.c_double]
    l.oracle_qwen3_rope.argtypes = [_f32p, _sz, _sz, _sz, ctypes.c_double]
    l.oracle_qwen3_attention.argtypes = [_f32p, _f32p, _sz, _sz, _sz, _f32p, _sz, _sz, _sz,
                                         _f32p]
    l.oracle_qwen3_attention_sequence.restype = ctypes.c_int
    l.oracle_qwen3_attention_sequence.argtypes = ([_f32p] * 3 + [_sz] * 4 + [_f32p, _f32p] +
                                                  [ctypes.c_double] * 2 + [_f32p] * 4)
    l.oracle_kquant_block_bytes.restype = _sz
    l.oracle_kquant_block_bytes.argtypes = [ctypes.c_int]
    l.oracle_kquant_dequantize.argtypes = [ctypes.c_int, ctypes.c_void_p, _sz, _f32p]
    l.oracle_kquant_matmul.argtypes = [ctypes.c_int, ctypes.c_void_p, _sz, _sz, _f32p, _sz,
                                       ctypes.c_int, ctypes.c_int, _f32p]
    l.oracle_argmax.restype = ctypes.c_int32
    l.oracle_argmax.argtypes = [_f32p, _sz, _f32p]


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32)).copy()


def _p(a: np.ndarray, t=_f32p):
    return a.ctypes.data_as(t)


# ---------------------------------------------------------------- f16 -----

def f32_to_f16_bits(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16_array(_p(x), _p(out, _u16p), x.size)
    return out


def f16_bits_to_f32(bits) -> np.ndarray:
    bits = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16)).copy()
    out = np.empty(bits.shape, dtype=np.float32)
    lib().oracle_f16_to_f32_array(_p(bits, _u16p), _p(out), bits.size)
    return out


# -------------------------------------------------------------- norms -----

def qk_norm_f32_batched(values, weight, tokens, heads, head_dim, eps):
    v = _f32(values)
    w = _f32(weight)
    lib().oracle_qk_norm_f32_batched(_p(v), _p(w), tokens, heads, head_dim, eps)
    return v


def norm_gated(values, weight, gate, tokens, heads, head_dim, eps):
    v, w, g = _f32(values), _f32(weight), _f32(gate)
    lib().oracle_norm_gated_f32(_p(v), _p(w), _p(g), tokens, heads, head_dim, eps)
    return v


def l2_norm(values, rows, row_size, eps):
    v = _f32(values)
    lib().oracle_l2_norm_f32(_p(v), rows, row_size, eps)
    return v


def split_qkv_l2_norm(source, tokens, key_heads, value_heads, head_dim, eps):
    s = _f32(source)
    q = np.zeros(tokens * key_heads * head_dim, np.float32)
    k = np.zeros_like(q)
    v = np.zeros(tokens * value_heads * head_dim, np.float32)
    lib().oracle_split_qkv_l2_norm(_p(s), _p(q), _p(k), _p(v), tokens, key_heads,
                                   value_heads, head_dim, eps)
    return q, k, v


# ---------------------------------------------------------------- gdn -----

def gated_delta_net(query, key, value, gate, beta, state, tokens, key_heads, value_heads,
                    head_dim):
    q, k, v, g, b, s = (_f32(x) for x in (query, key, value, gate, beta, state))
    out = np.zeros(tokens * value_heads * head_dim, np.float32)
    lib().oracle_gated_delta_net(_p(q), _p(k), _p(v), _p(g), _p(b), _p(s), tokens, key_heads,
                                 value_heads, head_dim, _p(out))
    return out, s


def ssm_conv(inp, kernel, conv_kernel, channels, tokens, sequences):
    x, w = _f32(inp), _f32(kernel)
    out = np.zeros(sequences * tokens * channels, np.float32)
    lib().oracle_ssm_conv(_p(x), _p(w), conv_kernel, channels, tokens, sequences, _p(out))
    return out


def ssm_conv1_stateful(state, inp, kernel, conv_kernel, channels):
    st, x, w = _f32(state), _f32(inp), _f32(kernel)
    out = np.zeros(channels, np.float32)
    lib().oracle_ssm_conv1_stateful(_p(st), _p(x), _p(w), conv_kernel, channels, _p(out))
    return out, st


def build_ssm_conv_state(state, inp, conv_kernel, channels, tokens):
    st, x = _f32(state), _f32(inp)
    ci = np.zeros(channels * (conv_kernel - 1 + tokens), np.float32)
    lib().oracle_build_ssm_conv_state(_p(st), _p(x), conv_kernel, channels, tokens, _p(ci))
    return ci, st


# --------------------------------------------------------------- rope -----

def mrope(values, positions, tokens, heads, head_dim, n_dims, sections, theta):
    v = _f32(values)
    pos = np.ascontiguousarray(np.asarray(positions, dtype=np.int32)).copy()
    s = list(sections)
    lib().oracle_mrope_f32(_p(v), _p(pos, _i32p), tokens, heads, head_dim, n_dims,
                           s[0], s[1], s[2], s[3], theta)
    return v


def make_mrope_positions(start_position, tokens):
    pos = np.zeros(4 * tokens, np.int32)
    lib().oracle_make_mrope_positions(_p(pos, _i32p), start_position, tokens)
    return pos


# -------------------------------------------------------- elementwise -----

def sigmoid(values):
    v = _f32(values)
    lib().oracle_sigmoid_f32(_p(v), v.size)
    return v


def softplus(values):
    v = _f32(values)
    lib().oracle_softplus_f32(_p(v), v.size)
    return v


def silu(values):
    v = _f32(values)
    lib().oracle_silu_f32(_p(v), v.size)
    return v


def prepare_gdn_gate_beta(gate, beta, gate_bias, gate_scale, rows, row_size):
    g, b, gb, gs = _f32(gate), _f32(beta), _f32(gate_bias), _f32(gate_scale)
    lib().oracle_prepare_gdn_gate_beta(_p(g), _p(b), _p(gb), _p(gs), rows, row_size)
    return g, b


def copy_f32_rows(source, destination, rows, row_size, source_stride, source_offset,
                  destination_stride, destination_offset):
    s, d = _f32(source), _f32(destination)
    lib().oracle_copy_f32_rows(_p(s), _p(d), rows, row_size, source_stride, source_offset,
                               destination_stride, destination_offset)
    return d


def copy_f32_rows_to_f16(source, destination_bits, rows, row_size, source_stride,
                         source_offset, destination_stride, destination_offset):
    s = _f32(source)
    d = np.ascontiguousarray(np.asarray(destination_bits, dtype=np.uint16)).copy()
    lib().oracle_copy_f32_rows_to_f16(_p(s), _p(d, _u16p), rows, row_size, source_stride,
                                      source_offset, destination_stride, destination_offset)
    return d


# ---------------------------------------------------------- attention -----

def attention_batched(query, key_cache, value_cache, layer, start_position, tokens,
                      capacity_tokens, heads, kv_heads, head_dim, round_query_f16=False):
    """key_cache/value_cache: uint16 arrays hold f16 bits (F16 KV); float32 is F32 KV."""
    q = _f32(query)
    kc = np.ascontiguousarray(key_cache)
    vc = np.ascontiguousarray(value_cache)
    kv_f16 = kc.dtype == np.uint16
    assert vc.dtype == kc.dtype and kc.dtype in (np.uint16, np.float32)
    out = np.zeros(tokens * heads * head_dim, np.float32)
    lib().oracle_attention_batched(_p(q), kc.ctypes.data_as(ctypes.c_void_p),
                                   vc.ctypes.data_as(ctypes.c_void_p), int(kv_f16), layer,
                                   start_position, tokens, capacity_tokens, heads, kv_heads,
                                   head_dim, int(bool(round_query_f16)), _p(out))
    return out


def sigmoid_gate_mul(output, gate):
    o, g = _f32(output), _f32(gate)
    lib().oracle_sigmoid_gate_mul(_p(o), _p(g), o.size)
    return o


# ------------------------------------------------------ legacy Qwen3 -----

def qwen3_qk_norm(values, heads, head_dim, weight, eps):
    v, w = _f32(values), _f32(weight)
    lib().oracle_qwen3_qk_norm(_p(v), heads, head_dim, _p(w), eps)
    return v


def qwen3_rope(values, heads, head_dim, position, theta):
    v = _f32(values)
    lib().oracle_qwen3_rope(_p(v), heads, head_dim, position, theta)
    return v


def qwen3_attention(key_cache, value_cache, capacity_tokens, layer, position, query, heads,
                    kv_heads, head_dim):
    kc, vc, q = _f32(key_cache), _f32(value_cache), _f32(query)
    out = np.zeros(heads * head_dim, np.float32)
    lib().oracle_qwen3_attention(_p(kc), _p(vc), capacity_tokens, layer, position, _p(q),
                                 heads, kv_heads, head_dim, _p(out))
    return out


def qwen3_attention_sequence(q_raw, k_raw, v_raw, positions, heads, kv_heads, head_dim,
                             q_norm_w, k_norm_w, eps, theta):
    """Returns (key_cache, value_cache, q_normed_roped, attention_out)."""
    q, k, v = _f32(q_raw), _f32(k_raw), _f32(v_raw)
    qw, kw = _f32(q_norm_w), _f32(k_norm_w)
    kc = np.zeros(positions * kv_heads * head_dim, np.float32)
    vc = np.zeros_like(kc)
    qo = np.zeros(positions * heads * head_dim, np.float32)
    out = np.zeros_like(qo)
    rc = lib().oracle_qwen3_attention_sequence(_p(q), _p(k), _p(v), positions, heads, kv_heads,
                                               head_dim, _p(qw), _p(kw), eps, theta, _p(kc),
                                               _p(vc), _p(qo), _p(out))
    assert rc == 0
    return kc, vc, qo, out


def mul(target, rhs):
    t, r = _f32(target), _f32(rhs)
    lib().oracle_mul_f32(_p(t), _p(r), t.size)
    return t


def add(target, delta):
    t, d = _f32(target), _f32(delta)
    lib().oracle_add_f32(_p(t), _p(d), t.size)
    return t


def silu_mul(gate, up):
    g, u = _f32(gate), _f32(up)
    lib().oracle_silu_mul_f32(_p(g), _p(u), g.size)
    return g


def rms_norm_batched(values, weight, tokens, size, eps):
    """rms_norm_f32_f32_batched (mps_backend.mm:1890-1920): the per-row RMSNorm
    with weight, which is qk_norm_f32_batched with one head of `size`."""
    return qk_norm_f32_batched(values, weight, tokens, 1, size, eps)


# ------------------------------------------------------------ K-quants -----
# Formats (oracle/kquant_oracle.c): GGUF Q4_K, Q5_K, Q6_K, 256 values per block.
KQUANT_FORMATS = {"q4_k": 0, "q5_k": 1, "q6_k": 2}
KQUANT_BLOCK_BYTES = {"q4_k": 144, "q5_k": 176, "q6_k": 210}


def _bytes(data) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(data, dtype=np.uint8)).copy()


def kquant_dequantize(fmt, data, blocks):
    """`blocks` consecutive blocks of format `fmt` -> 256 * blocks floats."""
    d = _bytes(data)
    assert d.size >= blocks * KQUANT_BLOCK_BYTES[fmt]
    out = np.empty(256 * blocks, np.float32)
    lib().oracle_kquant_dequantize(KQUANT_FORMATS[fmt], d.ctypes.data, blocks, _p(out))
    return out


def kquant_matmul(fmt, weight, rows, cols, x, tokens, weight_f16=False, input_f16=False):
    """out [tokens][rows] = W [rows][cols] (quantized rows) times x [tokens][cols]."""
    w = _bytes(weight)
    xx = _f32(x)
    assert cols % 256 == 0 and w.size >= rows * (cols // 256) * KQUANT_BLOCK_BYTES[fmt]
    assert xx.size >= tokens * cols
    out = np.empty(tokens * rows, np.float32)
    lib().oracle_kquant_matmul(KQUANT_FORMATS[fmt], w.ctypes.data, rows, cols, _p(xx), tokens,
                               int(weight_f16), int(input_f16), _p(out))
    return out


def argmax(values, probability=False):
    """argmax_f32_i32 (index) or argmax_prob_f32_i32 ((index, probability))."""
    v = _f32(values)
    p = np.zeros(1, np.float32)
    idx = int(lib().oracle_argmax(_p(v), v.size, _p(p) if probability else None))
    return (idx, float(p[0])) if probability else idx
