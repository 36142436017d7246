"""ctypes binding of the C ABI in include/kraken_hip.h (libkraken_hip.so).

This is the Python side used by the tests and bench.py; C++ callers use the
header-only `kraken::hip::HipContext` in include/kraken/hip_context.hpp.
Device memory comes from the library's own `make_buffer` or from any object
exposing a device pointer and size (torch tensors included), passed as a
`kraken_buffer {data, byte_size}` view.

The library must be built (kraken-infer_amd/Makefile, or
__graft_entry__.build()); importing this module on a machine without the built
library raises immediately -- there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# KRAKEN_HIP_LIBRARY selects another build of the same library (e.g. an
# installed copy); the default is the in-tree build.
LIB_PATH = os.environ.get("KRAKEN_HIP_LIBRARY") or os.path.join(_HERE, "build",
                                                                "libkraken_hip.so")

OK, INVALID_ARGUMENT, UNAVAILABLE, INTERNAL_ERROR = 0, 1, 2, 3
STATUS_NAMES = {OK: "ok", INVALID_ARGUMENT: "invalid_argument", UNAVAILABLE: "unavailable",
                INTERNAL_ERROR: "internal_error"}


class KrakenBuffer(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("byte_size", ctypes.c_size_t)]


class KrakenError(RuntimeError):
    def __init__(self, code: int, message: str, op: str = ""):
        super().__init__(f"{op}: {STATUS_NAMES.get(code, code)}: {message}")
        self.code = code
        self.message = message


_sz = ctypes.c_size_t
_f = ctypes.c_float
_B = KrakenBuffer
_ctx = ctypes.c_void_p

# name -> argument types after the context pointer (all return int).
SIGNATURES = {
    "kraken_hip_attention_f32_batched_f16_kv": [_B, _B, _B] + [_sz] * 7 + [_B],
    "kraken_hip_attention_f16q_batched_f16_kv": [_B, _B, _B] + [_sz] * 7 + [_B],
    "kraken_hip_attention_f32_batched": [_B, _B, _B] + [_sz] * 7 + [_B],
    "kraken_hip_attention_f32_batched_f16_kv_gated": [_B, _B, _B, _B] + [_sz] * 7 + [_B],
    "kraken_hip_attention_f32_batched_f16_kv_gated_no_alloc": [_B, _B, _B, _B] + [_sz] * 7
                                                              + [_B],
    "kraken_hip_gated_delta_net_f32_batched_in_place_at": [_B] * 6 + [_sz] * 5 + [_B],
    "kraken_hip_gated_delta_net_f32_batched_in_place": [_B] * 6 + [_sz] * 4 + [_B],
    "kraken_hip_gated_delta_net_f32_in_place_at": [_B] * 6 + [_sz] * 4 + [_B],
    "kraken_hip_ssm_conv_f32": [_B, _B] + [_sz] * 4 + [_B],
    "kraken_hip_build_ssm_conv_state_f32": [_B, _sz, _B, _sz, _sz, _sz, _B],
    "kraken_hip_ssm_conv1_f32_stateful_at": [_B, _sz, _B, _B, _sz, _sz, _B],
    "kraken_hip_qwen35_conv_split_l2_f32": [_B, _B, _sz, _B] + [_sz] * 5 + [_f, _B, _B, _B],
    "kraken_hip_attention_f32_ragged_f16_kv": [_B] * 6 + [_sz] * 5 + [_B],
    "kraken_hip_append_kv_ragged_f16": [_B] * 6 + [_sz] * 2,
    "kraken_hip_gated_delta_net_f32_ragged_decode": [_B] * 7 + [_sz] * 4 + [_B],
    "kraken_hip_qwen35_conv_split_l2_ragged_decode_f32": [_B] * 4 + [_sz] * 5 + [_f, _B, _B, _B],
    "kraken_hip_qwen35_gdn_layer_ragged_decode_f32": [_B] * 4 + [_sz] + [_B] * 8 + [_sz] * 4
                                                     + [_f, _B],
    "kraken_hip_qwen35_gdn_state_ragged_decode_f32": [_B] * 9 + [_sz] * 4 + [_f, _B, _B],
    "kraken_hip_qwen35_gdn_gated_f32": [_B] * 10 + [_sz] * 5 + [_f, _B],
    "kraken_hip_split_qkv_l2_norm_f32_qwen35": [_B] * 4 + [_sz] * 4 + [_f],
    "kraken_hip_l2_norm_f32_in_place": [_B, _sz, _sz, _f],
    "kraken_hip_qk_norm_f32_f32_batched": [_B, _B, _sz, _sz, _sz, _f],
    "kraken_hip_qwen35_norm_gated_f32_in_place": [_B, _B, _B, _sz, _sz, _sz, _f],
    "kraken_hip_prepare_qwen35_gdn_gate_beta_f32": [_B] * 4 + [_sz, _sz],
    "kraken_hip_mrope_f32_in_place": [_B, _B] + [_sz] * 8 + [_f],
    "kraken_hip_qwen35_attention_prologue_f16_kv": [_B] * 6 + [_sz, _B, _B] + [_sz] * 12
                                                   + [_f, _f, _B, _B],
    "kraken_hip_qwen35_attention_prologue_gated_f16_kv": [_B] * 6 + [_sz, _B, _B] + [_sz] * 12
                                                         + [_f, _f, _B, _B, _B],
    "kraken_hip_copy_f32_rows_to_f16": [_B, _B] + [_sz] * 6,
    "kraken_hip_copy_f32_rows": [_B, _B] + [_sz] * 6,
    "kraken_hip_copy_f16_rows": [_B, _B] + [_sz] * 6,
    "kraken_hip_sigmoid_f32_in_place": [_B, _sz],
    "kraken_hip_softplus_f32_in_place": [_B, _sz],
    "kraken_hip_silu_f32_in_place": [_B, _sz],
    "kraken_hip_mul_f32_in_place": [_B, _B, _sz],
    "kraken_hip_add_f32_row_in_place": [_B, _B, _sz, _sz],
    "kraken_hip_mul_f32_row_in_place": [_B, _B, _sz, _sz],
    "kraken_hip_add_f32_in_place": [_B, _B, _sz],
    "kraken_hip_silu_mul_f32_in_place": [_B, _B, _sz],
    "kraken_hip_rms_norm_f32_f32_batched": [_B, _B, _sz, _sz, _f, _B],
    "kraken_hip_matvec_q4_k_f32_device": [_B, _sz, _sz, _B, _B],
    "kraken_hip_matvec_q4_k_f32_top1": [_B, _sz, _sz, _B, _B, _B],
    "kraken_hip_matvec_q4_k_f32_argmax": [_B, _sz, _sz, _B, _B],
    "kraken_hip_matmul_q4_k_f32_device": [_B, _sz, _sz, _sz, _B, _B],
    "kraken_hip_dequantize_row_q4_k_f32": [_B, _sz, _sz, _B],
    "kraken_hip_dequantize_rows_q4_k_f32": [_B, _sz, _B, _sz, _sz, _B],
    "kraken_hip_matvec_q5_k_f32_device": [_B, _sz, _sz, _B, _B],
    "kraken_hip_matvec_q5_k_f32_top1": [_B, _sz, _sz, _B, _B, _B],
    "kraken_hip_matvec_q5_k_f32_argmax": [_B, _sz, _sz, _B, _B],
    "kraken_hip_matmul_q5_k_f32_device": [_B, _sz, _sz, _sz, _B, _B],
    "kraken_hip_dequantize_row_q5_k_f32": [_B, _sz, _sz, _B],
    "kraken_hip_dequantize_rows_q5_k_f32": [_B, _sz, _B, _sz, _sz, _B],
    "kraken_hip_matvec_q6_k_f32_device": [_B, _sz, _sz, _B, _B],
    "kraken_hip_matvec_q6_k_f32_top1": [_B, _sz, _sz, _B, _B, _B],
    "kraken_hip_matvec_q6_k_f32_argmax": [_B, _sz, _sz, _B, _B],
    "kraken_hip_matmul_q6_k_f32_device": [_B, _sz, _sz, _sz, _B, _B],
    "kraken_hip_dequantize_row_q6_k_f32": [_B, _sz, _sz, _B],
    "kraken_hip_dequantize_rows_q6_k_f32": [_B, _sz, _B, _sz, _sz, _B],
    "kraken_hip_kquant_matvec_fused_f32": [ctypes.c_uint32, _B, _sz, _sz, _B, _B, _f, _B, _B, _B],
    "kraken_hip_kquant_top1_fused_f32": [ctypes.c_uint32, _B, _sz, _sz, _B, _B, _f, _B, _B],
    "kraken_hip_kquant_matmul_fused_f32": [ctypes.c_uint32, _B, _sz, _sz, _sz, _B, _B, _B, _B],
    "kraken_hip_kquant_matmul_multi_f32": [_sz, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                           _sz, _sz, _B, ctypes.c_void_p],
    "kraken_hip_kquant_matvec_multi_f32": [_sz, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                           _sz, _B, _B, _f, _B, ctypes.c_void_p,
                                           ctypes.c_void_p],
    "kraken_hip_kquant_matvec_multi_conv_f32": [_sz, ctypes.c_void_p, ctypes.c_void_p,
                                                ctypes.c_void_p, _sz, _B, _B, _f,
                                                ctypes.c_void_p, _B, _B, _B, _sz],
    "kraken_hip_kquant_matvec_head_norm_f32": [ctypes.c_uint32, _B, _sz, _sz, _B, _B, _sz, _f,
                                               _B, _B],
    "kraken_hip_argmax_f32_i32": [_B, _sz, _B],
    "kraken_hip_argmax_prob_f32_i32": [_B, _sz, _B, _B],
    "kraken_hip_begin_graph": [],
    "kraken_hip_commit_graph": [],
    "kraken_hip_make_buffer": [_sz, ctypes.POINTER(_B)],
    "kraken_hip_free_buffer": [ctypes.POINTER(_B)],
    "kraken_hip_copy_to_buffer": [_B, ctypes.c_void_p, _sz],
    "kraken_hip_copy_to_buffer_at": [_B, _sz, ctypes.c_void_p, _sz],
    "kraken_hip_copy_from_buffer": [_B, ctypes.c_void_p, _sz],
    "kraken_hip_copy_from_buffer_at": [_B, _sz, ctypes.c_void_p, _sz],
    "kraken_hip_copy_buffer_region": [_B, _B, _sz, _sz, _sz],
    "kraken_hip_zero_buffer": [_B, _sz],
    "kraken_hip_copy_regions": [_B, _B, ctypes.c_void_p, _sz],
    "kraken_hip_context_set_stream": [ctypes.c_void_p],
}

# Measurement aids (include/kraken_hip_diag.h), in libkraken_hip_diag.so.
DIAG_SIGNATURES = {
    "kraken_hip_diag_stream_read": [_B, _sz, _B],
    "kraken_hip_diag_mfma_f16": [ctypes.c_uint32, ctypes.c_uint32, _B],
    "kraken_hip_diag_mfma_f16_denormals": [_B],
}
DIAG_LIB_PATH = os.path.join(os.path.dirname(LIB_PATH), "libkraken_hip_diag.so")

_lib = None
_diag = None


def lib():
    """Loads libkraken_hip.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C kraken-infer_amd` or "
                "`python -c 'import __graft_entry__ as g; g.build()'`")
        l = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [_ctx] + args
        l.kraken_hip_context_create.restype = ctypes.c_int
        l.kraken_hip_context_create.argtypes = [ctypes.POINTER(_ctx)]
        l.kraken_hip_context_create_validation_only.restype = ctypes.c_int
        l.kraken_hip_context_create_validation_only.argtypes = [ctypes.POINTER(_ctx)]
        l.kraken_hip_context_destroy.restype = None
        l.kraken_hip_context_destroy.argtypes = [_ctx]
        l.kraken_hip_abort_graph.restype = None
        l.kraken_hip_abort_graph.argtypes = [_ctx]
        l.kraken_hip_context_stream.restype = ctypes.c_void_p
        l.kraken_hip_context_stream.argtypes = [_ctx]
        l.kraken_hip_last_error.restype = ctypes.c_char_p
        l.kraken_hip_last_error.argtypes = []
        _lib = l
    return _lib


def diag_lib():
    """Loads the measurement-probe library (bench.py and its tests only)."""
    global _diag
    if _diag is None:
        lib()
        if not os.path.exists(DIAG_LIB_PATH):
            raise RuntimeError(f"{DIAG_LIB_PATH} is missing: build it with `make -C kraken-infer_amd`")
        d = ctypes.CDLL(DIAG_LIB_PATH)
        for name, args in DIAG_SIGNATURES.items():
            fn = getattr(d, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [_ctx] + args
        d.kraken_hip_diag_last_error.restype = ctypes.c_char_p
        d.kraken_hip_diag_last_error.argtypes = []
        _diag = d
    return _diag


def last_error() -> str:
    return lib().kraken_hip_last_error().decode()


def as_buffer(obj) -> KrakenBuffer:
    """kraken_buffer view of a DeviceBuffer, a torch tensor, a (ptr, bytes) pair or None."""
    if obj is None:
        return KrakenBuffer(None, 0)
    if isinstance(obj, KrakenBuffer):
        return obj
    if isinstance(obj, DeviceBuffer):
        return obj.view
    if isinstance(obj, tuple):
        return KrakenBuffer(obj[0], obj[1])
    if hasattr(obj, "data_ptr") and hasattr(obj, "element_size"):  # torch.Tensor
        return KrakenBuffer(obj.data_ptr(), obj.numel() * obj.element_size())
    raise TypeError(f"cannot make a kraken_buffer from {type(obj)}")


class DeviceBuffer:
    """Device allocation owned through the context (make_buffer / free_buffer)."""

    def __init__(self, ctx: "Context", byte_size: int, dtype=np.float32):
        self.ctx = ctx
        self.dtype = np.dtype(dtype)
        self.view = KrakenBuffer()
        ctx._check("kraken_hip_make_buffer", lib().kraken_hip_make_buffer(
            ctx.handle, byte_size, ctypes.byref(self.view)))

    @property
    def byte_size(self) -> int:
        return self.view.byte_size

    def free(self):
        if self.view.data:
            lib().kraken_hip_free_buffer(self.ctx.handle, ctypes.byref(self.view))

    def upload(self, array, offset_bytes: int = 0):
        a = np.ascontiguousarray(array)
        self.ctx._check("kraken_hip_copy_to_buffer_at", lib().kraken_hip_copy_to_buffer_at(
            self.ctx.handle, self.view, offset_bytes, a.ctypes.data, a.nbytes))
        return self

    def download(self, count: int | None = None, dtype=None, offset_bytes: int = 0) -> np.ndarray:
        dt = np.dtype(dtype) if dtype is not None else self.dtype
        n = count if count is not None else (self.byte_size - offset_bytes) // dt.itemsize
        out = np.empty(n, dt)
        self.ctx._check("kraken_hip_copy_from_buffer_at", lib().kraken_hip_copy_from_buffer_at(
            self.ctx.handle, self.view, offset_bytes, out.ctypes.data, out.nbytes))
        return out

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """One kraken_hip_context.  Op methods take buffers (see as_buffer) and raise
    KrakenError on a non-OK status; `status(name, ...)` returns the raw code."""

    def __init__(self, validation_only: bool = False):
        self.handle = _ctx()
        fn = (lib().kraken_hip_context_create_validation_only if validation_only
              else lib().kraken_hip_context_create)
        code = fn(ctypes.byref(self.handle))
        if code != OK:
            raise KrakenError(code, last_error(), "kraken_hip_context_create")
        self.validation_only = validation_only

    def close(self):
        if self.handle:
            lib().kraken_hip_context_destroy(self.handle)
            self.handle = _ctx()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, name: str, code: int):
        if code != OK:
            raise KrakenError(code, last_error(), name)

    def status(self, name: str, *args) -> int:
        """Calls kraken_hip_<name> and returns its status code."""
        full = "kraken_hip_" + name
        diag = full in DIAG_SIGNATURES
        fn = getattr(diag_lib() if diag else lib(), full)
        types = DIAG_SIGNATURES[full] if diag else SIGNATURES[full]
        conv = [as_buffer(a) if t is KrakenBuffer else a for a, t in zip(args, types)]
        return fn(self.handle, *conv)

    def call(self, name: str, *args):
        code = self.status(name, *args)
        if code != OK and "kraken_hip_" + name in DIAG_SIGNATURES:
            raise KrakenError(code, diag_lib().kraken_hip_diag_last_error().decode(), name)
        self._check(name, code)

    def __getattr__(self, name):
        if "kraken_hip_" + name in SIGNATURES or "kraken_hip_" + name in DIAG_SIGNATURES:
            return lambda *args: self.call(name, *args)
        raise AttributeError(name)

    def kquant_matvec_multi(self, ggml_types, weights, rows, cols, input, norm_weight, eps,
                            up, residuals, outputs):
        """kraken_hip_kquant_matvec_multi_f32 with Python sequences for the
        per-matrix arrays (residual entries may be None)."""
        n = len(weights)
        types = (ctypes.c_uint32 * n)(*ggml_types)
        ws = (KrakenBuffer * n)(*[as_buffer(w) for w in weights])
        rs = (ctypes.c_size_t * n)(*rows)
        res = (KrakenBuffer * n)(*[as_buffer(r) for r in residuals])
        outs = (KrakenBuffer * n)(*[as_buffer(o) for o in outputs])
        self.call("kquant_matvec_multi_f32", n, types, ws, rs, cols, input, norm_weight, eps, up,
                  res, outs)

    def kquant_matmul_multi(self, ggml_types, weights, rows, cols, tokens, input, outputs):
        """kraken_hip_kquant_matmul_multi_f32 with Python sequences for the
        per-matrix arrays."""
        n = len(weights)
        types = (ctypes.c_uint32 * n)(*ggml_types)
        ws = (KrakenBuffer * n)(*[as_buffer(w) for w in weights])
        rs = (ctypes.c_size_t * n)(*rows)
        outs = (KrakenBuffer * n)(*[as_buffer(o) for o in outputs])
        self.call("kquant_matmul_multi_f32", n, types, ws, rs, cols, tokens, input, outs)

    def kquant_matvec_multi_conv(self, ggml_types, weights, rows, cols, input, norm_weight, eps,
                                 outputs, conv_pool, conv_offset, conv_weights, conv_kernel=4):
        """kraken_hip_kquant_matvec_multi_conv_f32 with Python sequences for the
        per-matrix arrays."""
        n = len(weights)
        types = (ctypes.c_uint32 * n)(*ggml_types)
        ws = (KrakenBuffer * n)(*[as_buffer(w) for w in weights])
        rs = (ctypes.c_size_t * n)(*rows)
        outs = (KrakenBuffer * n)(*[as_buffer(o) for o in outputs])
        self.call("kquant_matvec_multi_conv_f32", n, types, ws, rs, cols, input, norm_weight, eps,
                  outs, conv_pool, conv_offset, conv_weights, conv_kernel)

    def buffer(self, array=None, *, byte_size: int | None = None, dtype=np.float32):
        """Device buffer holding `array` (or `byte_size` uninitialised bytes)."""
        if array is not None:
            a = np.ascontiguousarray(array)
            buf = DeviceBuffer(self, max(a.nbytes, 4), a.dtype)
            if a.nbytes:
                buf.upload(a)
            return buf
        return DeviceBuffer(self, byte_size, dtype)

    def set_stream(self, stream_handle: int | None):
        self.call("context_set_stream", ctypes.c_void_p(stream_handle or 0))

    @property
    def stream(self) -> int:
        return lib().kraken_hip_context_stream(self.handle) or 0

    def abort_graph(self):
        lib().kraken_hip_abort_graph(self.handle)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


class NumpyOps:
    """numpy-in / numpy-out front end with the oracle's function names
    (oracle/oracle.py), so one test body can run against either."""

    def __init__(self, ctx: Context):
        self.ctx = ctx

    def _buf(self, a, dtype=np.float32):
        return self.ctx.buffer(np.ascontiguousarray(np.asarray(a, dtype=dtype)))

    def qk_norm_f32_batched(self, values, weight, tokens, heads, head_dim, eps):
        v, w = self._buf(values), self._buf(weight)
        self.ctx.qk_norm_f32_f32_batched(v, w, tokens, heads, head_dim, eps)
        return v.download(np.asarray(values).size)

    def norm_gated(self, values, weight, gate, tokens, heads, head_dim, eps):
        v, w, g = self._buf(values), self._buf(weight), self._buf(gate)
        self.ctx.qwen35_norm_gated_f32_in_place(v, w, g, tokens, heads, head_dim, eps)
        return v.download(np.asarray(values).size)

    def l2_norm(self, values, rows, row_size, eps):
        v = self._buf(values)
        self.ctx.l2_norm_f32_in_place(v, rows, row_size, eps)
        return v.download(np.asarray(values).size)

    def split_qkv_l2_norm(self, source, tokens, key_heads, value_heads, head_dim, eps):
        s = self._buf(source)
        q = self.ctx.buffer(byte_size=4 * tokens * key_heads * head_dim)
        k = self.ctx.buffer(byte_size=4 * tokens * key_heads * head_dim)
        v = self.ctx.buffer(byte_size=4 * tokens * value_heads * head_dim)
        self.ctx.split_qkv_l2_norm_f32_qwen35(s, q, k, v, tokens, key_heads, value_heads,
                                              head_dim, eps)
        return q.download(), k.download(), v.download()

    def gated_delta_net(self, query, key, value, gate, beta, state, tokens, key_heads,
                        value_heads, head_dim, state_offset=0):
        q, k, v, g, b = (self._buf(x) for x in (query, key, value, gate, beta))
        st_arr = _f32(state)
        st = self._buf(st_arr)
        out = self.ctx.buffer(byte_size=4 * tokens * value_heads * head_dim)
        self.ctx.gated_delta_net_f32_batched_in_place_at(q, k, v, g, b, st, state_offset, tokens,
                                                         key_heads, value_heads, head_dim, out)
        return out.download(), st.download(st_arr.size)

    def ssm_conv(self, inp, kernel, conv_kernel, channels, tokens, sequences):
        x, w = self._buf(inp), self._buf(kernel)
        out = self.ctx.buffer(byte_size=4 * sequences * tokens * channels)
        self.ctx.ssm_conv_f32(x, w, conv_kernel, channels, tokens, sequences, out)
        return out.download()

    def ssm_conv1_stateful(self, state, inp, kernel, conv_kernel, channels):
        st, x, w = self._buf(state), self._buf(inp), self._buf(kernel)
        out = self.ctx.buffer(byte_size=4 * channels)
        self.ctx.ssm_conv1_f32_stateful_at(st, 0, x, w, conv_kernel, channels, out)
        return out.download(), st.download(np.asarray(state).size)

    def build_ssm_conv_state(self, state, inp, conv_kernel, channels, tokens):
        st, x = self._buf(state), self._buf(inp)
        ci = self.ctx.buffer(byte_size=4 * channels * (conv_kernel - 1 + tokens))
        self.ctx.build_ssm_conv_state_f32(st, 0, x, conv_kernel, channels, tokens, ci)
        return ci.download(), st.download(np.asarray(state).size)

    def mrope(self, values, positions, tokens, heads, head_dim, n_dims, sections, theta):
        v = self._buf(values)
        p = self._buf(positions, np.int32)
        s = list(sections)
        self.ctx.mrope_f32_in_place(v, p, tokens, heads, head_dim, n_dims, s[0], s[1], s[2],
                                    s[3], theta)
        return v.download(np.asarray(values).size)

    def _unary(self, name, values):
        v = self._buf(values)
        n = np.asarray(values).size
        self.ctx.call(name, v, n)
        return v.download(n)

    def sigmoid(self, values):
        return self._unary("sigmoid_f32_in_place", values)

    def softplus(self, values):
        return self._unary("softplus_f32_in_place", values)

    def silu(self, values):
        return self._unary("silu_f32_in_place", values)

    def mul(self, target, rhs):
        t, r = self._buf(target), self._buf(rhs)
        n = np.asarray(target).size
        self.ctx.mul_f32_in_place(t, r, n)
        return t.download(n)

    def prepare_gdn_gate_beta(self, gate, beta, gate_bias, gate_scale, rows, row_size):
        g, b, gb, gs = (self._buf(x) for x in (gate, beta, gate_bias, gate_scale))
        self.ctx.prepare_qwen35_gdn_gate_beta_f32(g, b, gb, gs, rows, row_size)
        n = rows * row_size
        return g.download(n), b.download(n)

    def copy_f32_rows(self, source, destination, rows, row_size, source_stride, source_offset,
                      destination_stride, destination_offset):
        s, d = self._buf(source), self._buf(destination)
        self.ctx.copy_f32_rows(s, d, rows, row_size, source_stride, source_offset,
                               destination_stride, destination_offset)
        return d.download(np.asarray(destination).size)

    def copy_f32_rows_to_f16(self, source, destination_bits, rows, row_size, source_stride,
                             source_offset, destination_stride, destination_offset):
        s = self._buf(source)
        d = self._buf(destination_bits, np.uint16)
        self.ctx.copy_f32_rows_to_f16(s, d, rows, row_size, source_stride, source_offset,
                                      destination_stride, destination_offset)
        return d.download(np.asarray(destination_bits).size, np.uint16)

    def attention_batched(self, query, key_cache, value_cache, layer, start_position, tokens,
                          capacity_tokens, heads, kv_heads, head_dim, gate=None):
        """uint16 caches hold f16 bits (F16 KV path); float32 caches take the F32 KV path."""
        kc = np.ascontiguousarray(key_cache)
        vc = np.ascontiguousarray(value_cache)
        q = self._buf(query)
        kb, vb = self.ctx.buffer(kc), self.ctx.buffer(vc)
        out = self.ctx.buffer(byte_size=4 * tokens * heads * head_dim)
        if kc.dtype == np.uint16:
            if gate is not None:
                self.ctx.attention_f32_batched_f16_kv_gated(
                    q, kb, vb, self._buf(gate), layer, start_position, tokens, capacity_tokens,
                    heads, kv_heads, head_dim, out)
            else:
                self.ctx.attention_f32_batched_f16_kv(q, kb, vb, layer, start_position, tokens,
                                                      capacity_tokens, heads, kv_heads,
                                                      head_dim, out)
        else:
            assert gate is None
            self.ctx.attention_f32_batched(q, kb, vb, layer, start_position, tokens,
                                           capacity_tokens, heads, kv_heads, head_dim, out)
        return out.download()

    # ---- K-quant projections and argmax (oracle.kquant_* / oracle.argmax) ----

    def kquant_dequantize(self, fmt, data, blocks):
        """blocks super-blocks -> 256 * blocks f32 values (dequantize_rows_*
        with one 256-value row per block, rows in order)."""
        w = self.ctx.buffer(np.ascontiguousarray(data, np.uint8))
        ids = self._buf(np.arange(blocks), np.int32)
        out = self.ctx.buffer(byte_size=4 * 256 * blocks)
        getattr(self.ctx, f"dequantize_rows_{fmt}_f32")(w, blocks, ids, blocks, 256, out)
        return out.download(256 * blocks)

    def kquant_dequantize_row(self, fmt, data, row, cols):
        w = self.ctx.buffer(np.ascontiguousarray(data, np.uint8))
        out = self.ctx.buffer(byte_size=4 * cols)
        getattr(self.ctx, f"dequantize_row_{fmt}_f32")(w, row, cols, out)
        return out.download(cols)

    def kquant_matmul(self, fmt, weight, rows, cols, x, tokens, weight_f16=False,
                      input_f16=False):
        """output [tokens][rows].  The device picks the arithmetic by token
        count (fp32 up to 8 tokens, f16 operands above); the flags exist for
        signature parity with the oracle and are not consulted."""
        w = self.ctx.buffer(np.ascontiguousarray(weight, np.uint8))
        xb = self._buf(np.asarray(x, np.float32).reshape(-1))
        out = self.ctx.buffer(byte_size=4 * rows * tokens)
        if tokens == 1:
            getattr(self.ctx, f"matvec_{fmt}_f32_device")(w, rows, cols, xb, out)
        else:
            getattr(self.ctx, f"matmul_{fmt}_f32_device")(w, rows, cols, tokens, xb, out)
        return out.download(rows * tokens)

    def kquant_top1(self, fmt, weight, rows, cols, x, probability=False):
        w = self.ctx.buffer(np.ascontiguousarray(weight, np.uint8))
        xb = self._buf(np.asarray(x, np.float32).reshape(-1))
        tok = self.ctx.buffer(np.array([-7], np.int32))
        if probability:
            prob = self._buf(np.array([-1.0], np.float32))
            getattr(self.ctx, f"matvec_{fmt}_f32_top1")(w, rows, cols, xb, tok, prob)
            return int(tok.download(1)[0]), float(prob.download(1)[0])
        getattr(self.ctx, f"matvec_{fmt}_f32_argmax")(w, rows, cols, xb, tok)
        return int(tok.download(1)[0])

    def argmax(self, values, probability=False):
        v = _f32(values).reshape(-1)
        vb = self._buf(v)
        tok = self.ctx.buffer(np.array([-7], np.int32))
        if probability:
            prob = self._buf(np.array([-1.0], np.float32))
            self.ctx.argmax_prob_f32_i32(vb, v.size, tok, prob)
            return int(tok.download(1)[0]), float(prob.download(1)[0])
        self.ctx.argmax_f32_i32(vb, v.size, tok)
        return int(tok.download(1)[0])
