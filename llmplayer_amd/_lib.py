"""ctypes binding of libllmp_hip.so -- the Python twin of the Java FFM binding a maintainer
adds to the reference (CudaBindings.java:23-95 binds libcuda the same way: downcall handles,
long device pointers, int status codes).

The library is loaded from the package directory only; there is no fallback.  A missing or
unloadable library raises immediately, so no caller can silently run without the HIP path.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libllmp_hip.so")

LLMP_OK = 0
ERR_NAMES = {
    1: "LLMP_ERR_INVALID_ARG", 2: "LLMP_ERR_OUT_OF_RANGE", 3: "LLMP_ERR_NOT_INIT",
    4: "LLMP_ERR_NO_DEVICE", 5: "LLMP_ERR_OUT_OF_MEMORY", 6: "LLMP_ERR_UNSUPPORTED",
    7: "LLMP_ERR_HIP", 8: "LLMP_ERR_BAD_HANDLE",
}
LLMP_KV_F32, LLMP_KV_Q8_0, LLMP_KV_Q8_0_TRUNC = 0, 1, 2
LLMP_ROPE_NORMAL, LLMP_ROPE_NEOX = 0, 2
LLMP_ROPE_SEL_NONE, LLMP_ROPE_SEL_GLOBAL, LLMP_ROPE_SEL_LOCAL = -1, 0, 1
LLMP_NORM_SEQUENTIAL, LLMP_NORM_V = 1, 2
LLMP_GGML_F32, LLMP_GGML_F16, LLMP_GGML_Q4_0, LLMP_GGML_Q8_0 = 0, 1, 2, 8
LLMP_GGML_Q4_K, LLMP_GGML_Q6_K, LLMP_GGML_BF16 = 12, 14, 30
LLMP_GGML_Q5_0, LLMP_GGML_Q3_K, LLMP_GGML_Q5_K = 6, 11, 13
LLMP_GGML_IQ4_NL, LLMP_GGML_IQ4_XS, LLMP_GGML_MXFP4 = 20, 23, 39
LLMP_GGML_Q5_1, LLMP_GGML_Q2_K = 7, 10
LLMP_GGML_IQ3_XXS, LLMP_GGML_IQ3_S, LLMP_GGML_IQ2_S = 18, 21, 22
(LLMP_W_ATTN_NORM, LLMP_W_Q, LLMP_W_K, LLMP_W_V, LLMP_W_QKV, LLMP_W_O, LLMP_W_Q_BIAS, LLMP_W_K_BIAS,
 LLMP_W_V_BIAS, LLMP_W_O_BIAS, LLMP_W_POST_ATTN_NORM) = range(11)
LLMP_INPUT_F32, LLMP_INPUT_Q8_1 = 0, 1
LLMP_PROF_DECODE_SPLIT, LLMP_PROF_DECODE_REDUCE = 0, 1
LLMP_PROF_PREFILL_APPEND, LLMP_PROF_PREFILL_ATTN = 2, 3

_u64, _i32, _f32 = C.c_uint64, C.c_int, C.c_float
_pu64 = C.POINTER(C.c_uint64)
_pf = C.POINTER(C.c_float)
_vp = C.c_void_p

# name -> argtypes (every function returns int status)
SIGNATURES = {
    "llmp_init": [_i32],
    "llmp_shutdown": [],
    "llmp_device_info": [C.POINTER(_i32), C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.c_char_p, _i32],
    "llmp_last_error": [C.c_char_p, _i32],
    "llmp_malloc": [_pu64, _u64],
    "llmp_free": [_u64],
    "llmp_memcpy_htod": [_u64, _vp, _u64, _u64],
    "llmp_memcpy_dtoh": [_vp, _u64, _u64, _u64],
    "llmp_memcpy_dtod": [_u64, _u64, _u64, _u64],
    "llmp_memset_zero": [_u64, _u64, _u64],
    "llmp_stream_create": [_pu64],
    "llmp_stream_destroy": [_u64],
    "llmp_stream_sync": [_u64],
    "llmp_event_create": [_pu64],
    "llmp_event_destroy": [_u64],
    "llmp_event_record": [_u64, _u64],
    "llmp_event_sync": [_u64],
    "llmp_event_elapsed_ms": [_pf, _u64, _u64],
    "llmp_kv_create": [_i32, _i32, _i32, _i32, _i32, _pu64],
    "llmp_kv_destroy": [_u64],
    "llmp_kv_read": [_u64, _i32, _i32, _i32, _pf, _pf],
    "llmp_kv_write": [_u64, _i32, _i32, _i32, _pf, _pf],
    "llmp_kv_read_q8": [_u64, _i32, _i32, _i32, C.POINTER(C.c_int8), _pf, C.POINTER(C.c_int8), _pf],
    "llmp_kv_write_q8": [_u64, _i32, _i32, _i32, C.POINTER(C.c_int8), _pf, C.POINTER(C.c_int8), _pf],
    "llmp_kv_layer_ptrs": [_u64, _i32, _pu64, _pu64],
    "llmp_kv_clear": [_u64, _u64],
    "llmp_rope_table": [_i32, _i32, _f32, _f32, _pf, _i32, _pf, _pf],
    "llmp_rope_table_yarn": [_i32, _i32, _f32, _pf, _i32, _f32, _i32, _f32, _f32, _f32, _pf, _pf, _pf],
    "llmp_rope_upload": [_u64, _i32, _pf, _pf, _i32, _i32],
    "llmp_layer_config": [_u64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _f32,
                          _f32, _pf, _pf],
    "llmp_attn_decode": [_u64, _i32, _i32, _u64, _u64, _u64, _u64, _i32, _u64],
    "llmp_attn_decode_devpos": [_u64, _i32, _u64, _u64, _u64, _u64, _u64, _i32, _u64],
    "llmp_attn_decode_ex": [_u64, _i32, _i32, _u64, _u64, _u64, _u64, _u64, _u64, _i32, _u64],
    "llmp_layer_sinks": [_u64, _i32, _pf],
    "llmp_attn_prefill": [_u64, _i32, _i32, _i32, _u64, _u64, _u64, _u64, _u64],
    "llmp_attn_prefill_ex": [_u64, _i32, _i32, _i32, _u64, _u64, _u64, _u64, _u64, _u64],
    "llmp_layer_norm_mode": [_u64, _i32, _i32],
    "llmp_block_config": [_u64, _i32, _f32],
    "llmp_block_input_mode": [_u64, _i32],
    "llmp_layer_weight": [_u64, _i32, _i32, _i32, _i32, _i32, C.c_void_p, _u64],
    "llmp_attn_block": [_u64, _i32, _i32, _u64, _u64, _i32, _u64],
    "llmp_attn_block_batch": [_u64, _i32, _i32, _i32, _u64, _u64],
    "llmp_attn_decode_shared": [_u64, _i32, _i32, _i32, _u64, _u64, _u64, _u64, _i32, _u64],
    "llmp_attn_prefill_shared": [_u64, _i32, _i32, _i32, _i32, _u64, _u64, _u64, _u64],
    "llmp_attn_prefill_f32": [_u64, _i32, _i32, _i32, _u64, _u64, _u64, _u64, _u64, _u64],
    "llmp_attn_prefill_f32_static": [_u64, _i32, _i32, _i32, _u64, _u64, _u64, _u64, _u64, _u64],
    "llmp_attn_prefill_shared_f32": [_u64, _i32, _i32, _i32, _i32, _u64, _u64, _u64, _u64],
    "llmp_decode_plan": [_u64, _i32, _i32, _i32, C.POINTER(_i32), C.POINTER(_i32),
                         C.POINTER(_i32), C.POINTER(_i32)],
    "llmp_graph_begin": [_u64],
    "llmp_graph_end": [_u64, _pu64],
    "llmp_graph_launch": [_u64, _u64],
    "llmp_graph_destroy": [_u64],
    "llmp_profile_enable": [_u64, _i32],
    "llmp_profile_read": [_u64, _i32, C.POINTER(_i32), C.POINTER(C.c_double)],
    "llmp_profile_reset": [_u64],
    "llmp_copy_kernel": [_u64, _u64, _u64, _u64],
}

_lib = None
_lock = threading.Lock()


class LlmpError(RuntimeError):
    """A non-zero status from the library, reported as the reference reports CUDA failures:
    RuntimeException("HIP error in <op>: <code>") (CudaContext.checkError, CudaContext.java:664-668)."""

    def __init__(self, op: str, code: int, message: str):
        self.op, self.code, self.message = op, code, message
        super().__init__(f"HIP error in {op}: {code} ({ERR_NAMES.get(code, '?')}): {message}")


def load() -> C.CDLL:
    """Load libllmp_hip.so from the package directory (raises if it was not built)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                                  "(the HIP path has no CPU fallback)")
            L = C.CDLL(LIB_PATH)
            for name, args in SIGNATURES.items():
                fn = getattr(L, name)
                fn.argtypes = args
                fn.restype = C.c_int
            _lib = L
        return _lib


def last_error() -> str:
    buf = C.create_string_buffer(1024)
    load().llmp_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def call(name: str, *args) -> None:
    """Call `name` and raise LlmpError on a non-zero status."""
    rc = getattr(load(), name)(*args)
    if rc != LLMP_OK:
        raise LlmpError(name, rc, last_error())


def status(name: str, *args) -> int:
    """Call `name` and return its raw status (for tests of the error plumbing)."""
    return getattr(load(), name)(*args)
