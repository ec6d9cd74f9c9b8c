"""TEST INFRASTRUCTURE ONLY -- ctypes view of the C restatement in attn_oracle.c.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module,
and only as the checker; the product path (llmplayer_amd/) never touches it.

Every function wraps the C function of the same name, which cites the reference Java code it
restates (Attention.java, KVCache.java, RoPE.java, SimdVectorOps.java, ScalarOps.java under
/root/reference/src/main/).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
# LLMP_ORACLE_LIB names another build of the same sources (the sanitizer build of the CPU tests).
_LIB_PATH = os.environ.get("LLMP_ORACLE_LIB") or os.path.join(_HERE, "libattn_oracle.so")
_lib = None

ARCH_OTHER, ARCH_GEMMA2, ARCH_GEMMA3, ARCH_GPT_OSS, ARCH_COHERE2, ARCH_GPT_OSS_MOE = 0, 1, 2, 3, 4, 5
ROPE_NORMAL, ROPE_NEOX = 0, 2


def build(force: bool = False) -> str:
    """Compile libattn_oracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B", "-C", _HERE], check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


class _Cfg(C.Structure):
    _fields_ = [
        ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("head_size", C.c_int),
        ("rope_dim", C.c_int), ("rope_type", C.c_int), ("max_seq", C.c_int),
        ("norm_eps", C.c_float), ("sliding_window", C.c_int),
        ("attention_scale", C.c_float), ("softcap", C.c_float), ("arch", C.c_int),
        ("no_rope_interval", C.c_int), ("nope_on_global", C.c_int),
        ("sinks", C.POINTER(C.c_float)),
    ]


class _BlockW(C.Structure):
    _fields_ = [
        ("dim", C.c_int), ("residual_scale", C.c_float),
        ("attn_norm", C.POINTER(C.c_float)), ("post_attn_norm", C.POINTER(C.c_float)),
        ("wq", C.POINTER(C.c_uint8)), ("wk", C.POINTER(C.c_uint8)), ("wv", C.POINTER(C.c_uint8)),
        ("wqkv", C.POINTER(C.c_uint8)), ("wo", C.POINTER(C.c_uint8)),
        ("wq_type", C.c_int), ("wk_type", C.c_int), ("wv_type", C.c_int), ("wqkv_type", C.c_int),
        ("wo_type", C.c_int),
        ("q_bias", C.POINTER(C.c_float)), ("k_bias", C.POINTER(C.c_float)),
        ("v_bias", C.POINTER(C.c_float)), ("o_bias", C.POINTER(C.c_float)),
        ("q8_1_input", C.c_int),
    ]


@dataclass
class OracleConfig:
    """Attention hyper-parameters read by Attention.forwardFromProjections."""
    n_heads: int
    n_kv_heads: int
    head_size: int
    max_seq: int
    rope_type: int = ROPE_NORMAL
    rope_dim: int = 0          # 0 -> head_size
    norm_eps: float = 1e-5
    sliding_window: int = 0
    attention_scale: float = 0.0
    softcap: float = 0.0
    arch: int = ARCH_OTHER
    no_rope_interval: int = 0
    nope_on_global: bool = False
    sinks: Optional[np.ndarray] = None   # [n_heads] attention-sink logits (GPT-OSS)

    def c(self) -> _Cfg:
        sinks = None
        if self.sinks is not None:
            self._sinks_keep = np.ascontiguousarray(self.sinks, np.float32)
            assert self._sinks_keep.size == self.n_heads
            sinks = self._sinks_keep.ctypes.data_as(C.POINTER(C.c_float))
        return _Cfg(self.n_heads, self.n_kv_heads, self.head_size,
                    self.rope_dim or self.head_size, self.rope_type, self.max_seq,
                    self.norm_eps, self.sliding_window, self.attention_scale, self.softcap,
                    self.arch, self.no_rope_interval, int(self.nope_on_global), sinks)

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_size


_F = C.POINTER(C.c_float)


def lib():
    global _lib
    if _lib is None:
        build()
        L = C.CDLL(_LIB_PATH)
        L.orc_dot.restype = C.c_float
        L.orc_dot.argtypes = [_F, _F, C.c_int]
        L.orc_saxpy.argtypes = [C.c_float, _F, _F, C.c_int]
        L.orc_softmax.argtypes = [_F, C.c_int]
        L.orc_softmax_with_sink.argtypes = [_F, C.c_int, C.c_float]
        L.orc_sigmoid_gate.argtypes = [_F, _F, C.c_int]
        L.orc_per_head_norm.argtypes = [_F, _F, C.c_int, C.c_int, C.c_float]
        L.orc_rope_tables.argtypes = [C.c_int, C.c_int, C.c_float, C.c_float, _F, C.c_int, _F, _F]
        L.orc_rope_tables_yarn.argtypes = [C.c_int, C.c_int, C.c_float, _F, C.c_int, C.c_float,
                                           C.c_int, C.c_float, C.c_float, C.c_float, _F, _F, _F]
        L.orc_rope_apply_all.argtypes = [_F, C.c_int, C.c_int, C.c_int, C.c_int, _F, _F, C.c_int]
        L.orc_is_global_layer.restype = C.c_int
        L.orc_is_global_layer.argtypes = [C.c_int, C.c_int]
        L.orc_start_pos.restype = C.c_int
        L.orc_start_pos.argtypes = [C.POINTER(_Cfg), C.c_int, C.c_int]
        L.orc_forward_from_projections.argtypes = [
            C.POINTER(_Cfg), _F, _F, _F, _F, _F, _F, _F, _F, _F, C.c_int, C.c_int, _F, _F,
            C.c_int, C.c_int]
        L.orc_prefill_sequential.argtypes = [
            C.POINTER(_Cfg), _F, _F, _F, _F, _F, _F, _F, _F, _F, C.c_int, C.c_int, C.c_int,
            _F, C.c_int]
        L.orc_max_threads.restype = C.c_int
        _I8 = C.POINTER(C.c_int8)
        L.orc_round_half_up.restype = C.c_int
        L.orc_round_half_up.argtypes = [C.c_float]
        L.orc_q8_quantize.argtypes = [_F, C.c_int, _I8, _F]
        L.orc_q8_dot.restype = C.c_float
        L.orc_q8_dot.argtypes = [_F, _I8, _F, C.c_int]
        L.orc_q8_saxpy.argtypes = [C.c_float, _I8, _F, _F, C.c_int]
        L.orc_q8_quantize_simd8.argtypes = [_F, C.c_int, _I8, _F]
        L.orc_q8_dot_simd8.restype = C.c_float
        L.orc_q8_dot_simd8.argtypes = [_F, _I8, _F, C.c_int]
        L.orc_q8_saxpy_simd8.argtypes = [C.c_float, _I8, _F, _F, C.c_int]
        L.orc_forward_from_projections_q8.argtypes = [
            C.POINTER(_Cfg), _I8, _F, _I8, _F, _F, _F, _F, _F, _F, _F, _F, C.c_int, C.c_int, _F,
            _F, C.c_int, C.c_int, C.c_int]
        L.orc_prefill_sequential_q8.argtypes = [
            C.POINTER(_Cfg), _I8, _F, _I8, _F, _F, _F, _F, _F, _F, _F, _F, C.c_int, C.c_int,
            C.c_int, _F, C.c_int, C.c_int]
        L.orc_rms_norm_seq.argtypes = [_F, _F, C.c_int, C.c_float]
        L.orc_forward_gemma4.argtypes = [
            C.POINTER(_Cfg), _F, _F, _F, _F, _F, _F, _F, _F, _F, C.c_int, C.c_int, _F, _F,
            C.c_int]
        _U8 = C.POINTER(C.c_uint8)
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_ggml_block.restype = C.c_int
        L.orc_ggml_block.argtypes = [C.c_int, C.POINTER(C.c_int)]
        L.orc_dequant_row.restype = C.c_int
        L.orc_dequant_row.argtypes = [C.c_int, _U8, C.c_int, _F]
        L.orc_matmul.restype = C.c_int
        L.orc_matmul.argtypes = [C.c_int, _U8, C.c_int, C.c_int, _F, _F]
        L.orc_rmsnorm.argtypes = [_F, _F, _F, C.c_int, C.c_float]
        L.orc_rmsnorm_staged.argtypes = [_F, _F, _F, C.c_int, C.c_float]
        L.orc_quantize_q8_1.argtypes = [_F, C.c_int, C.POINTER(C.c_int8), _F, _F]
        L.orc_q8_1_routed.restype = C.c_int
        L.orc_q8_1_routed.argtypes = [C.c_int]
        L.orc_iq_grid.restype = C.c_uint64
        L.orc_iq_grid.argtypes = [C.c_int, C.c_int]
        L.orc_ksigns_entry.restype = C.c_int
        L.orc_ksigns_entry.argtypes = [C.c_int]
        L.orc_matmul_q8_1.restype = C.c_int
        L.orc_matmul_q8_1.argtypes = [C.c_int, _U8, C.c_int, C.c_int, C.POINTER(C.c_int8), _F, _F,
                                      _F]
        L.orc_attn_block.restype = C.c_int
        L.orc_attn_block.argtypes = [C.POINTER(_Cfg), C.POINTER(_BlockW), _F, _F, _F, _F, _F,
                                     _F, _F, C.c_int, C.c_int, C.c_int, _F]
        _lib = L
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_F)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def dot(a, b) -> np.float32:
    a, b = f32(a), f32(b)
    return np.float32(lib().orc_dot(_p(a), _p(b), a.size))


def saxpy(alpha, x, y) -> np.ndarray:
    x, y = f32(x), f32(y).copy()
    lib().orc_saxpy(float(np.float32(alpha)), _p(x), _p(y), x.size)
    return y


def softmax(x) -> np.ndarray:
    x = f32(x).copy()
    lib().orc_softmax(_p(x), x.size)
    return x


def softmax_with_sink(x, sink) -> np.ndarray:
    """Qwen3MoEInferenceEngine.softmaxWithSink."""
    x = f32(x).copy()
    lib().orc_softmax_with_sink(_p(x), x.size, float(np.float32(sink)))
    return x


def sigmoid_gate(out, gate) -> np.ndarray:
    """out * sigmoid(gate) as the Qwen3.5 attention output gate computes it."""
    out, gate = f32(out).copy(), f32(gate)
    assert out.size == gate.size
    lib().orc_sigmoid_gate(_p(out), _p(gate), out.size)
    return out


def per_head_norm(vec, w, n_heads, head_size, eps) -> np.ndarray:
    vec, w = f32(vec).copy(), f32(w)
    lib().orc_per_head_norm(_p(vec), _p(w), n_heads, head_size, float(np.float32(eps)))
    return vec


def rope_tables(rope_dim, max_seq, theta, linear_freq_scale=1.0, freq_factors=None):
    half = rope_dim // 2
    cos_t = np.zeros((max_seq, half), np.float32)
    sin_t = np.zeros((max_seq, half), np.float32)
    ff = f32(freq_factors) if freq_factors is not None else None
    lib().orc_rope_tables(rope_dim, max_seq, float(np.float32(theta)),
                          float(np.float32(linear_freq_scale)), _p(ff),
                          0 if ff is None else ff.size, _p(cos_t), _p(sin_t))
    return cos_t, sin_t


def rope_tables_yarn(rope_dim, max_seq, theta, scaling_factor, orig_ctx, yarn_log_mul=0.0,
                     beta_fast=32.0, beta_slow=1.0, freq_factors=None):
    """RoPE tables of the YaRN branch (RoPE.java:45-117) and the attention-magnitude factor
    mscale.  Returns (cos [max_seq, R/2], sin, mscale)."""
    half = rope_dim // 2
    cos_t = np.zeros((max_seq, half), np.float32)
    sin_t = np.zeros((max_seq, half), np.float32)
    ff = f32(freq_factors) if freq_factors is not None else None
    ms = np.zeros(1, np.float32)
    lib().orc_rope_tables_yarn(rope_dim, max_seq, float(np.float32(theta)), _p(ff),
                               0 if ff is None else ff.size, float(np.float32(scaling_factor)),
                               int(orig_ctx), float(np.float32(beta_fast)),
                               float(np.float32(beta_slow)), float(np.float32(yarn_log_mul)),
                               _p(cos_t), _p(sin_t), _p(ms))
    return cos_t, sin_t, np.float32(ms[0])


def rope_apply_all(vec, n_heads, head_size, rope_dim, rope_type, cos_t, sin_t, pos):
    vec = f32(vec).copy()
    lib().orc_rope_apply_all(_p(vec), n_heads, head_size, rope_dim, rope_type,
                             _p(f32(cos_t)), _p(f32(sin_t)), pos)
    return vec


def is_global_layer(arch, layer) -> bool:
    return bool(lib().orc_is_global_layer(arch, layer))


def start_pos(cfg: OracleConfig, layer, pos) -> int:
    c = cfg.c()
    return lib().orc_start_pos(C.byref(c), layer, pos)


def forward_from_projections(cfg: OracleConfig, kcache, vcache, q, k, v, layer, pos,
                             qnorm_w=None, knorm_w=None, rope_cos=None, rope_sin=None,
                             use_flash=False, n_threads=1, gate=None):
    """Runs Attention.forwardFromProjections for one layer-call.

    kcache/vcache: float32 [max_seq, kvDim] (the reference layout), modified in place (the
    new K/V rows are appended at `pos`).  Returns (out[Hq*D], q_after, k_after): q and k
    after QK-norm and RoPE, as state.q / state.k hold them after the call.  cfg.sinks selects
    GPT-OSS's sink softmax; `gate` ([Hq*D]) applies the Qwen3.5 output gate to out."""
    c = cfg.c()
    q, k, v = f32(q).copy(), f32(k).copy(), f32(v)
    assert kcache.dtype == np.float32 and kcache.flags["C_CONTIGUOUS"]
    assert vcache.dtype == np.float32 and vcache.flags["C_CONTIGUOUS"]
    assert kcache.size >= cfg.max_seq * cfg.kv_dim and vcache.size >= cfg.max_seq * cfg.kv_dim
    assert 0 <= pos < cfg.max_seq
    out = np.zeros(cfg.n_heads * cfg.head_size, np.float32)
    att = np.zeros(cfg.n_heads * (pos + 1), np.float32)
    lib().orc_forward_from_projections(
        C.byref(c), _p(kcache), _p(vcache),
        _p(f32(qnorm_w)) if qnorm_w is not None else None,
        _p(f32(knorm_w)) if knorm_w is not None else None,
        _p(f32(rope_cos)) if rope_cos is not None else None,
        _p(f32(rope_sin)) if rope_sin is not None else None,
        _p(q), _p(k), _p(v), layer, pos, _p(out), _p(att), int(use_flash), int(n_threads))
    if gate is not None:
        out = sigmoid_gate(out, gate)
    return out, q, k


def prefill_sequential(cfg: OracleConfig, kcache, vcache, q, k, v, layer, pos0,
                       qnorm_w=None, knorm_w=None, rope_cos=None, rope_sin=None, n_threads=1,
                       gate=None):
    """P sequential single-token calls (the reference's prefill).  q: [P, Hq*D],
    k/v: [P, kvDim].  Returns out [P, Hq*D]; the caches gain rows pos0..pos0+P-1.
    `gate` ([P, Hq*D]) applies the Qwen3.5 output gate to each token's output."""
    c = cfg.c()
    q, k, v = f32(q), f32(k), f32(v)
    P = q.shape[0]
    assert pos0 + P <= cfg.max_seq
    out = np.zeros((P, cfg.n_heads * cfg.head_size), np.float32)
    lib().orc_prefill_sequential(
        C.byref(c), _p(kcache), _p(vcache),
        _p(f32(qnorm_w)) if qnorm_w is not None else None,
        _p(f32(knorm_w)) if knorm_w is not None else None,
        _p(f32(rope_cos)) if rope_cos is not None else None,
        _p(f32(rope_sin)) if rope_sin is not None else None,
        _p(q), _p(k), _p(v), layer, pos0, P, _p(out), int(n_threads))
    if gate is not None:
        out = sigmoid_gate(out.reshape(-1), f32(gate).reshape(-1)).reshape(out.shape)
    return out


def _pi8(a):
    assert a.dtype == np.int8 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.POINTER(C.c_int8))


def round_half_up(y) -> int:
    return lib().orc_round_half_up(float(np.float32(y)))


# The two Q8_0 contracts the JVM chooses between (KVCache.loadQ8Ops, KVCache.java:54-62).
Q8_SCALAR = 1   # quantizeBlocksScalar / dotQ8BlockScalar / saxpyQ8BlockScalar
Q8_SIMD8 = 2    # SimdQ8KvOps on an 8-lane float species (AVX2): truncating quantize, FMA lanes


def q8_quantize(x, mode=Q8_SCALAR):
    """Returns (int8 quants[n], fp32 scales[n/32]) (quantizeBlocksScalar, or
    SimdQ8KvOps.quantize for Q8_SIMD8)."""
    x = f32(x)
    q = np.zeros(x.size, np.int8)
    sc = np.zeros(x.size // 32, np.float32)
    fn = lib().orc_q8_quantize_simd8 if mode == Q8_SIMD8 else lib().orc_q8_quantize
    fn(_p(x), x.size, _pi8(q), _p(sc))
    return q, sc


def q8_dot(q, kq, ks, mode=Q8_SCALAR) -> np.float32:
    q = f32(q)
    fn = lib().orc_q8_dot_simd8 if mode == Q8_SIMD8 else lib().orc_q8_dot
    return np.float32(fn(_p(q), _pi8(np.ascontiguousarray(kq, np.int8)), _p(f32(ks)), q.size))


def q8_saxpy(w, vq, vs, out, mode=Q8_SCALAR):
    out = f32(out).copy()
    fn = lib().orc_q8_saxpy_simd8 if mode == Q8_SIMD8 else lib().orc_q8_saxpy
    fn(float(np.float32(w)), _pi8(np.ascontiguousarray(vq, np.int8)), _p(f32(vs)), _p(out),
       out.size)
    return out


def prefill_sequential_q8(cfg: OracleConfig, kq, ks, vq, vs, q, k, v, layer, pos0,
                          qnorm_w=None, knorm_w=None, rope_cos=None, rope_sin=None, n_threads=1,
                          mode=Q8_SCALAR, gate=None):
    """prefill_sequential over a Q8_0 cache (kq/vq int8 [max_seq, kvDim], ks/vs fp32
    [max_seq, kvDim/32], modified in place: rows pos0..pos0+P-1 are quantised as each token
    appends them).  Returns out [P, Hq*D]."""
    c = cfg.c()
    q, k, v = f32(q), f32(k), f32(v)
    P = q.shape[0]
    assert pos0 + P <= cfg.max_seq
    for a in (kq, vq):
        assert a.dtype == np.int8 and a.flags["C_CONTIGUOUS"] and a.size >= cfg.max_seq * cfg.kv_dim
    for a in (ks, vs):
        assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
        assert a.size >= cfg.max_seq * cfg.kv_dim // 32
    out = np.zeros((P, cfg.n_heads * cfg.head_size), np.float32)
    lib().orc_prefill_sequential_q8(
        C.byref(c), _pi8(kq), _p(ks), _pi8(vq), _p(vs),
        _p(f32(qnorm_w)) if qnorm_w is not None else None,
        _p(f32(knorm_w)) if knorm_w is not None else None,
        _p(f32(rope_cos)) if rope_cos is not None else None,
        _p(f32(rope_sin)) if rope_sin is not None else None,
        _p(q), _p(k), _p(v), layer, pos0, P, _p(out), int(n_threads), int(mode))
    if gate is not None:
        out = sigmoid_gate(out.reshape(-1), f32(gate).reshape(-1)).reshape(out.shape)
    return out


def forward_from_projections_q8(cfg: OracleConfig, kq, ks, vq, vs, q, k, v, layer, pos,
                                qnorm_w=None, knorm_w=None, rope_cos=None, rope_sin=None,
                                use_flash=False, n_threads=1, mode=Q8_SCALAR, gate=None):
    """Attention.forwardFromProjections over a Q8_0 cache.  kq/vq: int8 [max_seq, kvDim],
    ks/vs: float32 [max_seq, kvDim/32], modified in place (row `pos` is quantized and
    stored).  `mode` selects the JVM's Q8_0 contract.  Returns (out, q_after, k_after)."""
    c = cfg.c()
    q, k, v = f32(q).copy(), f32(k).copy(), f32(v)
    for a in (kq, vq):
        assert a.dtype == np.int8 and a.flags["C_CONTIGUOUS"] and a.size >= cfg.max_seq * cfg.kv_dim
    for a in (ks, vs):
        assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
        assert a.size >= cfg.max_seq * cfg.kv_dim // 32
    assert 0 <= pos < cfg.max_seq
    out = np.zeros(cfg.n_heads * cfg.head_size, np.float32)
    att = np.zeros(cfg.n_heads * (pos + 1), np.float32)
    lib().orc_forward_from_projections_q8(
        C.byref(c), _pi8(kq), _p(ks), _pi8(vq), _p(vs),
        _p(f32(qnorm_w)) if qnorm_w is not None else None,
        _p(f32(knorm_w)) if knorm_w is not None else None,
        _p(f32(rope_cos)) if rope_cos is not None else None,
        _p(f32(rope_sin)) if rope_sin is not None else None,
        _p(q), _p(k), _p(v), layer, pos, _p(out), _p(att), int(use_flash), int(n_threads),
        int(mode))
    if gate is not None:
        out = sigmoid_gate(out, gate)
    return out, q, k


def rms_norm_seq(x, w, eps) -> np.ndarray:
    """RMSNorm.apply with offsets / applyNoScale (w None): sequential unfused sum of squares."""
    x = f32(x).copy()
    lib().orc_rms_norm_seq(_p(x), _p(f32(w)) if w is not None else None, x.size, float(eps))
    return x


def forward_gemma4(cfg: OracleConfig, kcache, vcache, q, k, v, pos, is_swa, qnorm_w=None,
                   knorm_w=None, rope_cos=None, rope_sin=None, n_threads=1):
    """Attention half of Gemma4InferenceEngine.forwardLayer over one layer's cache
    ([max_seq, kvDim] fp32, modified in place when the layer has its own KV).  k = v = None
    is a shared-KV layer (reads the source layer's cache, appends nothing).  cfg.head_size is
    the layer type's head size.  Returns (out, q_after, k_after, v_after)."""
    c = cfg.c()
    q = f32(q).copy()
    k = f32(k).copy() if k is not None else None
    v = f32(v).copy() if v is not None else None
    for a in (kcache, vcache):
        assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"] and a.size >= cfg.max_seq * cfg.kv_dim
    assert 0 <= pos < cfg.max_seq
    out = np.zeros(cfg.n_heads * cfg.head_size, np.float32)
    att = np.zeros(cfg.n_heads * (pos + 1), np.float32)
    lib().orc_forward_gemma4(
        C.byref(c), _p(kcache), _p(vcache),
        _p(f32(qnorm_w)) if qnorm_w is not None else None,
        _p(f32(knorm_w)) if knorm_w is not None else None,
        _p(f32(rope_cos)) if rope_cos is not None else None,
        _p(f32(rope_sin)) if rope_sin is not None else None,
        _p(q), _p(k) if k is not None else None, _p(v) if v is not None else None,
        int(bool(is_swa)), pos, _p(out), _p(att), int(n_threads))
    return out, q, k, v


# ---- attention half of a layer over GGUF-format projection weights ----------------------
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K, GGML_BF16 = 0, 1, 2, 8, 12, 14, 30
GGML_Q5_0, GGML_Q3_K, GGML_Q5_K, GGML_IQ4_NL, GGML_IQ4_XS, GGML_MXFP4 = 6, 11, 13, 20, 23, 39
GGML_IQ3_XXS, GGML_IQ3_S, GGML_IQ2_S = 18, 21, 22


def f16_to_f32(h: int) -> np.float32:
    """Float16.toFloat (Float16.java:11-34)."""
    return np.float32(lib().orc_f16_to_f32(int(h) & 0xFFFF))


def ggml_block(t: int):
    """(weights per block, bytes per block) of a GGMLType id (GGMLType.java:4-35)."""
    b = C.c_int()
    n = lib().orc_ggml_block(int(t), C.byref(b))
    if n == 0:
        raise ValueError(f"unsupported GGML type {t}")
    return n, b.value


def iq_grid(t: int) -> np.ndarray:
    """The codebook of an IQ format (IQ3_XXS: 256 words, IQ3_S: 512, IQ2_S: 1024 of 8 bytes) as
    the oracle holds it (IQGridTables.java:30-398)."""
    n = {GGML_IQ3_XXS: 256, GGML_IQ3_S: 512, GGML_IQ2_S: 1024}[t]
    return np.array([lib().orc_iq_grid(int(t), i) for i in range(n)], dtype=np.uint64)


def ksigns(i: int) -> int:
    """IQGridTables.KSIGNS_IQ2XS[i] as the oracle forms it (the 7-bit index plus a parity bit)."""
    return int(lib().orc_ksigns_entry(int(i)))


def ggml_row_bytes(t: int, cols: int) -> int:
    n, b = ggml_block(t)
    assert cols % n == 0
    return cols // n * b


def _u8p(a):
    assert a.dtype == np.uint8 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.POINTER(C.c_uint8))


def dequant_rows(t: int, w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Dequantised [rows, cols] weights exactly as the tensor class's dot() stages them."""
    w = np.ascontiguousarray(w, np.uint8).reshape(-1)
    rb = ggml_row_bytes(t, cols)
    assert w.size >= rows * rb
    out = np.zeros((rows, cols), np.float32)
    for r in range(rows):
        seg = w[r * rb:(r + 1) * rb]
        assert lib().orc_dequant_row(int(t), _u8p(seg), cols, _p(out[r])) == 0
    return out


def matmul(t: int, w: np.ndarray, rows: int, cols: int, x, out=None) -> np.ndarray:
    """FloatTensor.matmulParallel: out[row] += dot(row, x)."""
    w = np.ascontiguousarray(w, np.uint8).reshape(-1)
    x = f32(x)
    out = np.zeros(rows, np.float32) if out is None else f32(out).copy()
    assert w.size >= rows * ggml_row_bytes(t, cols) and x.size >= cols
    assert lib().orc_matmul(int(t), _u8p(w), rows, cols, _p(x), _p(out)) == 0
    return out


def rmsnorm(x, w, eps) -> np.ndarray:
    """SimdVectorOps.rmsnorm."""
    x = f32(x)
    out = np.zeros_like(x)
    lib().orc_rmsnorm(_p(out), _p(x), _p(f32(w)), x.size, float(eps))
    return out


def rmsnorm_staged(x, w, eps) -> np.ndarray:
    """The library's staged RMSNorm (the reduction order the Q8_1 mode quantises after)."""
    x = f32(x)
    out = np.zeros_like(x)
    lib().orc_rmsnorm_staged(_p(out), _p(x), _p(f32(w)), x.size, float(eps))
    return out


def quantize_q8_1(x):
    """Q8_1 blocks of 32 (quantize_q8.cu): (int8 quants [n], scales [n/32], sums [n/32])."""
    x = f32(x)
    assert x.size % 32 == 0
    q = np.zeros(x.size, np.int8)
    d = np.zeros(x.size // 32, np.float32)
    s = np.zeros(x.size // 32, np.float32)
    lib().orc_quantize_q8_1(_p(x), x.size, q.ctypes.data_as(C.POINTER(C.c_int8)), _p(d), _p(s))
    return q, d, s


def q8_1_routed(t: int) -> bool:
    """Whether the reference GPU runs type t on its Q8_1 input (CudaForwardPass.java:216-226,
    2029-2038)."""
    return bool(lib().orc_q8_1_routed(int(t)))


def matmul_q8_1(t: int, w: np.ndarray, rows: int, cols: int, q, d, s, out=None) -> np.ndarray:
    """The reference GPU's int8 matvec (matmul_<type>_dp4a*.cu: Q4_K, Q8_0, Q5_0, Q3_K, Q5_K,
    IQ4_NL, IQ4_XS) on a Q8_1 input: out[row] += dot."""
    w = np.ascontiguousarray(w, np.uint8).reshape(-1)
    q = np.ascontiguousarray(q, np.int8)
    out = np.zeros(rows, np.float32) if out is None else f32(out).copy()
    assert w.size >= rows * ggml_row_bytes(t, cols) and q.size >= cols
    rc = lib().orc_matmul_q8_1(int(t), _u8p(w), rows, cols, q.ctypes.data_as(C.POINTER(C.c_int8)),
                               _p(f32(d)), _p(f32(s)), _p(out))
    assert rc == 0, "no int8 matvec for this type"
    return out


@dataclass
class BlockWeights:
    """Projection weights of one layer's attention half: raw GGUF bytes (uint8) with their
    GGMLType, fp32 norms and biases.  wqkv (merged) replaces wq/wk/wv when given."""
    dim: int
    wq: Optional[np.ndarray] = None
    wk: Optional[np.ndarray] = None
    wv: Optional[np.ndarray] = None
    wo: Optional[np.ndarray] = None
    wq_type: int = GGML_F32
    wk_type: int = GGML_F32
    wv_type: int = GGML_F32
    wo_type: int = GGML_F32
    wqkv: Optional[np.ndarray] = None
    wqkv_type: int = GGML_F32
    attn_norm: Optional[np.ndarray] = None
    post_attn_norm: Optional[np.ndarray] = None
    q_bias: Optional[np.ndarray] = None
    k_bias: Optional[np.ndarray] = None
    v_bias: Optional[np.ndarray] = None
    o_bias: Optional[np.ndarray] = None
    residual_scale: float = 0.0
    q8_1_input: bool = False     # the reference GPU's Q8_1-input matvecs (q8_1_routed types)

    def c(self):
        keep = []

        def fp(a):
            if a is None:
                return None
            a = f32(a)
            keep.append(a)
            return a.ctypes.data_as(C.POINTER(C.c_float))

        def up(a):
            if a is None:
                return None
            a = np.ascontiguousarray(a, np.uint8)
            keep.append(a)
            return a.ctypes.data_as(C.POINTER(C.c_uint8))
        s = _BlockW(self.dim, float(self.residual_scale), fp(self.attn_norm),
                    fp(self.post_attn_norm), up(self.wq), up(self.wk), up(self.wv),
                    up(self.wqkv), up(self.wo), self.wq_type, self.wk_type, self.wv_type,
                    self.wqkv_type, self.wo_type, fp(self.q_bias), fp(self.k_bias),
                    fp(self.v_bias), fp(self.o_bias), int(bool(self.q8_1_input)))
        return s, keep


def attn_block(cfg: OracleConfig, bw: BlockWeights, kcache, vcache, x, layer, pos,
               qnorm_w=None, knorm_w=None, rope_cos=None, rope_sin=None, n_threads=1,
               return_attn=False):
    """The attention half of TransformerBlock.forward (pre-norm, projections, attention core,
    Wo, post-norm, residual scale, residual add) over fp32 caches [max_seq, kvDim] (row `pos`
    appended).  Returns the updated residual x [dim], and with return_attn also the attention
    output [q_dim] (the output projection's input)."""
    c = cfg.c()
    s, keep = bw.c()
    x = f32(x).copy()
    assert x.size == bw.dim
    attn = np.zeros(cfg.n_heads * cfg.head_size, np.float32)
    rc = lib().orc_attn_block(
        C.byref(c), C.byref(s), _p(kcache), _p(vcache),
        _p(f32(qnorm_w)) if qnorm_w is not None else None,
        _p(f32(knorm_w)) if knorm_w is not None else None,
        _p(f32(rope_cos)) if rope_cos is not None else None,
        _p(f32(rope_sin)) if rope_sin is not None else None,
        _p(x), layer, pos, int(n_threads), _p(attn))
    assert rc == 0, "unsupported weight type or shape"
    del keep
    return (x, attn) if return_attn else x


def max_threads() -> int:
    return lib().orc_max_threads()
