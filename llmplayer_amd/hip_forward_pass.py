"""Host-side mirror of the reference's GPU forward-pass attention section, over libllmp_hip.so.

The reference's engine drives the GPU through a class found by reflection
(InferenceEngine.tryInitForwardPass, InferenceEngine.java:119-160) whose attention half is
`forwardAttentionPart(layer, position)` (CudaForwardPass.java:1495-1588), reached publicly
through `forwardAttentionOnly(...)` (:1481-1488) and gated by the static
`isSupportedForAttention(config, weights)` (:1223-1244).  HipForwardPass keeps those names and
their meaning for the attention steps (2b'-5: QK-norm, RoPE, KV append, attention) with the
semantics of Attention.forwardFromProjections (Attention.java:284-367): sliding window,
local/global RoPE, soft-cap and custom scale, which the reference GPU path lacks.

The Q/K/V projections, Wo and the residual are outside this path: the section takes the
projections in device buffers (gpuQ, gpuK, gpuV) and leaves the attention output in gpuXb2,
which is where the reference's projection and Wo kernels read and write.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

from . import _lib
from ._lib import LlmpError, call

_F = C.POINTER(C.c_float)

# ModelArchitecture names used by the attention section.
ARCH_LLAMA, ARCH_QWEN3, ARCH_GEMMA2, ARCH_GEMMA3 = "llama", "qwen3", "gemma2", "gemma3"
ARCH_GPT_OSS, ARCH_COHERE2, ARCH_GEMMA4 = "gpt-oss", "cohere2", "gemma4"
# ModelConfig.java:295-314: rope type per architecture (0 NORMAL, 2 NEOX).
_NEOX_ARCHS = {"qwen2", "qwen3", "glm4", "phi3", "qwen3moe", "olmo2", "gpt-oss", "granitehybrid",
               "qwen35"}


def rope_type_for(arch: str) -> int:
    return _lib.LLMP_ROPE_NEOX if arch in _NEOX_ARCHS else _lib.LLMP_ROPE_NORMAL


def is_global_layer(arch: str, layer: int, sliding_window_pattern: Optional[Sequence[bool]] = None,
                    expert_count: int = 0) -> bool:
    """Attention.isGlobalLayer (Attention.java:250-276).  GPT-OSS with experts runs on the
    Qwen3MoE engine instead (LLMEngine.java:144), which windows the even layers
    (Qwen3MoEInferenceEngine.java:280-286) where Attention.isGlobalLayer makes them global."""
    if arch == ARCH_GPT_OSS and expert_count > 0:
        return layer % 2 == 1
    if arch == ARCH_GEMMA2:
        return layer % 2 == 1
    if arch == ARCH_GEMMA3:
        return layer % 6 == 5
    if arch == ARCH_GPT_OSS:
        return layer % 2 == 0
    if arch == ARCH_COHERE2:
        return layer % 4 == 3
    if arch == ARCH_GEMMA4:
        if sliding_window_pattern is not None and layer < len(sliding_window_pattern):
            return not sliding_window_pattern[layer]
        return layer % 6 == 5
    return True


@dataclass
class ModelConfig:
    """The ModelConfig fields the attention section reads (ModelConfig.java:242-511)."""
    head_count: int
    head_count_kv: int
    head_size: int
    block_count: int
    architecture: str = ARCH_LLAMA
    rope_freq_base: float = 10000.0
    rope_dim_count: int = 0               # 0 -> head_size
    rope_type: Optional[int] = None       # None -> per architecture
    rope_scaling_factor: float = 1.0      # linear scaling (InferenceEngine.java:61-64); YaRN
                                          # factor in the MoE engines (Qwen3MoEInferenceEngine.java:60-66)
    rope_orig_context_length: int = 0     # YaRN original context (ropeOrigContextLength)
    yarn_log_multiplier: float = 0.0      # YaRN attention-factor log multiplier
    rope_freq_base_swa: float = 10000.0   # Gemma 4 SWA theta
    norm_eps: float = 1e-5
    sliding_window: int = 0
    sliding_window_pattern: Optional[Sequence[bool]] = None
    attention_scale: float = 0.0
    attn_logit_soft_cap: float = 0.0
    no_rope_layer_interval: int = 0
    use_no_pe_on_global_layers: bool = False
    use_layer_norm: bool = False
    expert_count: int = 0                 # > 0 for MoE models (selects the Qwen3MoE engine rules)
    key_length: int = 0                   # Gemma 4: head size of full-attention layers (0 -> head_size)
    shared_kv_layers: int = 0             # Gemma 4: the last N layers reuse earlier layers' KV
    rope_freq_factors: Optional[np.ndarray] = None   # Gemma 4 full-attention RoPE factors

    @property
    def kv_dim(self) -> int:
        return self.head_count_kv * self.head_size

    @property
    def q_dim(self) -> int:
        return self.head_count * self.head_size

    def resolved_rope_type(self) -> int:
        return self.rope_type if self.rope_type is not None else rope_type_for(self.architecture)


@dataclass
class InferenceState:
    """The buffers of InferenceState (InferenceState.java:11-22) the attention section touches."""
    q: np.ndarray
    k: np.ndarray
    v: np.ndarray
    xb2: np.ndarray

    @classmethod
    def create(cls, config: ModelConfig) -> "InferenceState":
        return cls(np.zeros(config.q_dim, np.float32), np.zeros(config.kv_dim, np.float32),
                   np.zeros(config.kv_dim, np.float32), np.zeros(config.q_dim, np.float32))


def init(device: int = 0) -> None:
    call("llmp_init", device)


def shutdown() -> None:
    call("llmp_shutdown")


def device_info() -> dict:
    n_cu = C.c_int()
    tot, fr = C.c_int64(), C.c_int64()
    name = C.create_string_buffer(64)
    call("llmp_device_info", C.byref(n_cu), C.byref(tot), C.byref(fr), name, len(name))
    return {"n_cu": n_cu.value, "hbm_total": tot.value, "hbm_free": fr.value,
            "arch": name.value.decode()}


def _fp(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_F)


def _i8p(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.dtype == np.int8 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.POINTER(C.c_int8))


def to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def from_bf16(b: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 (exact)."""
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def prompt_input(x: np.ndarray, width: int, what: str):
    """A multi-token input array as the library takes it: fp32 projections (the CPU path's own
    values) or bf16 bit patterns (uint16).  Returns (contiguous [P, width] array, is_fp32).
    Any other dtype is rejected rather than converted, so a caller never hands the kernels
    reinterpreted bits."""
    a = np.asarray(x)
    if a.dtype == np.float32:
        f32 = True
    elif a.dtype == np.uint16:
        f32 = False
    else:
        raise TypeError(f"{what}: dtype {a.dtype} (expected float32 projections or uint16 bf16 bits)")
    a = np.ascontiguousarray(a)
    if a.size % width:
        raise ValueError(f"{what}: {a.size} values are not rows of {width}")
    return a.reshape(-1, width), f32


def rope_table(rope_dim: int, max_seq: int, theta: float, linear_freq_scale: float = 1.0,
               freq_factors: Optional[np.ndarray] = None):
    """cos/sin tables [max_seq][rope_dim/2] built as the RoPE constructor builds them
    (RoPE.java:45-106, non-YaRN branch), by the library's host helper."""
    half = rope_dim // 2
    cos_t = np.empty((max_seq, half), np.float32)
    sin_t = np.empty((max_seq, half), np.float32)
    ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, np.float32)
    call("llmp_rope_table", rope_dim, max_seq, float(theta), float(linear_freq_scale), _fp(ff),
         0 if ff is None else ff.size, _fp(cos_t), _fp(sin_t))
    return cos_t, sin_t


def rope_table_yarn(rope_dim: int, max_seq: int, theta: float, scaling_factor: float,
                    orig_ctx: int, yarn_log_mul: float = 0.0, beta_fast: float = 32.0,
                    beta_slow: float = 1.0, freq_factors: Optional[np.ndarray] = None):
    """cos/sin tables of the RoPE constructor's YaRN branch (RoPE.java:45-117) and its
    attention-magnitude factor mscale, by the library's host helper: (cos, sin, mscale)."""
    half = rope_dim // 2
    cos_t = np.empty((max_seq, half), np.float32)
    sin_t = np.empty((max_seq, half), np.float32)
    ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, np.float32)
    ms = np.zeros(1, np.float32)
    call("llmp_rope_table_yarn", rope_dim, max_seq, float(theta), _fp(ff), 0 if ff is None else ff.size,
         float(scaling_factor), int(orig_ctx), float(beta_fast), float(beta_slow), float(yarn_log_mul),
         _fp(cos_t), _fp(sin_t), _fp(ms))
    return cos_t, sin_t, np.float32(ms[0])


class DeviceBuffer:
    """A device allocation (CudaBufferManager.createBuffer analogue)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_uint64()
        call("llmp_malloc", C.byref(p), self.nbytes)
        self.ptr = p.value

    def upload(self, arr: np.ndarray, stream: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes, (arr.nbytes, self.nbytes)
        call("llmp_memcpy_htod", self.ptr, arr.ctypes.data, arr.nbytes, stream)

    def download(self, dtype=np.float32, count: Optional[int] = None, stream: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(count, dtype)
        call("llmp_memcpy_dtoh", out.ctypes.data, self.ptr, out.nbytes, stream)
        return out

    def free(self) -> None:
        if self.ptr:
            call("llmp_free", self.ptr)
            self.ptr = 0


class KvCache:
    """Device KV cache handle (llmp_kv_*): head-major pool, reference-layout read/write.

    dtype LLMP_KV_F32 (KVCache.Mode.FLOAT32), or LLMP_KV_Q8_0 / LLMP_KV_Q8_0_TRUNC
    (KVCache.Mode.Q8_0: int8 quants and one fp32 scale per 32 values, KVCache.java:11-28; new
    rows rounded half up like quantizeBlocksScalar, or truncated like SimdQ8KvOps on 8-lane
    hosts)."""

    def __init__(self, n_layers: int, max_seq: int, n_kv_heads: int, head_dim: int,
                 dtype: int = _lib.LLMP_KV_F32):
        h = C.c_uint64()
        call("llmp_kv_create", n_layers, max_seq, n_kv_heads, head_dim, dtype, C.byref(h))
        self.handle = h.value
        self.dtype = dtype
        self.n_layers, self.max_seq = n_layers, max_seq
        self.n_kv_heads, self.head_dim = n_kv_heads, head_dim

    @property
    def is_q8(self) -> bool:
        return self.dtype in (_lib.LLMP_KV_Q8_0, _lib.LLMP_KV_Q8_0_TRUNC)

    def read_q8(self, layer: int, pos0: int, n: int):
        """(k_quants, k_scales, v_quants, v_scales) in the reference layout
        (KVCache.keyQuants [pos][kvDim], keyScales [pos][kvDim/32])."""
        kq = np.empty((n, self.kv_dim), np.int8)
        vq = np.empty((n, self.kv_dim), np.int8)
        ks = np.empty((n, self.kv_dim // 32), np.float32)
        vs = np.empty((n, self.kv_dim // 32), np.float32)
        call("llmp_kv_read_q8", self.handle, layer, pos0, n, _i8p(kq), _fp(ks), _i8p(vq), _fp(vs))
        return kq, ks, vq, vs

    def write_q8(self, layer: int, pos0: int, kq, ks, vq, vs) -> None:
        kq = np.ascontiguousarray(kq, np.int8).reshape(-1, self.kv_dim)
        vq = np.ascontiguousarray(vq, np.int8).reshape(-1, self.kv_dim)
        ks = np.ascontiguousarray(ks, np.float32).reshape(-1, self.kv_dim // 32)
        vs = np.ascontiguousarray(vs, np.float32).reshape(-1, self.kv_dim // 32)
        n = kq.shape[0]
        if not (vq.shape[0] == ks.shape[0] == vs.shape[0] == n):
            raise ValueError("write_q8: quants and scales disagree on the row count")
        call("llmp_kv_write_q8", self.handle, layer, pos0, n, _i8p(kq), _fp(ks), _i8p(vq), _fp(vs))

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    def read(self, layer: int, pos0: int, n: int):
        k = np.empty((n, self.kv_dim), np.float32)
        v = np.empty((n, self.kv_dim), np.float32)
        call("llmp_kv_read", self.handle, layer, pos0, n, _fp(k), _fp(v))
        return k, v

    def write(self, layer: int, pos0: int, k: Optional[np.ndarray], v: Optional[np.ndarray]) -> None:
        k = None if k is None else np.ascontiguousarray(k, np.float32).reshape(-1, self.kv_dim)
        v = None if v is None else np.ascontiguousarray(v, np.float32).reshape(-1, self.kv_dim)
        n = (k if k is not None else v).shape[0]
        call("llmp_kv_write", self.handle, layer, pos0, n, _fp(k), _fp(v))

    def layer_ptrs(self, layer: int):
        kp, vp = C.c_uint64(), C.c_uint64()
        call("llmp_kv_layer_ptrs", self.handle, layer, C.byref(kp), C.byref(vp))
        return kp.value, vp.value

    def clear(self, stream: int = 0) -> None:
        call("llmp_kv_clear", self.handle, stream)

    def destroy(self) -> None:
        if self.handle:
            call("llmp_kv_destroy", self.handle)
            self.handle = 0


@dataclass
class GgufTensor:
    """A projection weight as a GGUF file stores it: GGMLType id, [rows][cols], raw bytes."""
    type: int
    rows: int
    cols: int
    data: np.ndarray     # uint8, rows * row_bytes(type, cols)


@dataclass
class TransformerLayerWeights:
    """The attention half of TransformerLayerWeights: wq/wk/wv (or merged wqkv) and wo as
    GGUF tensors, norms and biases as fp32 arrays (None where the model has none)."""
    wq: Optional[GgufTensor] = None
    wk: Optional[GgufTensor] = None
    wv: Optional[GgufTensor] = None
    wqkv: Optional[GgufTensor] = None
    wo: Optional[GgufTensor] = None
    attnNorm: Optional[np.ndarray] = None
    postAttnNorm: Optional[np.ndarray] = None
    qBias: Optional[np.ndarray] = None
    kBias: Optional[np.ndarray] = None
    vBias: Optional[np.ndarray] = None
    woBias: Optional[np.ndarray] = None


def kernel_group(head_size: int, group: int) -> int:
    """The GQA group the library's kernels run a layer with (llmp_runtime's kernel_group): the
    group itself for head_dim 64/128/256/512 with groups 1-8, 96 with 1-4 (Phi-3) and 80 with 1-2
    (Phi-2); a larger group runs as several groups of its largest such divisor per cached KV
    head (GLM-4's 16 and 24 query heads per KV head as 2 and 3 groups of 8); 0 for a head size
    with no kernel."""
    limit = {64: 8, 128: 8, 256: 8, 512: 8, 96: 4, 80: 2}.get(head_size, 0)
    if group < 1 or limit == 0:
        return 0
    for g in range(min(group, limit), 0, -1):
        if group % g == 0:
            return g
    return 0


class HipForwardPass:
    """Attention section of a GPU-resident forward pass on MI355X.

    Mirrors the CudaForwardPass constructor's attention set-up (CudaForwardPass.java:346-416:
    RoPE table upload, per-layer zero-filled KV, QK-norm weights) and its attention API.
    `qk_norm` holds per-layer (q_weights, k_weights) arrays of head_size floats, or None."""

    def __init__(self, config: ModelConfig, max_seq_len: int,
                 qk_norm: Optional[Sequence[Optional[tuple]]] = None, device: int = 0,
                 kv_dtype: int = _lib.LLMP_KV_F32,
                 sinks: Optional[Sequence[Optional[np.ndarray]]] = None):
        if not HipForwardPass.isSupportedForAttention(config):
            raise LlmpError("HipForwardPass", 6, "configuration not supported by the HIP attention path")
        init(device)
        self.config = config
        self.max_seq_len = max_seq_len
        c = config
        self.kv = KvCache(c.block_count, max_seq_len, c.head_count_kv, c.head_size, kv_dtype)
        rope_dim = c.rope_dim_count or c.head_size
        # InferenceEngine.java:58-78: global table with linear scaling; local table for
        # Gemma 3 (theta 10000) and Gemma 4 (SWA theta) when a sliding window exists.  The MoE
        # engine takes the scaling factor as YaRN's instead (Qwen3MoEInferenceEngine.java:60-66)
        # and scales scores by mscale^2/sqrt(headSize) (:277-279).
        self.mscale = np.float32(1.0)
        if c.expert_count > 0 and c.rope_scaling_factor > 1.0:
            cos_g, sin_g, self.mscale = rope_table_yarn(
                rope_dim, max_seq_len, c.rope_freq_base, c.rope_scaling_factor,
                c.rope_orig_context_length, c.yarn_log_multiplier)
        else:
            linear = c.rope_scaling_factor if c.rope_scaling_factor > 1.0 else 1.0
            cos_g, sin_g = rope_table(rope_dim, max_seq_len, c.rope_freq_base, linear)
        call("llmp_rope_upload", self.kv.handle, _lib.LLMP_ROPE_SEL_GLOBAL, _fp(cos_g), _fp(sin_g),
             max_seq_len, rope_dim // 2)
        self.has_local_rope = False
        if c.sliding_window > 0 and c.architecture in (ARCH_GEMMA3, ARCH_GEMMA4):
            theta_l = 10000.0 if c.architecture == ARCH_GEMMA3 else c.rope_freq_base_swa
            cos_l, sin_l = rope_table(rope_dim, max_seq_len, theta_l)
            call("llmp_rope_upload", self.kv.handle, _lib.LLMP_ROPE_SEL_LOCAL, _fp(cos_l),
                 _fp(sin_l), max_seq_len, rope_dim // 2)
            self.has_local_rope = True
        for layer in range(c.block_count):
            w = qk_norm[layer] if qk_norm is not None else None
            self.configure_layer(layer, w)
            if sinks is not None and sinks[layer] is not None:
                self.set_sinks(layer, sinks[layer])
        self.gpuQ = DeviceBuffer(c.q_dim * 4)
        self.gpuK = DeviceBuffer(c.kv_dim * 4)
        self.gpuV = DeviceBuffer(c.kv_dim * 4)
        self.gpuXb2 = DeviceBuffer(c.q_dim * 4)
        self.gpuGate = DeviceBuffer(c.q_dim * 4)   # attention output gate (Qwen3.5)
        # [position, position + 1] as int32 (CudaForwardPass.gpuTokenParams, :138-141)
        self.gpuTokenParams = DeviceBuffer(8)

    # -- reflection-contract statics -------------------------------------------------------
    @staticmethod
    def isSupportedForAttention(config: ModelConfig, weights=None) -> bool:
        """CudaForwardPass.isSupportedForAttention (CudaForwardPass.java:1223-1244) rejects
        LayerNorm models; the HIP section also needs a head shape it has a kernel for."""
        if config.use_layer_norm:
            return False
        if config.head_count <= 0 or config.head_count_kv <= 0:
            return False
        if config.head_count % config.head_count_kv:
            return False
        group = config.head_count // config.head_count_kv
        if kernel_group(config.head_size, group) == 0:
            return False
        rd = config.rope_dim_count or config.head_size
        return rd % 2 == 0 and rd <= config.head_size

    def getGpuLayerCount(self) -> int:
        return self.config.block_count

    # -- set-up ------------------------------------------------------------------------------
    def configure_layer(self, layer: int, qk_norm: Optional[tuple]) -> None:
        c = self.config
        is_global = is_global_layer(c.architecture, layer, c.sliding_window_pattern, c.expert_count)
        irope_skip = c.no_rope_layer_interval > 0 and \
            layer % c.no_rope_layer_interval == c.no_rope_layer_interval - 1
        cohere_skip = c.use_no_pe_on_global_layers and is_global
        if irope_skip or cohere_skip:
            rope_sel = _lib.LLMP_ROPE_SEL_NONE
        elif self.has_local_rope and not is_global:
            rope_sel = _lib.LLMP_ROPE_SEL_LOCAL
        else:
            rope_sel = _lib.LLMP_ROPE_SEL_GLOBAL
        qw = kw = None
        if qk_norm is not None:
            qw = np.ascontiguousarray(qk_norm[0], np.float32)
            kw = np.ascontiguousarray(qk_norm[1], np.float32)
            assert qw.size == c.head_size and kw.size == c.head_size
        scale = float(c.attention_scale)
        if scale <= 0.0 and self.mscale != np.float32(1.0):
            # YaRN: mscale * mscale / (float) Math.sqrt(headSize) (Qwen3MoEInferenceEngine.java:279)
            scale = float((self.mscale * self.mscale) / np.float32(np.sqrt(c.head_size)))
        call("llmp_layer_config", self.kv.handle, layer, c.head_count, c.head_count_kv,
             c.head_size, c.resolved_rope_type(), rope_sel, c.sliding_window, int(is_global),
             scale, float(c.attn_logit_soft_cap), float(c.norm_eps), _fp(qw), _fp(kw))

    def set_sinks(self, layer: int, sinks: Optional[np.ndarray]) -> None:
        """Per-query-head attention-sink logits of a layer (GPT-OSS attn_sinks,
        Qwen3MoEInferenceEngine.java:88-95), or None to remove them."""
        if sinks is None:
            call("llmp_layer_sinks", self.kv.handle, layer, None)
            return
        s = np.ascontiguousarray(sinks, np.float32).reshape(-1)
        if s.size != self.config.head_count:
            raise ValueError(f"sinks: {s.size} values for {self.config.head_count} heads")
        call("llmp_layer_sinks", self.kv.handle, layer, _fp(s))

    # -- per-token API -------------------------------------------------------------------------
    def uploadQKV(self, q: np.ndarray, k: np.ndarray, v: np.ndarray) -> None:
        self.gpuQ.upload(np.ascontiguousarray(q, np.float32))
        self.gpuK.upload(np.ascontiguousarray(k, np.float32))
        self.gpuV.upload(np.ascontiguousarray(v, np.float32))

    def uploadGate(self, gate: np.ndarray) -> None:
        """Attention output gate for the next gated call (Qwen3.5 attnGate, [Hq*D])."""
        self.gpuGate.upload(np.ascontiguousarray(gate, np.float32).reshape(self.config.q_dim))

    def forwardAttentionPart(self, layerIdx: int, position: int, splits: int = 0,
                             stream: int = 0, gated: bool = False) -> None:
        """Steps 2b'-5 on the device buffers: gpuQ/gpuK/gpuV -> KV append -> gpuXb2 (times
        sigmoid(gpuGate) when gated, Qwen35InferenceEngine.java:580-583)."""
        if gated:
            call("llmp_attn_decode_ex", self.kv.handle, layerIdx, position, 0, self.gpuQ.ptr,
                 self.gpuK.ptr, self.gpuV.ptr, self.gpuGate.ptr, self.gpuXb2.ptr, splits, stream)
            return
        call("llmp_attn_decode", self.kv.handle, layerIdx, position, self.gpuQ.ptr, self.gpuK.ptr,
             self.gpuV.ptr, self.gpuXb2.ptr, splits, stream)

    # -- the attention half of the layer (projections + residual) --------------------------
    def setBlockConfig(self, dim: int, residual_scale: float = 0.0,
                       input_mode: int = _lib.LLMP_INPUT_F32) -> None:
        """embeddingLength and Granite's residualScale (0 = off) for forwardAttentionBlock.
        input_mode LLMP_INPUT_Q8_1: Q4_K, Q8_0, Q5_0, Q3_K, Q5_K, IQ4_NL and IQ4_XS projections
        on a Q8_1 copy of the input with int8 dot products (CudaForwardPass's default dp4a
        matvecs, CudaForwardPass.java:783-790, 216-226);
        LLMP_INPUT_F32: the CPU engine's fp32 arithmetic."""
        call("llmp_block_config", self.kv.handle, dim, float(residual_scale))
        call("llmp_block_input_mode", self.kv.handle, int(input_mode))
        self.dim = dim
        if getattr(self, "gpuX", None) is None or self.gpuX.nbytes < dim * 4:
            self.gpuX = DeviceBuffer(dim * 4)

    def uploadLayerWeights(self, layer: int, lw: TransformerLayerWeights) -> None:
        """Hands a layer's attention weights to the library (repacked on the device)."""
        h = self.kv.handle

        def put(slot, t: Optional[GgufTensor]):
            if t is None:
                call("llmp_layer_weight", h, layer, slot, 0, 0, 0, None, 0)
                return
            d = np.ascontiguousarray(t.data, np.uint8)
            call("llmp_layer_weight", h, layer, slot, t.type, t.rows, t.cols,
                 d.ctypes.data_as(C.c_void_p), d.nbytes)

        def vec(slot, a: Optional[np.ndarray]):
            if a is None:
                call("llmp_layer_weight", h, layer, slot, 0, 0, 0, None, 0)
                return
            a = np.ascontiguousarray(a, np.float32).reshape(-1)
            call("llmp_layer_weight", h, layer, slot, _lib.LLMP_GGML_F32, 1, a.size,
                 a.ctypes.data_as(C.c_void_p), a.nbytes)
        for slot, t in ((_lib.LLMP_W_Q, lw.wq), (_lib.LLMP_W_K, lw.wk), (_lib.LLMP_W_V, lw.wv),
                        (_lib.LLMP_W_QKV, lw.wqkv), (_lib.LLMP_W_O, lw.wo)):
            put(slot, t)
        for slot, a in ((_lib.LLMP_W_ATTN_NORM, lw.attnNorm), (_lib.LLMP_W_POST_ATTN_NORM, lw.postAttnNorm),
                        (_lib.LLMP_W_Q_BIAS, lw.qBias), (_lib.LLMP_W_K_BIAS, lw.kBias),
                        (_lib.LLMP_W_V_BIAS, lw.vBias), (_lib.LLMP_W_O_BIAS, lw.woBias)):
            vec(slot, a)

    def uploadX(self, x: np.ndarray) -> None:
        """The residual stream into gpuX (CudaForwardPass.uploadX)."""
        self.gpuX.upload(np.ascontiguousarray(x, np.float32).reshape(self.dim))

    def downloadX(self) -> np.ndarray:
        return self.gpuX.download(np.float32, self.dim)

    def forwardAttentionBlock(self, layerIdx: int, position: int, splits: int = 0,
                              stream: int = 0, device_position: bool = False) -> None:
        """CudaForwardPass.forwardAttentionPart steps 1-6c on gpuX: pre-norm, projections,
        attention, output projection, post-norm and residual (gpuX holds the post-attention
        residual afterwards).  device_position reads the position from gpuTokenParams."""
        d = self.gpuTokenParams.ptr if device_position else 0
        call("llmp_attn_block", self.kv.handle, layerIdx, position, d, self.gpuX.ptr, splits, stream)

    def uploadXBatch(self, x: np.ndarray) -> None:
        """Residual rows of n tokens, [n, dim] fp32, into gpuXBatch (for forwardAttentionBlockBatch)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.dim)
        if getattr(self, "gpuXBatch", None) is None or self.gpuXBatch.nbytes < x.nbytes:
            if getattr(self, "gpuXBatch", None) is not None:
                self.gpuXBatch.free()
            self.gpuXBatch = DeviceBuffer(x.nbytes)
        self.gpuXBatch.upload(x)

    def downloadXBatch(self, n_tokens: int) -> np.ndarray:
        return self.gpuXBatch.download(np.float32, n_tokens * self.dim).reshape(n_tokens, self.dim)

    def forwardAttentionBlockBatch(self, layerIdx: int, pos0: int, n_tokens: int,
                                   stream: int = 0) -> None:
        """The attention half of n_tokens tokens at positions pos0.. on gpuXBatch (the rows of
        LLMEngine.forwardBatch's tokens, LLMEngine.java:1019-1033): what n_tokens
        forwardAttentionBlock calls compute, each projection weight read once per 16 tokens."""
        call("llmp_attn_block_batch", self.kv.handle, layerIdx, pos0, n_tokens,
             self.gpuXBatch.ptr, stream)

    def updateTokenParams(self, position: int) -> None:
        """Store [position, position+1] in device memory (CudaForwardPass.updateTokenParams /
        uploadXAndUpdateParams, CudaForwardPass.java:1283-1292), for graph-captured calls."""
        self.gpuTokenParams.upload(np.array([position, position + 1], np.int32))

    def forwardAttentionPartDevicePosition(self, layerIdx: int, splits: int = 0,
                                           stream: int = 0) -> None:
        """Steps 2b'-5 at the position held in gpuTokenParams, read when the kernels run
        (capturable once and replayed per token, like the reference's graph mode)."""
        call("llmp_attn_decode_devpos", self.kv.handle, layerIdx, self.gpuTokenParams.ptr,
             self.gpuQ.ptr, self.gpuK.ptr, self.gpuV.ptr, self.gpuXb2.ptr, splits, stream)

    def forwardAttentionOnly(self, state: InferenceState, layerIdx: int, position: int,
                             splits: int = 0, gate: Optional[np.ndarray] = None) -> None:
        """Attention for one layer from host projections in `state` (state.q, state.k,
        state.v) into state.xb2 -- the contract of Attention.forwardFromProjections
        (Attention.java:284-367) that GpuForwardPass.java:207-241 relies on.  `gate` applies
        the Qwen3.5 output gate."""
        self.uploadQKV(state.q, state.k, state.v)
        if gate is not None:
            self.uploadGate(gate)
        self.forwardAttentionPart(layerIdx, position, splits, gated=gate is not None)
        state.xb2[:] = self.downloadXb2()

    def prefill(self, layerIdx: int, pos0: int, q: np.ndarray, k: np.ndarray,
                v: np.ndarray, gate: Optional[np.ndarray] = None) -> np.ndarray:
        """Attention for P tokens at positions pos0..pos0+P-1 in one call (a prompt, or the
        draft tokens of a speculative verification; the reference runs P sequential forwards,
        InferenceEngine.java:374-381, LLMEngine.java:1019-1033).  Inputs [P, Hq*D] /
        [P, kvDim] are fp32 projections (the CPU path's contract: rows bit-identical to P
        decode appends) or bf16 bit patterns (uint16); all three share one dtype.  Returns
        fp32 [P, Hq*D].  `gate` ([P, Hq*D] fp32) applies the Qwen3.5 output gate."""
        c = self.config
        qa, f32 = prompt_input(q, c.q_dim, "prefill q")
        ka, kf = prompt_input(k, c.kv_dim, "prefill k")
        va, vf = prompt_input(v, c.kv_dim, "prefill v")
        if not (f32 == kf == vf):
            raise TypeError("prefill: q, k and v must share one dtype")
        P = qa.shape[0]
        if ka.shape[0] != P or va.shape[0] != P:
            raise ValueError(f"prefill: {P} query rows but {ka.shape[0]} / {va.shape[0]} k / v rows")
        bq, bk, bv = DeviceBuffer(qa.nbytes), DeviceBuffer(ka.nbytes), DeviceBuffer(va.nbytes)
        bo = DeviceBuffer(P * c.q_dim * 4)
        bufs = [bq, bk, bv, bo]
        try:
            bq.upload(qa)
            bk.upload(ka)
            bv.upload(va)
            gptr = 0
            if gate is not None:
                g = np.ascontiguousarray(gate, np.float32).reshape(P, c.q_dim)
                bg = DeviceBuffer(g.nbytes)
                bufs.append(bg)
                bg.upload(g)
                gptr = bg.ptr
            call("llmp_attn_prefill_f32" if f32 else "llmp_attn_prefill_ex", self.kv.handle,
                 layerIdx, pos0, P, bq.ptr, bk.ptr, bv.ptr, gptr, bo.ptr, 0)
            return bo.download(np.float32, P * c.q_dim).reshape(P, c.q_dim)
        finally:
            for b in bufs:
                b.free()

    def decodePlan(self, layerIdx: int, position: int, splits: int = 0) -> dict:
        """The launch llmp_attn_decode would make for this call."""
        sp, wv, rps, st = C.c_int(), C.c_int(), C.c_int(), C.c_int()
        call("llmp_decode_plan", self.kv.handle, layerIdx, position, splits, C.byref(sp),
             C.byref(wv), C.byref(rps), C.byref(st))
        return {"splits": sp.value, "waves": wv.value, "rows_per_split": rps.value,
                "start": st.value}

    def downloadXb2(self) -> np.ndarray:
        return self.gpuXb2.download(np.float32, self.config.q_dim)

    def sync(self, stream: int = 0) -> None:
        call("llmp_stream_sync", stream)

    def close(self) -> None:
        for b in ("gpuQ", "gpuK", "gpuV", "gpuXb2", "gpuGate", "gpuTokenParams", "gpuX",
                  "gpuXBatch"):
            buf = getattr(self, b, None)
            if buf is not None:
                buf.free()
        if getattr(self, "kv", None) is not None:
            self.kv.destroy()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


@dataclass
class Gemma4State:
    """The buffers of Gemma4State the attention half uses (qLarge, kLarge, vLarge, xb2Large):
    sized for the larger head size; a layer uses the first Hq*headSize / Hkv*headSize floats."""
    q: np.ndarray
    k: np.ndarray
    v: np.ndarray
    xb2: np.ndarray


class Gemma4HipForwardPass:
    """Attention half of Gemma4InferenceEngine.forwardLayer (Gemma4InferenceEngine.java:
    295-420) on MI355X.

    Gemma 4 mixes sliding-window layers (head size `head_size`, RoPE theta
    rope_freq_base_swa) and full-attention layers (head size `key_length`, theta
    rope_freq_base with rope_freq_factors), picked by sliding_window_pattern
    (isSwaLayer, :184-189).  Each head size gets its own KV handle.  Per-head QK-norm and the
    weightless V-norm follow RMSNorm.apply's sequential order (llmp_layer_norm_mode), the
    attention scale is 1.0 (:372), and the last shared_kv_layers layers compute no K/V: they
    attend to the cache of the last own-KV layer of their type before the shared boundary
    (kvSourceLayer, :171-180) through llmp_attn_decode_shared.  Shared layers keep a
    configuration slot in their handle (their q-norm weights are their own); the planes of
    that slot stay unused.  qk_norm[layer] = (q_weights, k_weights) of that layer's head size,
    or None."""

    def __init__(self, config: ModelConfig, max_seq_len: int,
                 qk_norm: Optional[Sequence[Optional[tuple]]] = None, device: int = 0):
        c = config
        init(device)
        self.config = c
        self.max_seq_len = max_seq_len
        self.head_swa = c.head_size
        self.head_full = c.key_length if c.key_length > 0 else c.head_size
        L = c.block_count
        self.first_shared = L - c.shared_kv_layers
        self.kv = {}        # is_swa -> KvCache
        self.slot = []      # layer -> index inside its handle
        counts = {True: 0, False: 0}
        for layer in range(L):
            t = self.isSwaLayer(layer)
            self.slot.append(counts[t])
            counts[t] += 1
        rope_type = c.resolved_rope_type()
        for t, n in counts.items():
            if n == 0:
                continue
            D = self.head_size(t)
            kv = KvCache(n, max_seq_len, c.head_count_kv, D, _lib.LLMP_KV_F32)
            self.kv[t] = kv
            # Gemma4InferenceEngine.java:133-139: RoPE dim = head size of the layer type.
            theta = (c.rope_freq_base_swa or 10000.0) if t else c.rope_freq_base
            cos_t, sin_t = rope_table(D, max_seq_len, theta, 1.0,
                                      None if t else c.rope_freq_factors)
            call("llmp_rope_upload", kv.handle, _lib.LLMP_ROPE_SEL_GLOBAL, _fp(cos_t), _fp(sin_t),
                 max_seq_len, D // 2)
        for layer in range(L):
            t = self.isSwaLayer(layer)
            D = self.head_size(t)
            qw = kw = None
            w = qk_norm[layer] if qk_norm is not None else None
            if w is not None:
                qw = np.ascontiguousarray(w[0], np.float32)
                kw = np.ascontiguousarray(w[1], np.float32)
                assert qw.size == D and kw.size == D
            h = self.kv[t].handle
            call("llmp_layer_config", h, self.slot[layer], c.head_count, c.head_count_kv, D,
                 rope_type, _lib.LLMP_ROPE_SEL_GLOBAL, c.sliding_window if t else 0,
                 int(not t), 1.0, 0.0, float(c.norm_eps), _fp(qw), _fp(kw))
            call("llmp_layer_norm_mode", h, self.slot[layer],
                 _lib.LLMP_NORM_SEQUENTIAL | _lib.LLMP_NORM_V)
        Dmax = max(self.head_swa, self.head_full)
        self.gpuQ = DeviceBuffer(c.head_count * Dmax * 4)
        self.gpuK = DeviceBuffer(c.head_count_kv * Dmax * 4)
        self.gpuV = DeviceBuffer(c.head_count_kv * Dmax * 4)
        self.gpuXb2 = DeviceBuffer(c.head_count * Dmax * 4)

    def isSwaLayer(self, layer: int) -> bool:
        p = self.config.sliding_window_pattern
        if p is not None and layer < len(p):
            return bool(p[layer])
        return layer % 6 != 5

    def head_size(self, is_swa: bool) -> int:
        return self.head_swa if is_swa else self.head_full

    def hasOwnKv(self, layer: int) -> bool:
        return layer < self.first_shared

    def kvSourceLayer(self, layer: int) -> int:
        if self.hasOwnKv(layer):
            return layer
        return self.first_shared - 2 if self.isSwaLayer(layer) else self.first_shared - 1

    def createState(self) -> Gemma4State:
        c = self.config
        Dmax = max(self.head_swa, self.head_full)
        return Gemma4State(np.zeros(c.head_count * Dmax, np.float32),
                           np.zeros(c.head_count_kv * Dmax, np.float32),
                           np.zeros(c.head_count_kv * Dmax, np.float32),
                           np.zeros(c.head_count * Dmax, np.float32))

    def kv_cache(self, layer: int):
        """(KvCache, slot) holding `layer`'s own rows (its source layer's for shared layers)."""
        src = self.kvSourceLayer(layer)
        return self.kv[self.isSwaLayer(src)], self.slot[src]

    def forwardAttentionOnly(self, state: Gemma4State, layer: int, position: int,
                             splits: int = 0) -> None:
        """Steps 2-4 of forwardLayer from the projections in state.q (and state.k, state.v for
        layers with their own KV) into state.xb2 (the first Hq*headSize floats of each)."""
        c = self.config
        t = self.isSwaLayer(layer)
        D = self.head_size(t)
        qd, kvd = c.head_count * D, c.head_count_kv * D
        h = self.kv[t].handle
        self.gpuQ.upload(np.ascontiguousarray(state.q[:qd], np.float32))
        if self.hasOwnKv(layer):
            self.gpuK.upload(np.ascontiguousarray(state.k[:kvd], np.float32))
            self.gpuV.upload(np.ascontiguousarray(state.v[:kvd], np.float32))
            call("llmp_attn_decode_ex", h, self.slot[layer], position, 0, self.gpuQ.ptr,
                 self.gpuK.ptr, self.gpuV.ptr, 0, self.gpuXb2.ptr, splits, 0)
        else:
            src = self.kvSourceLayer(layer)
            call("llmp_attn_decode_shared", h, self.slot[layer], self.slot[src], position, 0,
                 self.gpuQ.ptr, 0, self.gpuXb2.ptr, splits, 0)
        state.xb2[:qd] = self.gpuXb2.download(np.float32, qd)

    def prefill(self, layer: int, pos0: int, q: np.ndarray,
                k: Optional[np.ndarray] = None,
                v: Optional[np.ndarray] = None) -> np.ndarray:
        """P tokens of one layer in one call ([P, Hq*D] / [P, Hkv*D], fp32 projections or
        bf16 bits (uint16), one dtype for all; k, v unused for shared layers).  Sliding-window
        layers only: the 512-dim full-attention heads have no prefill kernel
        (LLMP_ERR_UNSUPPORTED); the reference runs a prompt token by token."""
        c = self.config
        t = self.isSwaLayer(layer)
        D = self.head_size(t)
        qd, kvd = c.head_count * D, c.head_count_kv * D
        qa, f32 = prompt_input(q, qd, "prefill q")
        P = qa.shape[0]
        bufs = [DeviceBuffer(qa.nbytes), DeviceBuffer(P * qd * 4)]
        try:
            bufs[0].upload(qa)
            h = self.kv[t].handle
            if self.hasOwnKv(layer):
                ka, kf = prompt_input(k, kvd, "prefill k")
                va, vf = prompt_input(v, kvd, "prefill v")
                if not (f32 == kf == vf) or ka.shape[0] != P or va.shape[0] != P:
                    raise TypeError("prefill: q, k and v must share one dtype and row count")
                bk, bv = DeviceBuffer(ka.nbytes), DeviceBuffer(va.nbytes)
                bufs += [bk, bv]
                bk.upload(ka)
                bv.upload(va)
                call("llmp_attn_prefill_f32" if f32 else "llmp_attn_prefill_ex", h,
                     self.slot[layer], pos0, P, bufs[0].ptr, bk.ptr, bv.ptr, 0, bufs[1].ptr, 0)
            else:
                call("llmp_attn_prefill_shared_f32" if f32 else "llmp_attn_prefill_shared", h,
                     self.slot[layer], self.slot[self.kvSourceLayer(layer)], pos0, P,
                     bufs[0].ptr, 0, bufs[1].ptr, 0)
            return bufs[1].download(np.float32, P * qd).reshape(P, qd)
        finally:
            for b in bufs:
                b.free()

    def close(self) -> None:
        for b in (self.gpuQ, self.gpuK, self.gpuV, self.gpuXb2):
            b.free()
        for kv in self.kv.values():
            kv.destroy()
        self.kv = {}

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
