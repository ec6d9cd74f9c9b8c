"""Seeded decode-attention cases run through both the HIP path (HipForwardPass over
libllmp_hip.so) and the CPU oracle, with the comparison the path must pass:
  - output: max |gpu - oracle| <= 1e-4 (and <= 1e-4 + 1e-3*|oracle| elementwise);
  - cache: every row of the layer read back with llmp_kv_read is bit-identical to the
    oracle's cache after its own append (KV append and position indexing are exact).
"""
from __future__ import annotations

import sys
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from llmplayer_amd import hip_forward_pass as hfp
from oracle import oracle as orc

ATOL = 1e-4   # max-abs bar on the attention output
RTOL = 1e-3   # relative bar on the attention output

_ORC_ARCH = {hfp.ARCH_GEMMA2: orc.ARCH_GEMMA2, hfp.ARCH_GEMMA3: orc.ARCH_GEMMA3,
             hfp.ARCH_GPT_OSS: orc.ARCH_GPT_OSS, hfp.ARCH_COHERE2: orc.ARCH_COHERE2}


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _yarn(c: hfp.ModelConfig) -> bool:
    """The MoE engines take rope_scaling_factor as YaRN's (Qwen3MoEInferenceEngine.java:60-66)."""
    return c.expert_count > 0 and c.rope_scaling_factor > 1.0


def oracle_config(c: hfp.ModelConfig, max_seq: int, sinks=None) -> orc.OracleConfig:
    arch = _ORC_ARCH.get(c.architecture, orc.ARCH_OTHER)
    if c.architecture == hfp.ARCH_GPT_OSS and c.expert_count > 0:
        arch = orc.ARCH_GPT_OSS_MOE
    scale = c.attention_scale
    if scale <= 0 and _yarn(c):   # mscale^2 / (float) sqrt(headSize), :277-279
        _, _, ms = orc.rope_tables_yarn(c.rope_dim_count or c.head_size, 1, c.rope_freq_base,
                                        c.rope_scaling_factor, c.rope_orig_context_length,
                                        c.yarn_log_multiplier)
        scale = float((ms * ms) / np.float32(np.sqrt(c.head_size)))
    return orc.OracleConfig(
        n_heads=c.head_count, n_kv_heads=c.head_count_kv, head_size=c.head_size,
        max_seq=max_seq, rope_type=c.resolved_rope_type(), rope_dim=c.rope_dim_count or c.head_size,
        norm_eps=c.norm_eps, sliding_window=c.sliding_window, attention_scale=scale,
        softcap=c.attn_logit_soft_cap, arch=arch,
        no_rope_interval=c.no_rope_layer_interval, nope_on_global=c.use_no_pe_on_global_layers,
        sinks=sinks)


def oracle_tables(c: hfp.ModelConfig, max_seq: int, layer: int):
    """The table Attention.java:317 selects for `layer` (None for a NoPE layer)."""
    rd = c.rope_dim_count or c.head_size
    is_global = hfp.is_global_layer(c.architecture, layer, c.sliding_window_pattern)
    irope = c.no_rope_layer_interval > 0 and layer % c.no_rope_layer_interval == c.no_rope_layer_interval - 1
    if irope or (c.use_no_pe_on_global_layers and is_global):
        return None, None
    if c.sliding_window > 0 and c.architecture in (hfp.ARCH_GEMMA3, hfp.ARCH_GEMMA4) and not is_global:
        theta = 10000.0 if c.architecture == hfp.ARCH_GEMMA3 else c.rope_freq_base_swa
        return orc.rope_tables(rd, max_seq, theta)
    if _yarn(c):
        cs, sn, _ = orc.rope_tables_yarn(rd, max_seq, c.rope_freq_base, c.rope_scaling_factor,
                                         c.rope_orig_context_length, c.yarn_log_multiplier)
        return cs, sn
    lin = c.rope_scaling_factor if c.rope_scaling_factor > 1.0 else 1.0
    return orc.rope_tables(rd, max_seq, c.rope_freq_base, lin)


@dataclass
class LayerData:
    kc: np.ndarray      # [max_seq, kvDim] oracle cache (reference layout)
    vc: np.ndarray
    q: np.ndarray
    k: np.ndarray
    v: np.ndarray
    qk_norm: Optional[tuple] = None


def make_layer(c: hfp.ModelConfig, max_seq: int, filled: int, seed: int, k_scale: float = 1.0,
               qk_norm: bool = False) -> LayerData:
    """Cache rows [0, filled) and the new token's q/k/v ~ N(0,1) (K scaled by k_scale);
    QK-norm gammas ~ U(0.5, 1.5)."""
    rng = np.random.default_rng(seed)
    kv = c.kv_dim
    kc = np.zeros((max_seq, kv), np.float32)
    vc = np.zeros((max_seq, kv), np.float32)
    kc[:filled] = rng.standard_normal((filled, kv), dtype=np.float32)
    if k_scale != 1.0:
        kc[:filled] *= np.float32(k_scale)
    vc[:filled] = rng.standard_normal((filled, kv), dtype=np.float32)
    q = rng.standard_normal(c.q_dim, dtype=np.float32)
    k = rng.standard_normal(kv, dtype=np.float32) * np.float32(k_scale)
    v = rng.standard_normal(kv, dtype=np.float32)
    w = None
    if qk_norm:
        w = (rng.uniform(0.5, 1.5, c.head_size).astype(np.float32),
             rng.uniform(0.5, 1.5, c.head_size).astype(np.float32))
    return LayerData(kc, vc, q, k, v, w)


def oracle_call(c: hfp.ModelConfig, max_seq: int, d: LayerData, layer: int, pos: int,
                n_threads: int = 8, sinks=None, gate=None):
    """Runs the oracle on a copy of the layer's cache; returns (out, kc_after, vc_after)."""
    oc = oracle_config(c, max_seq, sinks)
    cs, sn = oracle_tables(c, max_seq, layer)
    kc, vc = d.kc.copy(), d.vc.copy()
    qw, kw = (d.qk_norm if d.qk_norm is not None else (None, None))
    out, _, _ = orc.forward_from_projections(oc, kc, vc, d.q, d.k, d.v, layer, pos, qnorm_w=qw,
                                             knorm_w=kw, rope_cos=cs, rope_sin=sn,
                                             n_threads=n_threads, gate=gate)
    return out, kc, vc


def compare_out(got: np.ndarray, want: np.ndarray, what: str) -> float:
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = ATOL + RTOL * np.abs(want.astype(np.float64))
    worst = float(err.max())
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert worst <= ATOL and (err <= bound).all(), (
        f"{what}: max abs err {worst:.3e} (bar {ATOL}); "
        f"{int((err > bound).sum())} elements above {ATOL} + {RTOL}*|ref|")
    return worst


def compare_cache(fp: hfp.HipForwardPass, layer: int, kc: np.ndarray, vc: np.ndarray, what: str,
                  rows: Optional[tuple] = None) -> None:
    lo, hi = rows if rows is not None else (0, kc.shape[0])
    gk, gv = fp.kv.read(layer, lo, hi - lo)
    if not np.array_equal(gk, kc[lo:hi]):
        bad = np.argwhere(gk != kc[lo:hi])
        raise AssertionError(f"{what}: K cache differs at {len(bad)} elements, first "
                             f"(row {bad[0][0] + lo}, col {bad[0][1]}): "
                             f"{gk[tuple(bad[0])]!r} vs {kc[lo:hi][tuple(bad[0])]!r}")
    if not np.array_equal(gv, vc[lo:hi]):
        bad = np.argwhere(gv != vc[lo:hi])
        raise AssertionError(f"{what}: V cache differs at {len(bad)} elements, first row {bad[0][0] + lo}")


# ------------------------------------------------------------------- Q8_0 cache (KVCache.Mode.Q8_0)
@dataclass
class LayerDataQ8:
    kq: np.ndarray      # [max_seq, kvDim] int8 (KVCache.keyQuants layout)
    ks: np.ndarray      # [max_seq, kvDim/32] fp32 (KVCache.keyScales layout)
    vq: np.ndarray
    vs: np.ndarray
    q: np.ndarray
    k: np.ndarray
    v: np.ndarray
    qk_norm: Optional[tuple] = None


def quantize_rows(x: np.ndarray, mode: int = orc.Q8_SCALAR):
    """Rows [n, kvDim] -> (quants [n, kvDim] int8, scales [n, kvDim/32]) by the oracle's
    quantizer for `mode` (blocks of 32 never straddle rows: kvDim is a multiple of 32)."""
    n, kv = x.shape
    q, s = orc.q8_quantize(x.reshape(-1), mode)
    return q.reshape(n, kv), s.reshape(n, kv // 32)


def make_layer_q8(c: hfp.ModelConfig, max_seq: int, filled: int, seed: int, k_scale: float = 1.0,
                  qk_norm: bool = False, mode: int = orc.Q8_SCALAR) -> LayerDataQ8:
    """make_layer's rows [0, filled) quantized to Q8_0; rows beyond stay zero."""
    d = make_layer(c, max_seq, filled, seed, k_scale, qk_norm)
    kq, ks = quantize_rows(d.kc, mode)
    vq, vs = quantize_rows(d.vc, mode)
    return LayerDataQ8(kq, ks, vq, vs, d.q, d.k, d.v, d.qk_norm)


def oracle_call_q8(c: hfp.ModelConfig, max_seq: int, d: LayerDataQ8, layer: int, pos: int,
                   n_threads: int = 8, mode: int = orc.Q8_SCALAR, sinks=None, gate=None):
    """The oracle over copies of the Q8_0 cache; returns (out, (kq, ks, vq, vs) after)."""
    oc = oracle_config(c, max_seq, sinks)
    cs, sn = oracle_tables(c, max_seq, layer)
    kq, ks, vq, vs = d.kq.copy(), d.ks.copy(), d.vq.copy(), d.vs.copy()
    qw, kw = (d.qk_norm if d.qk_norm is not None else (None, None))
    out, _, _ = orc.forward_from_projections_q8(oc, kq, ks, vq, vs, d.q, d.k, d.v, layer, pos,
                                                qnorm_w=qw, knorm_w=kw, rope_cos=cs, rope_sin=sn,
                                                n_threads=n_threads, mode=mode, gate=gate)
    return out, (kq, ks, vq, vs)


def compare_cache_q8(fp: hfp.HipForwardPass, layer: int, want: tuple, what: str,
                     rows: Optional[tuple] = None) -> None:
    """Quants and scales read back with llmp_kv_read_q8 bit-identical to the oracle's."""
    lo, hi = rows if rows is not None else (0, want[0].shape[0])
    got = fp.kv.read_q8(layer, lo, hi - lo)
    for name, g, w in zip(("K quants", "K scales", "V quants", "V scales"), got, want):
        w = w[lo:hi]
        if not np.array_equal(g.view(np.uint8) if g.dtype == np.int8 else g.view(np.uint32),
                              w.view(np.uint8) if w.dtype == np.int8 else w.view(np.uint32)):
            bad = np.argwhere(g != w)
            first = tuple(bad[0]) if len(bad) else (0, 0)
            raise AssertionError(f"{what}: {name} differ at {len(bad)} elements, first "
                                 f"(row {first[0] + lo}, col {first[1]}): {g[first]!r} vs {w[first]!r}")
