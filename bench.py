#!/usr/bin/env python3
"""Decode-attention benchmark on one MI355X (BASELINE.json metric).

A step is one decode attention layer-call (QK-norm/RoPE prep, KV append, split-K
QK^T/softmax/PV and the log-sum-exp combine) at the Llama-3.2-3B head shape (24 query heads,
8 KV heads, head_dim 128, fp32 KV) for one new token at position ctx-1.  Successive steps
rotate over enough layer caches (>= 2 GiB) that every step reads its KV from HBM rather than
the 256 MB Infinity Cache.  Inputs are synthetic N(0,1) (K x 0.5) and resident in HBM before
the timed region.

value = KV-read GB/s = (2 * ctx * Hkv * D * 4 bytes) / (time per layer-call), whole region.
roofline.achieved = the same bytes / the split-K kernel's mean duration (HIP events around
each launch, on the library stream the kernel runs on).
cpu_baseline = the CPU restatement of the reference's Java attention (oracle/, parallel over
query heads like Attention.java:343), timed on this host on a bounded sample.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_GBPS = 8000.0            # MI355X HBM3E peak
HQ, HKV, D = 24, 8, 128       # Llama-3.2-3B head shape
THETA = 500000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def kv_bytes(ctx: int, q8: bool = False) -> int:
    """K and V bytes one layer-call reads: fp32 rows, or Q8_0 quants plus a 4-byte scale per
    32 values (1.125 bytes per value)."""
    return 2 * ctx * HKV * (D + D // 32 * 4) if q8 else 2 * ctx * HKV * D * 4


def fill_caches(fp, c, ctx: int, n_layers: int, q8: bool, rng) -> None:
    """Rows [0, ctx-1) of every rotated layer cache: N(0,1) fp32 rows (K x 0.5), or synthetic
    Q8_0 rows (uniform quants, block scales of the size N(0,1) blocks give, ~max/127)."""
    if q8:
        kq = rng.integers(-127, 128, (ctx - 1, c.kv_dim), dtype=np.int8)
        vq = rng.integers(-127, 128, (ctx - 1, c.kv_dim), dtype=np.int8)
        ks = np.full((ctx - 1, c.kv_dim // 32), 1.2 / 127, np.float32)
        vs = np.full((ctx - 1, c.kv_dim // 32), 2.4 / 127, np.float32)
        for layer in range(n_layers):
            fp.kv.write_q8(layer, 0, kq, ks, vq, vs)
            log(f"[bench] Q8_0 layer cache {layer + 1}/{n_layers} filled")
    else:
        kc = rng.standard_normal((ctx - 1, c.kv_dim), dtype=np.float32) * np.float32(0.5)
        vc = rng.standard_normal((ctx - 1, c.kv_dim), dtype=np.float32)
        for layer in range(n_layers):
            fp.kv.write(layer, 0, kc, vc)


def gpu_run(ctx: int, steps: int, warmup: int, splits: int, rotate_bytes: int,
            q8: bool = False) -> dict:
    from llmplayer_amd import _lib
    from llmplayer_amd import hip_forward_pass as hfp

    per_layer = kv_bytes(ctx, q8)
    n_layers = max(1, math.ceil(rotate_bytes / per_layer))
    c = hfp.ModelConfig(HQ, HKV, D, n_layers, architecture=hfp.ARCH_LLAMA, rope_freq_base=THETA)
    log(f"[bench] ctx {ctx}{' Q8_0' if q8 else ''}: {n_layers} layer caches x "
        f"{per_layer / 2**20:.0f} MiB")
    fp = hfp.HipForwardPass(c, ctx, kv_dtype=_lib.LLMP_KV_Q8_0 if q8 else _lib.LLMP_KV_F32)
    try:
        rng = np.random.default_rng(2024)
        fill_caches(fp, c, ctx, n_layers, q8, rng)
        fp.uploadQKV(rng.standard_normal(c.q_dim, dtype=np.float32),
                     rng.standard_normal(c.kv_dim, dtype=np.float32) * np.float32(0.5),
                     rng.standard_normal(c.kv_dim, dtype=np.float32))
        pos = ctx - 1
        h = fp.kv.handle
        plan = fp.decodePlan(0, pos, splits)
        for i in range(warmup):
            fp.forwardAttentionPart(i % n_layers, pos, splits)
        fp.sync()
        # Timed region: the K layer-calls captured once as a HIP graph and replayed, so the
        # GPU time is not bounded by per-call host launch cost (the reference's production
        # decode replays a CUDA graph the same way, CudaForwardPass.java:1760-1812).
        g = C.c_uint64()
        _lib.call("llmp_graph_begin", 0)
        for i in range(steps):
            fp.forwardAttentionPart(i % n_layers, pos, splits)
        _lib.call("llmp_graph_end", 0, C.byref(g))
        _lib.call("llmp_graph_launch", g.value, 0)
        fp.sync()
        e0, e1 = C.c_uint64(), C.c_uint64()
        _lib.call("llmp_event_create", C.byref(e0))
        _lib.call("llmp_event_create", C.byref(e1))
        _lib.call("llmp_event_record", e0.value, 0)
        _lib.call("llmp_graph_launch", g.value, 0)
        _lib.call("llmp_event_record", e1.value, 0)
        _lib.call("llmp_event_sync", e1.value)
        ms = C.c_float()
        _lib.call("llmp_event_elapsed_ms", C.byref(ms), e0.value, e1.value)
        _lib.call("llmp_graph_destroy", g.value)
        # Eager pass with a HIP event pair around every kernel launch (library stream): the
        # per-kernel mean durations behind roofline.achieved, and the eager per-call time.
        _lib.call("llmp_profile_reset", h)
        _lib.call("llmp_profile_enable", h, 1)
        _lib.call("llmp_event_record", e0.value, 0)
        for i in range(steps):
            fp.forwardAttentionPart(i % n_layers, pos, splits)
        _lib.call("llmp_event_record", e1.value, 0)
        _lib.call("llmp_event_sync", e1.value)
        ms_eager = C.c_float()
        _lib.call("llmp_event_elapsed_ms", C.byref(ms_eager), e0.value, e1.value)
        _lib.call("llmp_profile_enable", h, 0)
        res = {}
        for kind, name in ((_lib.LLMP_PROF_DECODE_SPLIT, "split"),
                           (_lib.LLMP_PROF_DECODE_REDUCE, "reduce")):
            cnt, tot = C.c_int(), C.c_double()
            _lib.call("llmp_profile_read", h, kind, C.byref(cnt), C.byref(tot))
            res[name] = (cnt.value, tot.value)
        _lib.call("llmp_event_destroy", e0.value)
        _lib.call("llmp_event_destroy", e1.value)
    finally:
        fp.close()
    ms_per_step = ms.value / steps
    split_ms = res["split"][1] / max(1, res["split"][0])
    reduce_ms = res["reduce"][1] / res["reduce"][0] if res["reduce"][0] else 0.0
    return {"ctx": ctx, "n_layers": n_layers, "ms_per_step": ms_per_step,
            "us_per_layer_call_eager": ms_eager.value / steps * 1e3,
            "us_per_layer_call": ms_per_step * 1e3,
            "kv_read_gbps": per_layer / (ms_per_step * 1e-3) / 1e9,
            "split_kernel_us": split_ms * 1e3, "reduce_kernel_us": reduce_ms * 1e3,
            "split_launches": res["split"][0], "plan": plan}


def prefill_run(P: int, steps: int, q8: bool = False) -> dict:
    """C5: prefill attention of P prompt tokens (Llama-3.2-1B shape 32/8/64, bf16 Q/K/V
    N(0,1), causal) in one llmp_attn_prefill call (exact K/V append + MFMA attention), over
    an fp32 or a Q8_0 cache.  Timed as a graph replay of `steps` calls; per-kernel means from
    an eager profiled pass."""
    from llmplayer_amd import _lib
    from llmplayer_amd import hip_forward_pass as hfp
    c = hfp.ModelConfig(32, 8, 64, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=THETA)
    fp = hfp.HipForwardPass(c, P, kv_dtype=_lib.LLMP_KV_Q8_0 if q8 else _lib.LLMP_KV_F32)
    bufs = []
    try:
        rng = np.random.default_rng(5)
        arrs = [hfp.to_bf16(rng.standard_normal((P, n), dtype=np.float32))
                for n in (c.q_dim, c.kv_dim, c.kv_dim)]
        for a in arrs:
            b = hfp.DeviceBuffer(a.nbytes)
            b.upload(a)
            bufs.append(b)
        out = hfp.DeviceBuffer(P * c.q_dim * 4)
        bufs.append(out)
        args = (fp.kv.handle, 0, 0, P, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, out.ptr, 0)
        for _ in range(3):
            _lib.call("llmp_attn_prefill", *args)
        g = C.c_uint64()
        _lib.call("llmp_graph_begin", 0)
        for _ in range(steps):
            _lib.call("llmp_attn_prefill", *args)
        _lib.call("llmp_graph_end", 0, C.byref(g))
        _lib.call("llmp_graph_launch", g.value, 0)
        _lib.call("llmp_stream_sync", 0)
        e0, e1 = C.c_uint64(), C.c_uint64()
        _lib.call("llmp_event_create", C.byref(e0))
        _lib.call("llmp_event_create", C.byref(e1))
        _lib.call("llmp_event_record", e0.value, 0)
        _lib.call("llmp_graph_launch", g.value, 0)
        _lib.call("llmp_event_record", e1.value, 0)
        _lib.call("llmp_event_sync", e1.value)
        ms = C.c_float()
        _lib.call("llmp_event_elapsed_ms", C.byref(ms), e0.value, e1.value)
        _lib.call("llmp_graph_destroy", g.value)
        _lib.call("llmp_event_destroy", e0.value)
        _lib.call("llmp_event_destroy", e1.value)
        h = fp.kv.handle
        _lib.call("llmp_profile_reset", h)
        _lib.call("llmp_profile_enable", h, 1)
        for _ in range(steps):
            _lib.call("llmp_attn_prefill", *args)
        _lib.call("llmp_profile_enable", h, 0)
        res = {}
        for kind, name in ((_lib.LLMP_PROF_PREFILL_APPEND, "append"),
                           (_lib.LLMP_PROF_PREFILL_ATTN, "attn")):
            cnt, tot = C.c_int(), C.c_double()
            _lib.call("llmp_profile_read", h, kind, C.byref(cnt), C.byref(tot))
            res[name] = tot.value / max(1, cnt.value) * 1e3
    finally:
        for b in bufs:
            b.free()
        fp.close()
    us = ms.value / steps * 1e3
    flops = 4.0 * c.head_count * c.head_size * P * (P + 1) / 2   # causal QK^T + PV
    return {"P": P, "us_per_call": round(us, 2), "attn_kernel_us": round(res["attn"], 2),
            "append_kernel_us": round(res["append"], 2),
            "causal_tflops": round(flops / (us * 1e-6) / 1e12, 2),
            "attn_kernel_causal_tflops": round(flops / (res["attn"] * 1e-6) / 1e12, 2),
            "mfma_tflops_bf16x3": round(3 * flops / (res["attn"] * 1e-6) / 1e12, 2)}


def verify_run(ctx: int, K: int, steps: int, rotate_bytes: int, q8: bool = False) -> dict:
    """Speculative verification at the C3 shape: K draft tokens at positions ctx-K..ctx-1 in
    one llmp_attn_prefill call over a (ctx-K)-row fp32 or Q8_0 cache (the reference runs K
    sequential forwards, LLMEngine.java:1019-1033).  Layer caches rotate over >= 2 GiB; graph
    replay."""
    from llmplayer_amd import _lib
    from llmplayer_amd import hip_forward_pass as hfp
    per_layer = kv_bytes(ctx, q8)
    n_layers = max(1, math.ceil(rotate_bytes / per_layer))
    c = hfp.ModelConfig(HQ, HKV, D, n_layers, architecture=hfp.ARCH_LLAMA, rope_freq_base=THETA)
    fp = hfp.HipForwardPass(c, ctx, kv_dtype=_lib.LLMP_KV_Q8_0 if q8 else _lib.LLMP_KV_F32)
    bufs = []
    try:
        rng = np.random.default_rng(7)
        fill_caches(fp, c, ctx - K + 1, n_layers, q8, rng)
        arrs = [hfp.to_bf16(rng.standard_normal((K, n), dtype=np.float32))
                for n in (c.q_dim, c.kv_dim, c.kv_dim)]
        for arr in arrs:
            b = hfp.DeviceBuffer(arr.nbytes)
            b.upload(arr)
            bufs.append(b)
        out = hfp.DeviceBuffer(K * c.q_dim * 4)
        bufs.append(out)
        pos0 = ctx - K
        call = lambda layer: _lib.call("llmp_attn_prefill", fp.kv.handle, layer, pos0, K,
                                       bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, out.ptr, 0)
        for i in range(n_layers):
            call(i)
        _lib.call("llmp_stream_sync", 0)
        g = C.c_uint64()
        _lib.call("llmp_graph_begin", 0)
        for i in range(steps):
            call(i % n_layers)
        _lib.call("llmp_graph_end", 0, C.byref(g))
        _lib.call("llmp_graph_launch", g.value, 0)
        _lib.call("llmp_stream_sync", 0)
        e0, e1 = C.c_uint64(), C.c_uint64()
        _lib.call("llmp_event_create", C.byref(e0))
        _lib.call("llmp_event_create", C.byref(e1))
        _lib.call("llmp_event_record", e0.value, 0)
        _lib.call("llmp_graph_launch", g.value, 0)
        _lib.call("llmp_event_record", e1.value, 0)
        _lib.call("llmp_event_sync", e1.value)
        ms = C.c_float()
        _lib.call("llmp_event_elapsed_ms", C.byref(ms), e0.value, e1.value)
        _lib.call("llmp_graph_destroy", g.value)
        _lib.call("llmp_event_destroy", e0.value)
        _lib.call("llmp_event_destroy", e1.value)
    finally:
        for b in bufs:
            b.free()
        fp.close()
    us = ms.value / steps * 1e3
    return {"K": K, "ctx": ctx, "us_per_call": round(us, 2),
            "kv_read_gbps": round(kv_bytes(ctx - K, q8) / (us * 1e-6) / 1e9, 1)}


def synthetic_gguf(t: int, rows: int, cols: int, rng) -> np.ndarray:
    """Random GGUF-layout bytes of type t (Q4_K or Q6_K) with finite fp16 scale fields:
    uniform quants and scale bytes, super-block scales 2^-10 (d) and 2^-12 (dmin)."""
    ns = cols // 256
    if t == 12:     # Q4_K: d, dmin (fp16), 12 scale bytes, 128 nibble bytes
        b = rng.integers(0, 256, (rows, ns, 144), dtype=np.uint8)
        b[:, :, 0:2] = np.frombuffer(np.float16(2.0 ** -10).tobytes(), np.uint8)
        b[:, :, 2:4] = np.frombuffer(np.float16(2.0 ** -12).tobytes(), np.uint8)
    else:           # Q6_K: ql, qh, 16 int8 scales, d (fp16) at byte 208
        b = rng.integers(0, 256, (rows, ns, 210), dtype=np.uint8)
        b[:, :, 208:210] = np.frombuffer(np.float16(2.0 ** -12).tobytes(), np.uint8)
    return b.reshape(-1)


def block_run(ctx: int, steps: int, n_layers: int = 28, q8_input: bool = False) -> dict:
    """The attention half of a C3 (Llama-3.2-3B, dim 3072) layer with the Q4_K_M weight mix
    (Q4_K for q, k, o; Q6_K for v): pre-norm, projections, attention at ctx, output projection
    and residual, as a graph replay over n_layers layers with their own weights and caches.
    q8_input: the Q4_K projections on the Q8_1-quantised input (the reference GPU's int8
    matvecs) instead of the fp32 input."""
    from llmplayer_amd import _lib
    from llmplayer_amd import hip_forward_pass as hfp
    dim = 3072
    c = hfp.ModelConfig(HQ, HKV, D, n_layers, architecture=hfp.ARCH_LLAMA, rope_freq_base=THETA)
    fp = hfp.HipForwardPass(c, ctx)
    try:
        rng = np.random.default_rng(11)
        fill_caches(fp, c, ctx, n_layers, False, rng)
        fp.setBlockConfig(dim, 0.0, _lib.LLMP_INPUT_Q8_1 if q8_input else _lib.LLMP_INPUT_F32)
        wbytes = 0
        for layer in range(n_layers):
            lw = hfp.TransformerLayerWeights(attnNorm=np.ones(dim, np.float32))
            for name, t, rows, cols in (("wq", 12, c.q_dim, dim), ("wk", 12, c.kv_dim, dim),
                                        ("wv", 14, c.kv_dim, dim), ("wo", 12, dim, c.q_dim)):
                data = synthetic_gguf(t, rows, cols, rng)
                setattr(lw, name, hfp.GgufTensor(t, rows, cols, data))
                if layer == 0:
                    wbytes += data.nbytes
            fp.uploadLayerWeights(layer, lw)
        fp.uploadX(rng.standard_normal(dim).astype(np.float32))
        call = lambda layer: _lib.call("llmp_attn_block", fp.kv.handle, layer, ctx - 1, 0,
                                       fp.gpuX.ptr, 0, 0)
        for i in range(n_layers):
            call(i)
        _lib.call("llmp_stream_sync", 0)
        g = C.c_uint64()
        _lib.call("llmp_graph_begin", 0)
        for i in range(steps):
            call(i % n_layers)
        _lib.call("llmp_graph_end", 0, C.byref(g))
        _lib.call("llmp_graph_launch", g.value, 0)
        _lib.call("llmp_stream_sync", 0)
        e0, e1 = C.c_uint64(), C.c_uint64()
        _lib.call("llmp_event_create", C.byref(e0))
        _lib.call("llmp_event_create", C.byref(e1))
        _lib.call("llmp_event_record", e0.value, 0)
        _lib.call("llmp_graph_launch", g.value, 0)
        _lib.call("llmp_event_record", e1.value, 0)
        _lib.call("llmp_event_sync", e1.value)
        ms = C.c_float()
        _lib.call("llmp_event_elapsed_ms", C.byref(ms), e0.value, e1.value)
        _lib.call("llmp_graph_destroy", g.value)
        _lib.call("llmp_event_destroy", e0.value)
        _lib.call("llmp_event_destroy", e1.value)
    finally:
        fp.close()
    us = ms.value / steps * 1e3
    return {"ctx": ctx, "weights": "Q4_K_M mix (Q4_K q/k/o, Q6_K v)", "dim": dim,
            "input": "Q8_1 (int8 dot products for Q4_K)" if q8_input else "fp32",
            "us_per_layer_call": round(us, 2), "weight_bytes_per_layer": wbytes,
            "kv_bytes_per_layer": kv_bytes(ctx), "layers_rotated": n_layers}


def cpu_baseline(ctx: int, seconds: float) -> dict:
    """The oracle (CPU restatement of Attention.forwardFromProjections) on one layer-call of
    the same shape, parallel over query heads; median over a bounded sample."""
    from oracle import oracle as orc
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    threads = max(1, min(16, avail))
    oc = orc.OracleConfig(HQ, HKV, D, ctx, rope_type=0)
    rng = np.random.default_rng(2024)
    kc = np.zeros((ctx, HKV * D), np.float32)
    vc = np.zeros((ctx, HKV * D), np.float32)
    kc[:ctx - 1] = rng.standard_normal((ctx - 1, HKV * D), dtype=np.float32) * np.float32(0.5)
    vc[:ctx - 1] = rng.standard_normal((ctx - 1, HKV * D), dtype=np.float32)
    q = rng.standard_normal(HQ * D, dtype=np.float32)
    k = rng.standard_normal(HKV * D, dtype=np.float32) * np.float32(0.5)
    v = rng.standard_normal(HKV * D, dtype=np.float32)
    cs, sn = orc.rope_tables(D, ctx, THETA)
    for _ in range(2):
        orc.forward_from_projections(oc, kc, vc, q, k, v, 0, ctx - 1, rope_cos=cs, rope_sin=sn,
                                     n_threads=threads)
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        orc.forward_from_projections(oc, kc, vc, q, k, v, 0, ctx - 1, rope_cos=cs, rope_sin=sn,
                                     n_threads=threads)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": kv_bytes(ctx) / med / 1e9, "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{len(times)} layer-calls of the C3 shape at ctx {ctx} (median "
                      f"{med * 1e6:.0f} us/layer-call), oracle/attn_oracle.c, {threads} threads "
                      f"over query heads",
            "us_per_layer_call": med * 1e6}


def copy_calibration(mib: int) -> int:
    """A kernel of known traffic: mib MiB read and mib MiB written per launch."""
    from llmplayer_amd import _lib
    from llmplayer_amd.hip_forward_pass import DeviceBuffer
    n = mib * 2**20
    src, dst = DeviceBuffer(n), DeviceBuffer(n)
    for _ in range(5):
        _lib.call("llmp_copy_kernel", dst.ptr, src.ptr, n, 0)
    _lib.call("llmp_stream_sync", 0)
    src.free()
    dst.free()
    log(f"[bench] copy calibration: 5 launches x {mib} MiB read + {mib} MiB written")
    return 0


def profile_workload(ctx: int, steps: int, warmup: int, splits: int, rotate_bytes: int,
                     q8: bool = False) -> int:
    """Eager layer-calls only (the decode kernels as rocprofv3 sees them one by one)."""
    from llmplayer_amd import _lib
    from llmplayer_amd import hip_forward_pass as hfp
    per_layer = kv_bytes(ctx, q8)
    n_layers = max(1, math.ceil(rotate_bytes / per_layer))
    c = hfp.ModelConfig(HQ, HKV, D, n_layers, architecture=hfp.ARCH_LLAMA, rope_freq_base=THETA)
    fp = hfp.HipForwardPass(c, ctx, kv_dtype=_lib.LLMP_KV_Q8_0 if q8 else _lib.LLMP_KV_F32)
    try:
        rng = np.random.default_rng(2024)
        fill_caches(fp, c, ctx, n_layers, q8, rng)
        fp.uploadQKV(rng.standard_normal(c.q_dim, dtype=np.float32),
                     rng.standard_normal(c.kv_dim, dtype=np.float32) * np.float32(0.5),
                     rng.standard_normal(c.kv_dim, dtype=np.float32))
        plan = fp.decodePlan(0, ctx - 1, splits)
        for i in range(warmup + steps):
            fp.forwardAttentionPart(i % n_layers, ctx - 1, splits)
        fp.sync()
    finally:
        fp.close()
    log(f"[bench] profile workload: ctx {ctx}{' Q8_0' if q8 else ''}, {warmup}+{steps} eager "
        f"layer-calls over {n_layers} layer caches, plan {plan}")
    return 0


def profile_prefill(P: int, steps: int) -> int:
    """C5 prefill calls only (append + attention kernels as rocprofv3 sees them)."""
    r = prefill_run(P, steps)
    log(f"[bench] profile prefill: P={P}, {r}")
    return 0


def kernel_name(plan: dict) -> str:
    """The split kernel instantiation the library launches for the C3 shape (D=128, G=3)."""
    return f"decode_split_kernel<128, 3, 8, 2, {plan['waves']}, true>"


def traffic_from_profiles(ctx: int):
    """HBM bytes per launch of the split kernel from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration), if present."""
    tag = f"{ctx // 1024}k" if ctx % 1024 == 0 else str(ctx)
    path = os.path.join(ROOT, "profiles", f"decode_split_c3_ctx{tag}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")  # FETCH+WRITE, copy-calibrated


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--ctx2", type=int, default=4096, help="second context reported (0 = none)")
    ap.add_argument("--splits", type=int, default=0, help="split-K partitions (0 = library choice)")
    ap.add_argument("--rotate-gib", type=float, default=2.0)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-verify", dest="verify", action="store_false",
                    help="skip the speculative-verification (K draft tokens) measurement")
    ap.add_argument("--no-q8", dest="q8", action="store_false",
                    help="skip the Q8_0-cache decode measurement")
    ap.add_argument("--no-prefill", dest="prefill", action="store_false",
                    help="skip the C5 prefill measurement")
    ap.add_argument("--no-block", dest="block", action="store_false",
                    help="skip the attention-block (projections + attention) measurement")
    ap.add_argument("--block-q8", action="store_true",
                    help="--profile-block: the Q8_1 input mode")
    ap.add_argument("--profile-block", action="store_true",
                    help="for rocprofv3: the attention-block graph at --ctx2 only, then exit")
    ap.add_argument("--profile-workload", action="store_true",
                    help="for rocprofv3: only the warm-up and K eager layer-calls at --ctx "
                         "(no graph replay, no second context, no CPU baseline), then exit")
    ap.add_argument("--kv", choices=("f32", "q8"), default="f32",
                    help="KV cache of --profile-workload")
    ap.add_argument("--profile-verify", type=int, default=0, metavar="K",
                    help="for rocprofv3: speculative verification of K tokens at --ctx, then exit")
    ap.add_argument("--profile-prefill", type=int, default=0, metavar="P",
                    help="for rocprofv3: C5 prefill of P tokens (K graph + K eager calls), then exit")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="for rocprofv3 PMC calibration: 5 launches of the library's plain "
                         "copy kernel over MIB MiB, then exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build "
              "(decode attention runs on one MI355X; multi-GPU sharding is design-only)",
              file=sys.stderr)
        return 2
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        metric = json.load(f)["metric"]

    from llmplayer_amd import hip_forward_pass as hfp
    hfp.init(0)
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    if args.profile_workload:
        return profile_workload(args.ctx, args.steps, args.warmup, args.splits,
                                int(args.rotate_gib * 2**30), q8=args.kv == "q8")
    if args.profile_prefill:
        return profile_prefill(args.profile_prefill, args.steps)
    if args.profile_block:
        r = block_run(args.ctx2 or 4096, args.steps, q8_input=args.block_q8)
        log(f"[bench] profile block: {r}")
        return 0
    if args.profile_verify:
        r = verify_run(args.ctx, args.profile_verify, args.steps, int(args.rotate_gib * 2**30))
        log(f"[bench] profile verify: {r}")
        return 0
    info = hfp.device_info()
    log(f"[bench] device {info['arch']} with {info['n_cu']} CUs")
    rot = int(args.rotate_gib * 2**30)
    main_run = gpu_run(args.ctx, args.steps, args.warmup, args.splits, rot)
    log(f"[bench] ctx {args.ctx}: {main_run['us_per_layer_call']:.2f} us/layer-call, "
        f"{main_run['kv_read_gbps']:.0f} GB/s, split kernel {main_run['split_kernel_us']:.2f} us")
    second = None
    if args.ctx2:
        second = gpu_run(args.ctx2, args.steps, args.warmup, args.splits, rot)
        log(f"[bench] ctx {args.ctx2}: {second['us_per_layer_call']:.2f} us/layer-call, "
            f"{second['kv_read_gbps']:.0f} GB/s, split kernel {second['split_kernel_us']:.2f} us")

    q8_runs = []
    if args.q8:
        for ctx in [args.ctx] + ([args.ctx2] if args.ctx2 else []):
            r = gpu_run(ctx, args.steps, args.warmup, args.splits, rot, q8=True)
            log(f"[bench] ctx {ctx} Q8_0: {r['us_per_layer_call']:.2f} us/layer-call, "
                f"{r['kv_read_gbps']:.0f} GB/s, split kernel {r['split_kernel_us']:.2f} us")
            q8_runs.append(r)

    verify = []
    if args.verify:
        for K in (4, 8, 16):
            r = verify_run(args.ctx, K, 100, rot)
            r["decode_calls_us"] = round(K * main_run["us_per_layer_call"], 2)
            r["speedup_vs_k_decode_calls"] = round(r["decode_calls_us"] / r["us_per_call"], 2)
            log(f"[bench] verify K={K} at ctx {args.ctx}: {r['us_per_call']:.1f} us/call "
                f"({r['speedup_vs_k_decode_calls']:.2f}x vs {K} decode calls)")
            verify.append(r)

    prefill = []
    if args.prefill:
        for P in (512, 2048):
            r = prefill_run(P, 20)
            log(f"[bench] prefill C5 P={P}: {r['us_per_call']:.1f} us/call, attention kernel "
                f"{r['attn_kernel_us']:.1f} us ({r['attn_kernel_causal_tflops']:.1f} causal TFLOP/s)")
            prefill.append(r)

    block = block_q8 = None
    if args.block:
        block = block_run(args.ctx2 or 4096, 200)
        attn_us = second["us_per_layer_call"] if second is not None else None
        if attn_us is not None:
            block["attention_core_us"] = round(attn_us, 2)
            proj_us = block["us_per_layer_call"] - attn_us
            block["projections_us"] = round(proj_us, 2)
            if proj_us > 0:
                block["projection_weight_gbps"] = round(block["weight_bytes_per_layer"] / (proj_us * 1e-6) / 1e9, 1)
        log(f"[bench] attention block C3 Q4_K_M at ctx {block['ctx']}: {block['us_per_layer_call']:.1f} us/layer "
            f"({block['weight_bytes_per_layer'] / 1e6:.1f} MB of weights)")
        block_q8 = block_run(args.ctx2 or 4096, 200, q8_input=True)
        log(f"[bench] attention block C3 Q4_K_M at ctx {block_q8['ctx']}, Q8_1 input: "
            f"{block_q8['us_per_layer_call']:.1f} us/layer")

    # Prefill and verification over a Q8_0 cache (quantising append, dequantising staging).
    q8_prefill = q8_verify = None
    if args.q8 and args.prefill:
        q8_prefill = prefill_run(2048, 20, q8=True)
        log(f"[bench] prefill C5 P=2048 Q8_0: {q8_prefill['us_per_call']:.1f} us/call, attention "
            f"{q8_prefill['attn_kernel_us']:.1f} us, append {q8_prefill['append_kernel_us']:.1f} us")
    if args.q8 and args.verify:
        q8_verify = verify_run(args.ctx, 16, 100, rot, q8=True)
        q8_dec = [r for r in q8_runs if r["ctx"] == args.ctx]
        if q8_dec:
            q8_verify["decode_calls_us"] = round(16 * q8_dec[0]["us_per_layer_call"], 2)
            q8_verify["speedup_vs_k_decode_calls"] = round(
                q8_verify["decode_calls_us"] / q8_verify["us_per_call"], 2)
        log(f"[bench] verify K=16 at ctx {args.ctx} Q8_0: {q8_verify['us_per_call']:.1f} us/call")
    B = kv_bytes(args.ctx)
    achieved = B / (main_run["split_kernel_us"] * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / PEAK_GBPS, 4), "traffic": traffic_from_profiles(args.ctx),
                "kernel": kernel_name(main_run["plan"]),
                "algorithmic_bytes_per_launch": B,
                "kernel_mean_us": round(main_run["split_kernel_us"], 3)}
    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU restatement ...")
        cpu = cpu_baseline(args.ctx, args.cpu_seconds)
        log(f"[bench] CPU: {cpu['us_per_layer_call']:.0f} us/layer-call on {cpu['cores']} threads")
    line = {
        "metric": metric,
        "value": round(main_run["kv_read_gbps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_run["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) Q/K/V and KV cache (K x 0.5), seeded",
        "config": {"workload": f"C3 Llama-3.2-3B decode attention, ctx {args.ctx}",
                   "heads_q": HQ, "heads_kv": HKV, "head_dim": D, "ctx": args.ctx,
                   "splits": main_run["plan"]["splits"], "waves": main_run["plan"]["waves"],
                   "kv_layers_rotated": main_run["n_layers"]},
        "us_per_layer_call": round(main_run["us_per_layer_call"], 3),
        "kv_read_pct_of_hbm_peak": round(100 * main_run["kv_read_gbps"] / PEAK_GBPS, 2),
        "reduce_kernel_us": round(main_run["reduce_kernel_us"], 3),
        "us_per_layer_call_eager": round(main_run["us_per_layer_call_eager"], 3),
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if second is not None:
        line[f"ctx{args.ctx2}"] = {
            "us_per_layer_call": round(second["us_per_layer_call"], 3),
            "kv_read_gbps": round(second["kv_read_gbps"], 1),
            "kv_read_pct_of_hbm_peak": round(100 * second["kv_read_gbps"] / PEAK_GBPS, 2),
            "split_kernel_us": round(second["split_kernel_us"], 3),
            "reduce_kernel_us": round(second["reduce_kernel_us"], 3),
            "us_per_layer_call_eager": round(second["us_per_layer_call_eager"], 3),
            "kv_layers_rotated": second["n_layers"]}
    if q8_runs:
        f32_us = {args.ctx: main_run["us_per_layer_call"]}
        if second is not None:
            f32_us[args.ctx2] = second["us_per_layer_call"]
        line["q8_0_kv"] = []
        for r in q8_runs:
            bq = kv_bytes(r["ctx"], True)
            line["q8_0_kv"].append({
                "workload": f"C3 decode attention over a Q8_0 cache, ctx {r['ctx']}",
                "us_per_layer_call": round(r["us_per_layer_call"], 3),
                "kv_read_gbps": round(r["kv_read_gbps"], 1),
                "split_kernel_us": round(r["split_kernel_us"], 3),
                "split_kernel_gbps": round(bq / (r["split_kernel_us"] * 1e-6) / 1e9, 1),
                "split_kernel_pct_of_hbm_peak": round(
                    100.0 * bq / (r["split_kernel_us"] * 1e-6) / 1e9 / PEAK_GBPS, 2),
                "kernel": f"decode_q8_mfma_kernel<128, 3, {r['plan']['waves']}, true>",
                "reduce_kernel_us": round(r["reduce_kernel_us"], 3),
                "algorithmic_bytes_per_launch": bq,
                "splits": r["plan"]["splits"], "waves": r["plan"]["waves"],
                "speedup_vs_f32_cache": round(f32_us[r["ctx"]] / r["us_per_layer_call"], 3)})
    if prefill:
        line["prefill_c5_llama1b"] = prefill
    if verify:
        line["speculative_verify_c3"] = verify
    if block is not None:
        line["attn_block_c3_q4_k_m"] = block
    if block_q8 is not None:
        line["attn_block_c3_q4_k_m_q8_1_input"] = block_q8
    if q8_prefill is not None:
        line["q8_0_prefill_c5_llama1b"] = q8_prefill
    if q8_verify is not None:
        line["q8_0_speculative_verify_c3"] = q8_verify
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
