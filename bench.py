#!/usr/bin/env python3
"""Decode-attention benchmark on one MI355X (BASELINE.json metric).

A step is one decode attention layer-call (QK-norm/RoPE prep, KV append, split-K
QK^T/softmax/PV and the log-sum-exp combine) for one new token at position ctx-1.  The headline
is the Llama-3.2-3B head shape (C3: 24 query heads, 8 KV heads, head_dim 128, fp32 KV) at 32k
context; the same line carries every other decode config of BASELINE.json (C1, C2 at 1k/4k/16k
over its 28 layers, C4 local and global layers, the C3 split sweep), each with its µs per
layer-call, KV-read GB/s, % of HBM peak and a CPU baseline beside it.

Successive layer-calls rotate over enough layer caches (>= 2 GiB) that every call reads its KV
from HBM rather than the 256 MB Infinity Cache.  Inputs are synthetic N(0,1) (C3: K x 0.5),
resident in HBM before any timed region.

value = KV-read GB/s of the headline = (2 * ctx * Hkv * D * 4 bytes) / (time per layer-call)
over the K timed steps (one graph replay of K layer-calls, HIP events on the library stream).
Every row also reports the median over >= 7 replays of a graph of >= 100 layer-calls.
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
import re
import statistics
import sys
import time
from dataclasses import dataclass

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_GBPS = 8000.0            # MI355X HBM3E peak
MEDIAN_CALLS = 100            # layer-calls per replayed graph of a row (at least)
MEDIAN_REPLAYS = 7            # replays per row; the row reports their median


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


@dataclass(frozen=True)
class Shape:
    """One BASELINE.json decode config: head shape, RoPE, QK-norm, window, layer pattern."""
    key: str
    name: str
    hq: int
    hkv: int
    d: int
    arch: str
    theta: float
    qk_norm: bool = False
    window: int = 0
    k_scale: float = 1.0
    period: int = 1          # layers per repeating pattern (C2: its 28 layers; C4: 5 local + 1 global)


C1 = Shape("C1", "Llama-3.2-1B", 32, 8, 64, "llama", 500000.0)
C2 = Shape("C2", "Qwen3-0.6B", 16, 8, 128, "qwen3", 1e6, qk_norm=True, period=28)
C3 = Shape("C3", "Llama-3.2-3B", 24, 8, 128, "llama", 500000.0, k_scale=0.5)
C4 = Shape("C4", "Gemma-3-1B", 4, 1, 256, "gemma3", 1e6, qk_norm=True, window=512, period=6)
HQ, HKV, D = C3.hq, C3.hkv, C3.d


def is_local(shape: Shape, layer: int) -> bool:
    """Gemma 3: every 6th layer is global (Attention.isGlobalLayer, Attention.java:256-258)."""
    return shape.window > 0 and layer % 6 != 5


def attended(shape: Shape, layer: int, pos: int) -> int:
    return min(shape.window, pos + 1) if is_local(shape, layer) else pos + 1


def kv_bytes_rows(shape: Shape, n: int, q8: bool = False) -> int:
    """K and V bytes of n attended rows: fp32, or Q8_0 quants plus a 4-byte scale per 32
    values (1.125 bytes per value)."""
    per = shape.d + shape.d // 32 * 4 if q8 else shape.d * 4
    return 2 * n * shape.hkv * per


def kv_bytes(ctx: int, q8: bool = False) -> int:
    return kv_bytes_rows(C3, ctx, q8)


def host_facts() -> dict:
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    model = "?"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or avail
    return {"nproc": os.cpu_count(), "affinity_cpus": avail, "cpu_share": min(share, avail),
            "cpu_model": model}


class DecodeRig:
    """A HipForwardPass over n_layers layer caches of one shape, filled once: layer 0 from
    host N(0,1) rows (K x k_scale, or synthetic Q8_0 rows), the others by device copies."""

    def __init__(self, shape: Shape, ctx: int, rotate_bytes: int, q8: bool = False, seed: int = 2024):
        from llmplayer_amd import _lib
        from llmplayer_amd import hip_forward_pass as hfp
        self.shape, self.ctx, self.q8 = shape, ctx, q8
        per_layer = kv_bytes_rows(shape, ctx, q8)
        if shape.window > 0:
            # Window pattern: the global layers alone rotate over >= rotate_bytes (one in
            # `period` layers is global); local layers read only their window of each cache.
            n = shape.period * max(1, math.ceil(rotate_bytes / per_layer))
        else:
            n = max(shape.period, math.ceil(rotate_bytes / per_layer))
            n = ((n + shape.period - 1) // shape.period) * shape.period
        self.n_layers = n
        c = hfp.ModelConfig(shape.hq, shape.hkv, shape.d, n, architecture=shape.arch,
                            rope_freq_base=shape.theta, norm_eps=1e-6,
                            sliding_window=shape.window)
        self.c = c
        rng = np.random.default_rng(seed)
        qk = None
        if shape.qk_norm:   # per-layer weights ~U(0.5, 1.5), repeating with the layer pattern
            ws = [(rng.uniform(0.5, 1.5, shape.d).astype(np.float32),
                   rng.uniform(0.5, 1.5, shape.d).astype(np.float32)) for _ in range(shape.period)]
            qk = [ws[i % shape.period] for i in range(n)]
        self.fp = hfp.HipForwardPass(c, ctx, qk_norm=qk,
                                     kv_dtype=_lib.LLMP_KV_Q8_0 if q8 else _lib.LLMP_KV_F32)
        try:
            self._fill(rng)
            self.fp.uploadQKV(rng.standard_normal(c.q_dim, dtype=np.float32),
                              rng.standard_normal(c.kv_dim, dtype=np.float32) * np.float32(shape.k_scale),
                              rng.standard_normal(c.kv_dim, dtype=np.float32))
        except Exception:
            self.fp.close()
            raise
        log(f"[bench] {shape.key} ctx {ctx}{' Q8_0' if q8 else ''}: {n} layer caches x "
            f"{per_layer / 2**20:.1f} MiB")

    def _fill(self, rng) -> None:
        from llmplayer_amd import _lib
        c, rows = self.c, self.ctx - 1
        if rows <= 0:
            return
        if self.q8:
            kq = rng.integers(-127, 128, (rows, c.kv_dim), dtype=np.int8)
            vq = rng.integers(-127, 128, (rows, c.kv_dim), dtype=np.int8)
            ks = np.full((rows, c.kv_dim // 32), 1.2 / 127, np.float32)
            vs = np.full((rows, c.kv_dim // 32), 2.4 / 127, np.float32)
            self.fp.kv.write_q8(0, 0, kq, ks, vq, vs)
        else:
            kc = rng.standard_normal((rows, c.kv_dim), dtype=np.float32) * np.float32(self.shape.k_scale)
            vc = rng.standard_normal((rows, c.kv_dim), dtype=np.float32)
            self.fp.kv.write(0, 0, kc, vc)
        if self.n_layers > 1:
            k0, _ = self.fp.kv.layer_ptrs(0)
            k1, _ = self.fp.kv.layer_ptrs(1)
            span = k1 - k0          # one layer's K and V planes (and Q8_0 scales) are contiguous
            for layer in range(1, self.n_layers):
                kl, _ = self.fp.kv.layer_ptrs(layer)
                _lib.call("llmp_memcpy_dtod", kl, k0, span, 0)
            self.fp.sync()

    def layers(self, local=None):
        """Every layer, or only the local (True) / global (False) ones."""
        if local is None:
            return list(range(self.n_layers))
        return [l for l in range(self.n_layers) if is_local(self.shape, l) == local]

    def plan(self, layer: int, pos: int, splits: int) -> dict:
        return self.fp.decodePlan(layer, pos, splits)

    def call(self, layer: int, pos: int, splits: int) -> None:
        self.fp.forwardAttentionPart(layer, pos, splits)

    def graph_ms(self, layers, pos: int, splits: int, n_calls: int, replays: int):
        """Captures n_calls layer-calls (cycling over `layers`) once and returns the elapsed ms
        of each of `replays` replays (HIP events on the library stream)."""
        from llmplayer_amd import _lib
        g = C.c_uint64()
        _lib.call("llmp_graph_begin", 0)
        for i in range(n_calls):
            self.call(layers[i % len(layers)], pos, splits)
        _lib.call("llmp_graph_end", 0, C.byref(g))
        e0, e1 = C.c_uint64(), C.c_uint64()
        _lib.call("llmp_event_create", C.byref(e0))
        _lib.call("llmp_event_create", C.byref(e1))
        out = []
        try:
            _lib.call("llmp_graph_launch", g.value, 0)   # warm replay
            self.fp.sync()
            for _ in range(replays):
                _lib.call("llmp_event_record", e0.value, 0)
                _lib.call("llmp_graph_launch", g.value, 0)
                _lib.call("llmp_event_record", e1.value, 0)
                _lib.call("llmp_event_sync", e1.value)
                ms = C.c_float()
                _lib.call("llmp_event_elapsed_ms", C.byref(ms), e0.value, e1.value)
                out.append(ms.value)
        finally:
            _lib.call("llmp_graph_destroy", g.value)
            _lib.call("llmp_event_destroy", e0.value)
            _lib.call("llmp_event_destroy", e1.value)
        return out

    def kernel_means(self, layers, pos: int, splits: int, n_calls: int) -> dict:
        """Eager calls with a HIP event pair around every kernel launch (library stream): the
        mean split-K and combine kernel durations in µs, and the eager µs per layer-call."""
        from llmplayer_amd import _lib
        h = self.fp.kv.handle
        _lib.call("llmp_profile_reset", h)
        _lib.call("llmp_profile_enable", h, 1)
        t0 = time.perf_counter()
        for i in range(n_calls):
            self.call(layers[i % len(layers)], pos, splits)
        self.fp.sync()
        wall = time.perf_counter() - t0
        _lib.call("llmp_profile_enable", h, 0)
        res = {}
        for kind, name in ((_lib.LLMP_PROF_DECODE_SPLIT, "split"),
                           (_lib.LLMP_PROF_DECODE_REDUCE, "reduce")):
            cnt, tot = C.c_int(), C.c_double()
            _lib.call("llmp_profile_read", h, kind, C.byref(cnt), C.byref(tot))
            res[name + "_kernel_us"] = tot.value / cnt.value * 1e3 if cnt.value else 0.0
            res[name + "_launches"] = cnt.value
        res["eager_host_us_per_call"] = wall / n_calls * 1e6
        return res

    def close(self) -> None:
        self.fp.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def decode_row(rig: DecodeRig, pos: int, splits: int = 0, local=None, kernels: bool = True) -> dict:
    """One measured row: median µs per layer-call over MEDIAN_REPLAYS replays of a graph of
    >= MEDIAN_CALLS calls over the rig's layers, KV-read GB/s and % of peak, the split-K kernel's
    mean duration and its own fraction of peak, and the launch plan."""
    layers = rig.layers(local)
    n_calls = max(MEDIAN_CALLS, len(layers))
    for i in range(min(len(layers), 64)):
        rig.call(layers[i], pos, splits)
    rig.fp.sync()
    reps = rig.graph_ms(layers, pos, splits, n_calls, MEDIAN_REPLAYS)
    per_call = [r / n_calls * 1e3 for r in reps]
    med = statistics.median(per_call)
    n = attended(rig.shape, layers[0], pos)
    B = kv_bytes_rows(rig.shape, n, rig.q8)
    row = {"attended_rows": n, "kv_bytes_per_call": B,
           "us_per_layer_call": round(med, 3), "us_per_layer_call_min": round(min(per_call), 3),
           "layer_calls_timed": n_calls * MEDIAN_REPLAYS,
           "kv_read_gbps": round(B / (med * 1e-6) / 1e9, 1),
           "kv_read_pct_of_hbm_peak": round(100 * B / (med * 1e-6) / 1e9 / PEAK_GBPS, 2),
           "plan": rig.plan(layers[0], pos, splits), "layer_caches": len(layers)}
    if kernels:
        km = rig.kernel_means(layers, pos, splits, min(n_calls, 400))
        row["split_kernel_us"] = round(km["split_kernel_us"], 3)
        row["reduce_kernel_us"] = round(km["reduce_kernel_us"], 3)
        if km["split_kernel_us"] > 0:
            kg = B / (km["split_kernel_us"] * 1e-6) / 1e9
            row["split_kernel_gbps"] = round(kg, 1)
            row["split_kernel_frac_of_peak"] = round(kg / PEAK_GBPS, 4)
    return row


def headline_run(ctx: int, steps: int, warmup: int, splits: int, rotate_bytes: int) -> dict:
    """C3 at ctx: warm-up, then exactly `steps` layer-calls in one timed graph replay (the
    line's value and ms_per_step), then the median row and kernel means."""
    with DecodeRig(C3, ctx, rotate_bytes) as rig:
        pos = ctx - 1
        layers = rig.layers()
        for i in range(warmup):
            rig.call(layers[i % len(layers)], pos, splits)
        rig.fp.sync()
        ms = rig.graph_ms(layers, pos, splits, steps, 1)[0]
        row = decode_row(rig, pos, splits)
    row["ms_per_step"] = ms / steps
    row["us_per_layer_call_k_steps"] = round(ms / steps * 1e3, 3)
    row["kv_read_gbps_k_steps"] = round(kv_bytes(ctx) / (ms / steps * 1e-3) / 1e9, 1)
    row["n_layers"] = len(layers)
    return row


def config_rows(rotate_bytes: int) -> dict:
    """C1, C2 (all 28 layers at 1k/4k/16k), C4 (local and global layers at 8192)."""
    out = {}
    with DecodeRig(C1, 512, rotate_bytes) as rig:
        out["C1_llama3.2_1b_pos511"] = decode_row(rig, 511)
    log(f"[bench] C1: {out['C1_llama3.2_1b_pos511']['us_per_layer_call']} us/layer-call")
    for ctx in (1024, 4096, 16384):
        with DecodeRig(C2, ctx, rotate_bytes) as rig:
            r = decode_row(rig, ctx - 1)
        r["model_layers_timed"] = C2.period
        out[f"C2_qwen3_0.6b_ctx{ctx}"] = r
        log(f"[bench] C2 ctx {ctx}: {r['us_per_layer_call']} us/layer-call, "
            f"{r['kv_read_pct_of_hbm_peak']} % of peak")
    with DecodeRig(C4, 8192, rotate_bytes) as rig:
        for local, tag in ((True, "local_w512"), (False, "global")):
            r = decode_row(rig, 8191, local=local)
            out[f"C4_gemma3_1b_ctx8192_{tag}"] = r
            log(f"[bench] C4 {tag}: {r['us_per_layer_call']} us/layer-call")
    return out


def split_sweep(rotate_bytes: int) -> dict:
    """C3 at 4k and 32k with fixed split counts 8..128 and the library's own choice."""
    out = {}
    for ctx in (4096, 32768):
        rows = []
        with DecodeRig(C3, ctx, rotate_bytes) as rig:
            for s in (8, 16, 32, 64, 128, 0):
                r = decode_row(rig, ctx - 1, s, kernels=False)
                rows.append({"splits_requested": s or "auto", "splits": r["plan"]["splits"],
                             "waves": r["plan"]["waves"],
                             "us_per_layer_call": r["us_per_layer_call"],
                             "kv_read_pct_of_hbm_peak": r["kv_read_pct_of_hbm_peak"]})
        out[f"ctx{ctx}"] = rows
        log(f"[bench] C3 split sweep ctx {ctx}: " +
            ", ".join(f"{r['splits_requested']}:{r['us_per_layer_call']}" for r in rows))
    return out


# ------------------------------------------------------------------------ multi-token paths
def _timed_graph(fn, steps: int) -> float:
    """fn() enqueues one call; returns ms of one replay of a graph of `steps` calls."""
    from llmplayer_amd import _lib
    for _ in range(3):
        fn()
    _lib.call("llmp_stream_sync", 0)
    g = C.c_uint64()
    _lib.call("llmp_graph_begin", 0)
    for _ in range(steps):
        fn()
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
    return ms.value


def prefill_run(P: int, steps: int, q8: bool = False, f32: bool = False) -> dict:
    """C5: prefill attention of P prompt tokens (Llama-3.2-1B shape 32/8/64, N(0,1), causal)
    in one call (exact K/V append + MFMA attention), over an fp32 or a Q8_0 cache; inputs bf16
    (llmp_attn_prefill, the C5 config) or fp32 (llmp_attn_prefill_f32, the reference's own
    prompt contract).  Timed as a graph replay of `steps` calls; per-kernel means from an eager
    profiled pass."""
    from llmplayer_amd import _lib
    from llmplayer_amd import hip_forward_pass as hfp
    c = hfp.ModelConfig(32, 8, 64, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    fp = hfp.HipForwardPass(c, P, kv_dtype=_lib.LLMP_KV_Q8_0 if q8 else _lib.LLMP_KV_F32)
    bufs = []
    try:
        rng = np.random.default_rng(5)
        arrs = [rng.standard_normal((P, n), dtype=np.float32) for n in (c.q_dim, c.kv_dim, c.kv_dim)]
        if not f32:
            arrs = [hfp.to_bf16(a) for a in arrs]
        for a in arrs:
            b = hfp.DeviceBuffer(a.nbytes)
            b.upload(a)
            bufs.append(b)
        out = hfp.DeviceBuffer(P * c.q_dim * 4)
        bufs.append(out)
        h = fp.kv.handle
        if f32:
            fn = lambda: _lib.call("llmp_attn_prefill_f32", h, 0, 0, P, bufs[0].ptr, bufs[1].ptr,
                                   bufs[2].ptr, 0, out.ptr, 0)
        else:
            fn = lambda: _lib.call("llmp_attn_prefill", h, 0, 0, P, bufs[0].ptr, bufs[1].ptr,
                                   bufs[2].ptr, out.ptr, 0)
        ms = _timed_graph(fn, steps)
        _lib.call("llmp_profile_reset", h)
        _lib.call("llmp_profile_enable", h, 1)
        for _ in range(steps):
            fn()
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
    us = ms / steps * 1e3
    flops = 4.0 * c.head_count * c.head_size * P * (P + 1) / 2   # causal QK^T + PV
    return {"P": P, "inputs": "fp32" if f32 else "bf16", "us_per_call": round(us, 2),
            "attn_kernel_us": round(res["attn"], 2), "append_kernel_us": round(res["append"], 2),
            "causal_tflops": round(flops / (us * 1e-6) / 1e12, 2),
            "attn_kernel_causal_tflops": round(flops / (res["attn"] * 1e-6) / 1e12, 2),
            # fp16 MFMA work issued: 3 products for QK^T (hi/lo splits), 2 for PV when the V rows
            # are fp16-exact (bf16 rows in an fp32 cache: the V-lo product is skipped), else 3
            "mfma_tflops_issued_f16": round((3.0 if (f32 or q8) else 2.5) * flops / (res["attn"] * 1e-6) / 1e12, 2)}


def verify_run(ctx: int, K: int, steps: int, rotate_bytes: int, q8: bool = False,
               f32: bool = True) -> dict:
    """Speculative verification at the C3 shape: K draft tokens at positions ctx-K..ctx-1 in
    one multi-token call over a (ctx-K)-row fp32 or Q8_0 cache (the reference runs K
    sequential fp32 forwards, LLMEngine.java:1019-1033); fp32 inputs by default.  Layer caches
    rotate over >= 2 GiB; graph replay."""
    from llmplayer_amd import _lib
    from llmplayer_amd import hip_forward_pass as hfp
    n_layers = max(1, math.ceil(rotate_bytes / kv_bytes(ctx, q8)))
    c = hfp.ModelConfig(HQ, HKV, D, n_layers, architecture=hfp.ARCH_LLAMA, rope_freq_base=C3.theta)
    fp = hfp.HipForwardPass(c, ctx, kv_dtype=_lib.LLMP_KV_Q8_0 if q8 else _lib.LLMP_KV_F32)
    bufs = []
    try:
        rng = np.random.default_rng(7)
        rows = ctx - K
        if q8:
            fp.kv.write_q8(0, 0, rng.integers(-127, 128, (rows, c.kv_dim), dtype=np.int8),
                           np.full((rows, c.kv_dim // 32), 1.2 / 127, np.float32),
                           rng.integers(-127, 128, (rows, c.kv_dim), dtype=np.int8),
                           np.full((rows, c.kv_dim // 32), 2.4 / 127, np.float32))
        else:
            fp.kv.write(0, 0, rng.standard_normal((rows, c.kv_dim), dtype=np.float32) * np.float32(0.5),
                        rng.standard_normal((rows, c.kv_dim), dtype=np.float32))
        k0, _ = fp.kv.layer_ptrs(0)
        if n_layers > 1:
            span = fp.kv.layer_ptrs(1)[0] - k0
            for layer in range(1, n_layers):
                _lib.call("llmp_memcpy_dtod", fp.kv.layer_ptrs(layer)[0], k0, span, 0)
        arrs = [rng.standard_normal((K, n), dtype=np.float32) for n in (c.q_dim, c.kv_dim, c.kv_dim)]
        if not f32:
            arrs = [hfp.to_bf16(a) for a in arrs]
        for arr in arrs:
            b = hfp.DeviceBuffer(arr.nbytes)
            b.upload(arr)
            bufs.append(b)
        out = hfp.DeviceBuffer(K * c.q_dim * 4)
        bufs.append(out)
        pos0 = ctx - K
        state = {"i": 0}
        entry = "llmp_attn_prefill_f32" if f32 else "llmp_attn_prefill_ex"

        def fn():
            layer = state["i"] % n_layers
            state["i"] += 1
            _lib.call(entry, fp.kv.handle, layer, pos0, K, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr,
                      0, out.ptr, 0)
        for _ in range(n_layers):
            fn()
        ms = _timed_graph(fn, steps)
    finally:
        for b in bufs:
            b.free()
        fp.close()
    us = ms / steps * 1e3
    return {"K": K, "ctx": ctx, "inputs": "fp32" if f32 else "bf16", "us_per_call": round(us, 2),
            "kv_read_gbps": round(kv_bytes(ctx - K, q8) / (us * 1e-6) / 1e9, 1)}


# Per GGUF block type: (weights per block, bytes per block, byte offsets of its fp16 scale
# fields) (GGMLType.java:4-35 and each tensor class's layout).
GGUF_BLOCKS = {8: (32, 34, (0,)), 2: (32, 18, (0,)), 6: (32, 22, (0,)), 7: (32, 24, (0, 2)),
               20: (32, 18, (0,)), 39: (32, 17, ()), 10: (256, 84, (80, 82)), 11: (256, 110, (108,)),
               12: (256, 144, (0, 2)), 13: (256, 176, (0, 2)), 14: (256, 210, (208,)),
               23: (256, 136, (0,)), 18: (256, 98, (0,)), 21: (256, 110, (0,)), 22: (256, 82, (0,))}
GGUF_NAMES = {0: "F32", 1: "F16", 30: "BF16", 8: "Q8_0", 2: "Q4_0", 6: "Q5_0", 7: "Q5_1",
              20: "IQ4_NL", 39: "MXFP4", 10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K",
              14: "Q6_K", 23: "IQ4_XS", 18: "IQ3_XXS", 21: "IQ3_S", 22: "IQ2_S"}


def synthetic_gguf(t: int, rows: int, cols: int, rng) -> np.ndarray:
    """Random GGUF-layout bytes of type t: uniform quant and sub-block scale bytes, fp16 block
    scales 2^-10 (the second field, a min, 2^-12), MXFP4 exponents 2^-7; dense types normal
    values times 0.02."""
    if t in (0, 1, 30):
        w = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
        if t == 0:
            return w.view(np.uint8).reshape(-1)
        if t == 1:
            return w.astype(np.float16).view(np.uint8).reshape(-1)
        return (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1)
    bw, bb, scales = GGUF_BLOCKS[t]
    b = rng.integers(0, 256, (rows, cols // bw, bb), dtype=np.uint8)
    f16 = lambda v: np.frombuffer(np.float16(v).tobytes(), np.uint8)
    for i, o in enumerate(scales):
        b[:, :, o:o + 2] = f16(2.0 ** (-10 - 2 * i))
    if t == 39:
        b[:, :, 0] = 120
    return b.reshape(-1)


# GGUF weight mixes of the attention projections (q, k, v, o), as llama.cpp's quantiser assigns
# them: Q4_K_M keeps Q6_K for v; Q3_K_L takes Q5_K for v and o.
MIXES = {"q4_k_m": ((12, 12, 14, 12), "Q4_K_M mix (Q4_K q/k/o, Q6_K v)"),
         "q3_k_l": ((11, 11, 13, 13), "Q3_K_L mix (Q3_K q/k, Q5_K v/o)")}


def block_run(ctx: int, steps: int, n_layers: int = 28, q8_input: bool = False,
              mix: str = "q4_k_m") -> dict:
    """The attention half of a C3 (Llama-3.2-3B, dim 3072) layer with a GGUF weight mix (MIXES;
    default Q4_K_M: Q4_K for q, k, o and Q6_K for v): pre-norm, projections, attention at ctx,
    output projection and residual, as a graph replay over n_layers layers with their own
    weights and caches.  q8_input: the projections the reference GPU runs on int8 (Q4_K, Q3_K,
    Q5_K here; Q6_K stays fp32) on the Q8_1-quantised input instead of the fp32 input."""
    from llmplayer_amd import _lib
    from llmplayer_amd import hip_forward_pass as hfp
    dim = 3072
    types, label = MIXES[mix] if isinstance(mix, str) else (mix, "all " + GGUF_NAMES[mix[0]])
    c = hfp.ModelConfig(HQ, HKV, D, n_layers, architecture=hfp.ARCH_LLAMA, rope_freq_base=C3.theta)
    fp = hfp.HipForwardPass(c, ctx)
    try:
        rng = np.random.default_rng(11)
        kc = rng.standard_normal((ctx - 1, c.kv_dim), dtype=np.float32) * np.float32(0.5)
        vc = rng.standard_normal((ctx - 1, c.kv_dim), dtype=np.float32)
        for layer in range(n_layers):
            fp.kv.write(layer, 0, kc, vc)
        fp.setBlockConfig(dim, 0.0, _lib.LLMP_INPUT_Q8_1 if q8_input else _lib.LLMP_INPUT_F32)
        wbytes = 0
        tq, tk, tv, to = types
        for layer in range(n_layers):
            lw = hfp.TransformerLayerWeights(attnNorm=np.ones(dim, np.float32))
            for name, t, rows, cols in (("wq", tq, c.q_dim, dim), ("wk", tk, c.kv_dim, dim),
                                        ("wv", tv, c.kv_dim, dim), ("wo", to, dim, c.q_dim)):
                data = synthetic_gguf(t, rows, cols, rng)
                setattr(lw, name, hfp.GgufTensor(t, rows, cols, data))
                if layer == 0:
                    wbytes += data.nbytes
            fp.uploadLayerWeights(layer, lw)
        fp.uploadX(rng.standard_normal(dim).astype(np.float32))
        state = {"i": 0}

        def fn():
            layer = state["i"] % n_layers
            state["i"] += 1
            _lib.call("llmp_attn_block", fp.kv.handle, layer, ctx - 1, 0, fp.gpuX.ptr, 0, 0)
        for _ in range(n_layers):
            fn()
        ms = _timed_graph(fn, steps)
    finally:
        fp.close()
    us = ms / steps * 1e3
    return {"ctx": ctx, "weights": label, "dim": dim,
            "input": ("Q8_1 (int8 dot products for "
                      + ("Q4_K" if mix == "q4_k_m" else "Q3_K and Q5_K" if mix == "q3_k_l" else "Q5_K")
                      + ")") if q8_input else "fp32",
            "us_per_layer_call": round(us, 2), "weight_bytes_per_layer": wbytes,
            "kv_bytes_per_layer": kv_bytes(ctx), "layers_rotated": n_layers}


def block_batch_run(ctx: int, K: int, steps: int, n_layers: int = 28, mix="q4_k_m",
                    q8_input: bool = False) -> dict:
    """The attention half of a C3 layer (as block_run; default the Q4_K_M mix, or a MIXES key,
    or four GGML types) for K draft tokens at positions ctx-K .. ctx-1 in one
    llmp_attn_block_batch call (projection weights read once for the K tokens), against K
    single-token llmp_attn_block calls over the same layers; graph replays over n_layers
    layers with their own weights and caches.  q8_input: the Q8_1 input mode (the reference
    GPU's int8 matvecs for the routed types, in both the batched and the single-token calls)."""
    from llmplayer_amd import _lib
    from llmplayer_amd import hip_forward_pass as hfp
    dim = 3072
    types, label = MIXES[mix] if isinstance(mix, str) else (mix, "all " + GGUF_NAMES[mix[0]])
    c = hfp.ModelConfig(HQ, HKV, D, n_layers, architecture=hfp.ARCH_LLAMA, rope_freq_base=C3.theta)
    fp = hfp.HipForwardPass(c, ctx)
    try:
        rng = np.random.default_rng(13)
        kc = rng.standard_normal((ctx - K, c.kv_dim), dtype=np.float32) * np.float32(0.5)
        vc = rng.standard_normal((ctx - K, c.kv_dim), dtype=np.float32)
        for layer in range(n_layers):
            fp.kv.write(layer, 0, kc, vc)
        fp.setBlockConfig(dim, 0.0, _lib.LLMP_INPUT_Q8_1 if q8_input else _lib.LLMP_INPUT_F32)
        wbytes = 0
        for layer in range(n_layers):
            lw = hfp.TransformerLayerWeights(attnNorm=np.ones(dim, np.float32))
            for name, t, rows, cols in (("wq", types[0], c.q_dim, dim), ("wk", types[1], c.kv_dim, dim),
                                        ("wv", types[2], c.kv_dim, dim), ("wo", types[3], dim, c.q_dim)):
                data = synthetic_gguf(t, rows, cols, rng)
                setattr(lw, name, hfp.GgufTensor(t, rows, cols, data))
                if layer == 0:
                    wbytes += data.nbytes
            fp.uploadLayerWeights(layer, lw)
        x = (rng.standard_normal((K, dim)) * 0.1).astype(np.float32)
        fp.uploadXBatch(x)
        fp.uploadX(x[0])
        state = {"i": 0}

        def batch():
            layer = state["i"] % n_layers
            state["i"] += 1
            _lib.call("llmp_attn_block_batch", fp.kv.handle, layer, ctx - K, K, fp.gpuXBatch.ptr, 0)

        def singles():
            layer = state["i"] % n_layers
            state["i"] += 1
            for t in range(K):
                _lib.call("llmp_attn_block", fp.kv.handle, layer, ctx - K + t, 0, fp.gpuX.ptr, 0, 0)
        for _ in range(n_layers):
            batch()
        ms_b = _timed_graph(batch, steps)
        ms_s = _timed_graph(singles, max(1, steps // 4))
    finally:
        fp.close()
    us_b = ms_b / steps * 1e3
    us_s = ms_s / max(1, steps // 4) * 1e3
    return {"K": K, "ctx": ctx, "weights": label, "dim": dim, "input": "Q8_1" if q8_input else "fp32",
            "us_per_call": round(us_b, 2), "us_per_token": round(us_b / K, 2),
            "single_token_blocks_us": round(us_s, 2), "speedup_vs_single_token_blocks": round(us_s / us_b, 2),
            "weight_bytes_per_layer": wbytes, "kv_bytes_per_layer": kv_bytes(ctx - K),
            "layers_rotated": n_layers}


# ------------------------------------------------------------------------------ CPU baseline
def cpu_time(shape: Shape, ctx: int, seconds: float, threads: int, layer: int = 0) -> dict:
    """The oracle (CPU restatement of Attention.forwardFromProjections) on one layer-call of
    `shape` at position ctx-1, parallel over query heads; median over a bounded sample."""
    from oracle import oracle as orc
    arch = {"gemma3": orc.ARCH_GEMMA3}.get(shape.arch, orc.ARCH_OTHER)
    rope_type = 2 if shape.arch == "qwen3" else 0
    oc = orc.OracleConfig(shape.hq, shape.hkv, shape.d, ctx, rope_type=rope_type, norm_eps=1e-6,
                          sliding_window=shape.window, arch=arch)
    rng = np.random.default_rng(2024)
    kvd = shape.hkv * shape.d
    kc = np.zeros((ctx, kvd), np.float32)
    vc = np.zeros((ctx, kvd), np.float32)
    kc[:ctx - 1] = rng.standard_normal((ctx - 1, kvd), dtype=np.float32) * np.float32(shape.k_scale)
    vc[:ctx - 1] = rng.standard_normal((ctx - 1, kvd), dtype=np.float32)
    q = rng.standard_normal(shape.hq * shape.d, dtype=np.float32)
    k = rng.standard_normal(kvd, dtype=np.float32) * np.float32(shape.k_scale)
    v = rng.standard_normal(kvd, dtype=np.float32)
    theta = 10000.0 if is_local(shape, layer) else shape.theta
    cs, sn = orc.rope_tables(shape.d, ctx, theta)
    qw = kw = None
    if shape.qk_norm:
        qw = rng.uniform(0.5, 1.5, shape.d).astype(np.float32)
        kw = rng.uniform(0.5, 1.5, shape.d).astype(np.float32)
    run = lambda: orc.forward_from_projections(oc, kc, vc, q, k, v, layer, ctx - 1, qnorm_w=qw,
                                               knorm_w=kw, rope_cos=cs, rope_sin=sn,
                                               n_threads=threads)
    for _ in range(2):
        run()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    B = kv_bytes_rows(shape, attended(shape, layer, ctx - 1))
    return {"us_per_layer_call": round(med * 1e6, 1), "kv_read_gbps": round(B / med / 1e9, 2),
            "threads": threads, "calls": len(times)}


def cpu_threads(shape: Shape, facts: dict) -> int:
    """min(CPUs this process may use, the box's CPU share, Hq): the reference parallelises over
    query heads (Attention.java:343), so more threads than heads do not help."""
    return max(1, min(facts["affinity_cpus"], facts["cpu_share"], shape.hq))


def cpu_baselines(seconds: float, facts: dict) -> dict:
    out = {}
    for key, shape, ctx, layer, secs in (("C3_ctx32768", C3, 32768, 0, seconds),
                                         ("C3_ctx4096", C3, 4096, 0, seconds / 4),
                                         ("C1_pos511", C1, 512, 0, seconds / 8),
                                         ("C2_ctx4096", C2, 4096, 0, seconds / 4),
                                         ("C4_ctx8192_local", C4, 8192, 0, seconds / 8),
                                         ("C4_ctx8192_global", C4, 8192, 5, seconds / 8)):
        out[key] = cpu_time(shape, ctx, secs, cpu_threads(shape, facts), layer)
        log(f"[bench] CPU {key}: {out[key]['us_per_layer_call']} us/layer-call on "
            f"{out[key]['threads']} threads")
    return out


# ---------------------------------------------------------------------------- profiling modes
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
    """Eager C3 layer-calls only (the decode kernels as rocprofv3 sees them one by one)."""
    with DecodeRig(C3, ctx, rotate_bytes, q8=q8) as rig:
        plan = rig.plan(0, ctx - 1, splits)
        for i in range(warmup + steps):
            rig.call(i % rig.n_layers, ctx - 1, splits)
        rig.fp.sync()
        n = rig.n_layers
    log(f"[bench] profile workload: ctx {ctx}{' Q8_0' if q8 else ''}, {warmup}+{steps} eager "
        f"layer-calls over {n} layer caches, plan {plan}")
    return 0


SHAPES = {"C1": (C1, 512), "C2": (C2, 4096), "C3": (C3, 4096), "C4": (C4, 8192)}


def profile_config(key: str, ctx: int, steps: int, rotate_bytes: int, graph: bool,
                   local=None) -> int:
    """For rocprofv3: `steps` layer-calls of one decode config at position ctx-1, eager or as
    one graph replay (the timed form of the bench rows)."""
    shape, default_ctx = SHAPES[key]
    ctx = ctx or default_ctx
    with DecodeRig(shape, ctx, rotate_bytes) as rig:
        layers = rig.layers(local)
        for i in range(min(len(layers), 64)):
            rig.call(layers[i], ctx - 1, 0)
        rig.fp.sync()
        if graph:
            ms = rig.graph_ms(layers, ctx - 1, 0, steps, 1)[0]
            log(f"[bench] profile {key} ctx {ctx}: graph of {steps} calls, {ms / steps * 1e3:.2f} us/call")
        else:
            for i in range(steps):
                rig.call(layers[i % len(layers)], ctx - 1, 0)
            rig.fp.sync()
            log(f"[bench] profile {key} ctx {ctx}: {steps} eager calls")
        log(f"[bench] plan {rig.plan(layers[0], ctx - 1, 0)}")
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


def rocprof_mean_us(ctx: int):
    """The split kernel's average duration (µs) in the committed rocprofv3 kernel-stats
    summary of the same workload (profiles/decode_split_c3_ctx<k>_kernel_stats.md: a markdown
    copy of trace_kernel_stats.csv), if present."""
    tag = f"{ctx // 1024}k" if ctx % 1024 == 0 else str(ctx)
    path = os.path.join(ROOT, "profiles", f"decode_split_c3_ctx{tag}_kernel_stats.md")
    if not os.path.exists(path):
        return None
    col = None
    with open(path) as f:
        for line in f:
            cells = [x.strip() for x in line.strip().strip("|").split("|")]
            if "AverageNs" in cells:
                col = cells.index("AverageNs")
            elif col is not None and cells and "decode_split_kernel" in cells[0]:
                try:
                    return round(float(cells[col]) / 1e3, 3)
                except (ValueError, IndexError):
                    return None
    return None


def roofline_of(row: dict, ctx: int, kernel: str) -> dict:
    B = kv_bytes(ctx)
    k_us = row["split_kernel_us"]
    achieved = B / (k_us * 1e-6) / 1e9
    r = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS, "unit": "GB/s",
         "frac": round(achieved / PEAK_GBPS, 4), "traffic": traffic_from_profiles(ctx),
         "kernel": kernel, "algorithmic_bytes_per_launch": B, "kernel_mean_us": round(k_us, 3),
         "timing": "HIP events around each eager launch on the library stream"}
    rp = rocprof_mean_us(ctx)
    if rp:
        r["rocprof_kernel_mean_us"] = rp
        r["frac_rocprof"] = round(B / (rp * 1e-6) / 1e9 / PEAK_GBPS, 4)
    if row["plan"]["splits"] > 1 and not row.get("reduce_kernel_us"):
        r["split_merge"] = ("in the kernel: its last workgroup per KV head merges the splits, "
                            "so kernel_mean_us includes the merge and no combine kernel runs")
    return r


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
    ap.add_argument("--no-configs", dest="configs", action="store_false",
                    help="skip the C1/C2/C4 rows and the C3 split sweep")
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
    ap.add_argument("--block-mix", choices=sorted(MIXES), default="q4_k_m",
                    help="--profile-block: the projection weight mix")
    ap.add_argument("--profile-block", action="store_true",
                    help="for rocprofv3: the attention-block graph at --ctx2 only, then exit")
    ap.add_argument("--profile-formats", action="store_true",
                    help="for rocprofv3: the attention-block graph at --ctx2 with q, k, v and o "
                         "in each GGUF type in turn, then exit")
    ap.add_argument("--formats", default=None,
                    help="--profile-formats: comma-separated type names (F32, Q8_0, IQ3_S, ...)")
    ap.add_argument("--profile-block-batch", type=int, default=0, metavar="K",
                    help="for rocprofv3: the K-token attention-block graph at --ctx2 only, then exit")
    ap.add_argument("--profile-workload", action="store_true",
                    help="for rocprofv3: only the warm-up and K eager layer-calls at --ctx "
                         "(no graph replay, no second context, no CPU baseline), then exit")
    ap.add_argument("--kv", choices=("f32", "q8"), default="f32",
                    help="KV cache of --profile-workload")
    ap.add_argument("--profile-verify", type=int, default=0, metavar="K",
                    help="for rocprofv3: speculative verification of K tokens at --ctx, then exit")
    ap.add_argument("--profile-prefill", type=int, default=0, metavar="P",
                    help="for rocprofv3: C5 prefill of P tokens (K graph + K eager calls), then exit")
    ap.add_argument("--prefill-f32", action="store_true",
                    help="--profile-prefill: fp32 inputs (llmp_attn_prefill_f32)")
    ap.add_argument("--profile-config", choices=sorted(SHAPES), default=None,
                    help="for rocprofv3: --steps layer-calls of one decode config (C1 pos 511, "
                         "C2 at --ctx or 4096, C3, C4 at 8192), then exit")
    ap.add_argument("--graph", action="store_true", help="--profile-config: one graph replay")
    ap.add_argument("--local", choices=("all", "local", "global"), default="all",
                    help="--profile-config C4: which layers")
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
    rot = int(args.rotate_gib * 2**30)
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    if args.profile_workload:
        return profile_workload(args.ctx, args.steps, args.warmup, args.splits, rot,
                                q8=args.kv == "q8")
    if args.profile_config:
        loc = {"all": None, "local": True, "global": False}[args.local]
        ctx = args.ctx if args.ctx != 32768 or args.profile_config == "C3" else 0
        return profile_config(args.profile_config, ctx, args.steps, rot, args.graph, loc)
    if args.profile_prefill:
        r = prefill_run(args.profile_prefill, args.steps, f32=args.prefill_f32)
        log(f"[bench] profile prefill: P={args.profile_prefill}, {r}")
        return 0
    if args.profile_block:
        r = block_run(args.ctx2 or 4096, args.steps, q8_input=args.block_q8, mix=args.block_mix)
        log(f"[bench] profile block: {r}")
        return 0
    if args.profile_formats:
        # projection formats (all, or the --formats list), q, k, v and o of one type each (28
        # layers, graph replays); with --profile-block-batch K, K tokens per call
        pick = [t for t in GGUF_NAMES if args.formats is None or GGUF_NAMES[t] in args.formats.split(",")]
        for t in pick:
            if args.profile_block_batch:
                r = block_batch_run(args.ctx2 or 4096, args.profile_block_batch, args.steps, mix=(t, t, t, t))
            else:
                r = block_run(args.ctx2 or 4096, args.steps, mix=(t, t, t, t))
            log(f"[bench] profile formats: {GGUF_NAMES[t]} {r}")
        return 0
    if args.profile_block_batch:
        r = block_batch_run(args.ctx2 or 4096, args.profile_block_batch, args.steps, q8_input=args.block_q8)
        log(f"[bench] profile block batch: {r}")
        return 0
    if args.profile_verify:
        r = verify_run(args.ctx, args.profile_verify, args.steps, rot)
        log(f"[bench] profile verify: {r}")
        return 0
    info = hfp.device_info()
    facts = host_facts()
    log(f"[bench] device {info['arch']} with {info['n_cu']} CUs; host {facts}")
    main_run = headline_run(args.ctx, args.steps, args.warmup, args.splits, rot)
    log(f"[bench] C3 ctx {args.ctx}: {main_run['us_per_layer_call_k_steps']} us/layer-call over "
        f"{args.steps} steps (median {main_run['us_per_layer_call']}), split kernel "
        f"{main_run['split_kernel_us']} us")
    second = None
    if args.ctx2:
        with DecodeRig(C3, args.ctx2, rot) as rig:
            second = decode_row(rig, args.ctx2 - 1, args.splits)
        log(f"[bench] C3 ctx {args.ctx2}: {second['us_per_layer_call']} us/layer-call, "
            f"split kernel {second['split_kernel_us']} us")

    configs = sweep = None
    if args.configs:
        configs = config_rows(rot)
        sweep = split_sweep(rot)

    q8_runs = []
    if args.q8:
        for ctx in [args.ctx] + ([args.ctx2] if args.ctx2 else []):
            with DecodeRig(C3, ctx, rot, q8=True) as rig:
                r = decode_row(rig, ctx - 1, args.splits)
            r["ctx"] = ctx
            log(f"[bench] C3 ctx {ctx} Q8_0: {r['us_per_layer_call']} us/layer-call, split "
                f"kernel {r['split_kernel_us']} us")
            q8_runs.append(r)

    verify = []
    if args.verify:
        for K in (4, 8, 16):
            r = verify_run(args.ctx, K, 100, rot)
            r["decode_calls_us"] = round(K * main_run["us_per_layer_call"], 2)
            r["speedup_vs_k_decode_calls"] = round(r["decode_calls_us"] / r["us_per_call"], 2)
            log(f"[bench] verify K={K} at ctx {args.ctx}: {r['us_per_call']} us/call "
                f"({r['speedup_vs_k_decode_calls']}x vs {K} decode calls)")
            verify.append(r)

    prefill = []
    if args.prefill:
        for P, f32 in ((512, False), (2048, False), (2048, True)):
            r = prefill_run(P, 20, f32=f32)
            log(f"[bench] prefill C5 P={P} {r['inputs']}: {r['us_per_call']} us/call, attention "
                f"kernel {r['attn_kernel_us']} us ({r['attn_kernel_causal_tflops']} causal TFLOP/s)")
            prefill.append(r)

    block = block_q8 = block_q3kl = block_q3kl_q8 = block_batch = None
    if args.block:
        block = block_run(args.ctx2 or 4096, 200)
        if second is not None:
            attn_us = second["us_per_layer_call"]
            block["attention_core_us"] = round(attn_us, 2)
            proj_us = block["us_per_layer_call"] - attn_us
            block["projections_us"] = round(proj_us, 2)
            if proj_us > 0:
                block["projection_weight_gbps"] = round(block["weight_bytes_per_layer"] / (proj_us * 1e-6) / 1e9, 1)
        log(f"[bench] attention block C3 Q4_K_M at ctx {block['ctx']}: {block['us_per_layer_call']} us/layer")
        block_q8 = block_run(args.ctx2 or 4096, 200, q8_input=True)
        log(f"[bench] attention block, Q8_1 input: {block_q8['us_per_layer_call']} us/layer")
        block_q3kl = block_run(args.ctx2 or 4096, 200, mix="q3_k_l")
        if second is not None:
            block_q3kl["projections_us"] = round(block_q3kl["us_per_layer_call"] - second["us_per_layer_call"], 2)
            if block_q3kl["projections_us"] > 0:
                block_q3kl["projection_weight_gbps"] = round(
                    block_q3kl["weight_bytes_per_layer"] / (block_q3kl["projections_us"] * 1e-6) / 1e9, 1)
        log(f"[bench] attention block C3 Q3_K_L: {block_q3kl['us_per_layer_call']} us/layer")
        block_q3kl_q8 = block_run(args.ctx2 or 4096, 200, q8_input=True, mix="q3_k_l")
        log(f"[bench] attention block C3 Q3_K_L, Q8_1 input: {block_q3kl_q8['us_per_layer_call']} us/layer")
        block_batch = []
        for ctx_b, K, nl in ((4096, 4, 28), (4096, 16, 28), (32768, 4, 8), (32768, 16, 8)):
            r = block_batch_run(ctx_b, K, 40, nl)
            log(f"[bench] attention block, {K} tokens at ctx {ctx_b}: {r['us_per_call']} us/call "
                f"({r['single_token_blocks_us']} us as {K} single-token blocks)")
            block_batch.append(r)
        r = block_batch_run(4096, 16, 40, 28, q8_input=True)
        log(f"[bench] attention block, 16 tokens at ctx 4096, Q8_1 input: {r['us_per_call']} us/call "
            f"({r['single_token_blocks_us']} us as 16 single-token blocks)")
        block_batch.append(r)

    q8_prefill = q8_verify = None
    if args.q8 and args.prefill:
        q8_prefill = prefill_run(2048, 20, q8=True)
        log(f"[bench] prefill C5 P=2048 Q8_0: {q8_prefill['us_per_call']} us/call")
    if args.q8 and args.verify:
        q8_verify = verify_run(args.ctx, 16, 100, rot, q8=True)
        q8_dec = [r for r in q8_runs if r["ctx"] == args.ctx]
        if q8_dec:
            q8_verify["decode_calls_us"] = round(16 * q8_dec[0]["us_per_layer_call"], 2)
            q8_verify["speedup_vs_k_decode_calls"] = round(
                q8_verify["decode_calls_us"] / q8_verify["us_per_call"], 2)
        log(f"[bench] verify K=16 at ctx {args.ctx} Q8_0: {q8_verify['us_per_call']} us/call")

    cpu = cpu_all = None
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU restatement ...")
        cpu_all = cpu_baselines(args.cpu_seconds, facts) if args.configs else {
            "C3_ctx32768": cpu_time(C3, args.ctx, args.cpu_seconds, cpu_threads(C3, facts))}
        head = cpu_all["C3_ctx32768"]
        cpu = {"value": head["kv_read_gbps"], "unit": "GB/s", "cores": head["threads"],
               "kind": "port",
               "sample": f"{head['calls']} layer-calls of the C3 shape at ctx {args.ctx} "
                         f"(median {head['us_per_layer_call']} us/layer-call), "
                         f"oracle/attn_oracle.c, {head['threads']} threads over query heads",
               "us_per_layer_call": head["us_per_layer_call"],
               "threads_rule": "min(affinity CPUs, CPU share (OMP_NUM_THREADS), query heads)",
               **facts}

    ms_per_step = main_run["ms_per_step"]
    line = {
        "metric": metric,
        "value": main_run["kv_read_gbps_k_steps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) Q/K/V and KV cache (K x 0.5), seeded",
        "config": {"workload": f"C3 Llama-3.2-3B decode attention, ctx {args.ctx}",
                   "heads_q": HQ, "heads_kv": HKV, "head_dim": D, "ctx": args.ctx,
                   "splits": main_run["plan"]["splits"], "waves": main_run["plan"]["waves"],
                   "kv_layers_rotated": main_run["n_layers"]},
        "us_per_layer_call": main_run["us_per_layer_call_k_steps"],
        "kv_read_pct_of_hbm_peak": round(100 * main_run["kv_read_gbps_k_steps"] / PEAK_GBPS, 2),
        "median_us_per_layer_call": main_run["us_per_layer_call"],
        "median_layer_calls_timed": main_run["layer_calls_timed"],
        "reduce_kernel_us": main_run["reduce_kernel_us"],
        "roofline": roofline_of(main_run, args.ctx, kernel_name(main_run["plan"])),
        "cpu_baseline": cpu,
    }
    if second is not None:
        second["roofline"] = roofline_of(second, args.ctx2, kernel_name(second["plan"]))
        line[f"ctx{args.ctx2}"] = second
    if configs is not None:
        line["decode_configs"] = configs
        line["c3_split_sweep"] = sweep
    if cpu_all is not None:
        line["cpu_baseline_per_config"] = cpu_all
    if q8_runs:
        line["q8_0_kv"] = []
        for r in q8_runs:
            r["workload"] = f"C3 decode attention over a Q8_0 cache, ctx {r['ctx']}"
            r["kernel"] = f"decode_q8_mfma_kernel<128, 3, {r['plan']['waves']}, true>"
            line["q8_0_kv"].append(r)
    if prefill:
        line["prefill_c5_llama1b"] = prefill
    if verify:
        line["speculative_verify_c3"] = verify
    if block is not None:
        line["attn_block_c3_q4_k_m"] = block
    if block_q8 is not None:
        line["attn_block_c3_q4_k_m_q8_1_input"] = block_q8
    if block_q3kl is not None:
        line["attn_block_c3_q3_k_l"] = block_q3kl
    if block_q3kl_q8 is not None:
        line["attn_block_c3_q3_k_l_q8_1_input"] = block_q3kl_q8
    if block_batch:
        line["attn_block_batch_c3_q4_k_m"] = block_batch
    if q8_prefill is not None:
        line["q8_0_prefill_c5_llama1b"] = q8_prefill
    if q8_verify is not None:
        line["q8_0_speculative_verify_c3"] = q8_verify
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
