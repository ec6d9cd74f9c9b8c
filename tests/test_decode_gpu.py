"""GPU parity of the decode attention path (libllmp_hip.so through HipForwardPass) against the
CPU oracle on the BASELINE configurations, plus edge cases and error plumbing.

Bar: attention output max-abs error <= 1e-4 (and <= 1e-4 + 1e-3*|ref| elementwise) versus the
oracle (fp32 accumulate); the KV cache after the call is bit-identical to the oracle's (append
and position indexing exact)."""
import ctypes as C

import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from tests import decode_cases as dc

pytestmark = pytest.mark.gpu


def _run(fp, c, max_seq, d, layer, pos, splits, what, check_cache=True, oracle=None):
    dc.log(f"[gpu] {what}: layer={layer} pos={pos} splits={splits}")
    fp.kv.write(layer, 0, d.kc, d.vc)
    st = hfp.InferenceState.create(c)
    st.q[:], st.k[:], st.v[:] = d.q, d.k, d.v
    fp.forwardAttentionOnly(st, layer, pos, splits)
    out, kc, vc = oracle if oracle is not None else dc.oracle_call(c, max_seq, d, layer, pos)
    err = dc.compare_out(st.xb2, out, what)
    if check_cache:
        dc.compare_cache(fp, layer, kc, vc, what)
    else:
        dc.compare_cache(fp, layer, kc, vc, what, rows=(pos, pos + 1))
    dc.log(f"[gpu] {what}: ok, max abs err {err:.2e}")
    return out, kc, vc


# --------------------------------------------------------------------------- C1: Llama-3.2-1B
@pytest.mark.parametrize("splits", [0, 1, 3, 16, 64])
def test_c1_llama1b_pos511(splits):
    c = hfp.ModelConfig(32, 8, 64, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    d = dc.make_layer(c, 512, 511, seed=101)
    with hfp.HipForwardPass(c, 512) as fp:
        _run(fp, c, 512, d, 0, 511, splits, "C1 Llama-3.2-1B pos 511")


# ------------------------------------------------------------ C3: Llama-3.2-3B (headline shape)
@pytest.fixture(scope="module", params=[4096, 32768], ids=["ctx4k", "ctx32k"])
def c3(request):
    n = request.param
    c = hfp.ModelConfig(24, 8, 128, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    d = dc.make_layer(c, n, n - 1, seed=303, k_scale=0.5)
    ref = dc.oracle_call(c, n, d, 0, n - 1)
    fp = hfp.HipForwardPass(c, n)
    yield c, n, d, ref, fp
    fp.close()


@pytest.mark.parametrize("splits", [0, 8, 16, 32, 64, 128, 1000])
def test_c3_llama3b_split_sweep(c3, splits):
    # 8..32 splits at ctx 32768 run 8-wave workgroups (>= 1024 rows per split), the rest 4.
    c, n, d, ref, fp = c3
    _run(fp, c, n, d, 0, n - 1, splits, f"C3 Llama-3.2-3B ctx {n}", check_cache=(splits == 0),
         oracle=ref)


# ------------------------------------------------------------------- C2: Qwen3-0.6B, QK-norm
@pytest.mark.parametrize("n,layers", [(1024, range(28)), (4096, (0, 5, 13, 20, 27)),
                                      (16384, (0, 13, 27))])
def test_c2_qwen3_qknorm(n, layers):
    c = hfp.ModelConfig(16, 8, 128, 28, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6,
                        norm_eps=1e-6)
    datas = {l: dc.make_layer(c, n, n - 1, seed=2000 + l, qk_norm=True) for l in layers}
    qk = [datas[l].qk_norm if l in datas else (np.ones(128, np.float32),) * 2 for l in range(28)]
    with hfp.HipForwardPass(c, n, qk_norm=qk) as fp:
        for l in layers:
            _run(fp, c, n, datas[l], l, n - 1, 0, f"C2 Qwen3-0.6B ctx {n}",
                 check_cache=(n <= 4096))


# ---------------------------------------------------- C4: Gemma-3-1B, MQA, window 512 / global
def _gemma3(max_seq):
    return hfp.ModelConfig(4, 1, 256, 6, architecture=hfp.ARCH_GEMMA3, rope_freq_base=1e6,
                           norm_eps=1e-6, sliding_window=512)


def test_c4_gemma3_local_and_global_layers():
    c = _gemma3(8192)
    datas = {l: dc.make_layer(c, 8192, 8191, seed=400 + l, qk_norm=True) for l in range(6)}
    with hfp.HipForwardPass(c, 8192, qk_norm=[datas[l].qk_norm for l in range(6)]) as fp:
        for l in range(6):
            kind = "global" if l % 6 == 5 else "local W=512"
            _run(fp, c, 8192, datas[l], l, 8191, 0, f"C4 Gemma-3-1B ctx 8192 layer {l} ({kind})")


@pytest.mark.parametrize("pos", [0, 1, 510, 511, 512, 513, 1000])
def test_c4_window_boundaries(pos):
    c = _gemma3(1024)
    d = dc.make_layer(c, 1024, pos, seed=450 + pos, qk_norm=True)
    qk = [d.qk_norm] * 6
    with hfp.HipForwardPass(c, 1024, qk_norm=qk) as fp:
        _run(fp, c, 1024, d, 0, pos, 0, "C4 window boundary (local layer)")
        _run(fp, c, 1024, d, 5, pos, 0, "C4 window boundary (global layer)")


# ------------------------------------------------------------------------------ shapes
SHAPES = [(8, 8, 64), (16, 8, 64), (24, 8, 64), (32, 8, 64), (48, 8, 64), (64, 8, 64),
          (8, 8, 128), (16, 8, 128), (32, 4, 128), (48, 8, 128), (64, 8, 128),
          (4, 4, 256), (8, 4, 256), (12, 4, 256), (16, 4, 256), (24, 4, 256), (32, 4, 256),
          (4, 1, 256)]


@pytest.mark.parametrize("hq,hkv,dim", SHAPES, ids=[f"{a}-{b}-{c}" for a, b, c in SHAPES])
def test_every_supported_group_and_head_dim(hq, hkv, dim):
    c = hfp.ModelConfig(hq, hkv, dim, 1, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6,
                        norm_eps=1e-6)
    d = dc.make_layer(c, 1200, 999, seed=hq * 1000 + hkv * 10 + dim, qk_norm=True)
    with hfp.HipForwardPass(c, 1200, qk_norm=[d.qk_norm]) as fp:
        for splits in (0, 1, 7):
            _run(fp, c, 1200, d, 0, 999, splits, f"shape {hq}/{hkv}/{dim}")


@pytest.mark.parametrize("hq,hkv,pos", [(64, 8, 991), (64, 8, 511), (16, 2, 250), (32, 8, 671),
                                        (8, 8, 300)],
                         ids=["g8-991", "g8-511", "g8-250", "g4-671", "g1-300"])
def test_two_wave_workgroups_at_head_dim_64(hq, hkv, pos):
    """The default plan at head_dim 64 over short splits (at most 32 rows) runs 2-wave
    workgroups, whose LDS merge gives one thread to each of its 16 partials and G heads (128
    pairs at G=8: every thread of the workgroup)."""
    c = hfp.ModelConfig(hq, hkv, 64, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=5e5)
    d = dc.make_layer(c, 1024, pos, seed=hq + pos)
    with hfp.HipForwardPass(c, 1024) as fp:
        plan = fp.decodePlan(0, pos)
        assert plan["waves"] == 2 and plan["rows_per_split"] <= 32, plan
        _run(fp, c, 1024, d, 0, pos, 0, f"2-wave {hq}/{hkv}/64 pos {pos} {plan}")


# ------------------------------------------------------------------------------ edge cases
def test_pos0_output_is_v0():
    c = hfp.ModelConfig(32, 8, 64, 1, rope_freq_base=500000.0)
    d = dc.make_layer(c, 64, 0, seed=7)
    with hfp.HipForwardPass(c, 64) as fp:
        out, _, _ = _run(fp, c, 64, d, 0, 0, 0, "pos 0")
        got = fp.downloadXb2()
        assert np.array_equal(got, np.repeat(d.v.reshape(8, 64), 4, axis=0).reshape(-1))


def test_last_row_of_cache_and_splits_above_rows():
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    d = dc.make_layer(c, 300, 299, seed=8)
    with hfp.HipForwardPass(c, 300) as fp:
        _run(fp, c, 300, d, 0, 299, 1024, "pos = max_seq-1, splits 1024 > rows")
        _run(fp, c, 300, d, 0, 299, 299, "splits = rows - 1")


def test_nope_layer_and_softcap_and_custom_scale():
    c = hfp.ModelConfig(16, 4, 128, 4, architecture=hfp.ARCH_GEMMA2, rope_freq_base=1e4,
                        attn_logit_soft_cap=50.0, attention_scale=0.125, sliding_window=300,
                        no_rope_layer_interval=4)
    for layer in (0, 1, 3):
        d = dc.make_layer(c, 700, 650, seed=90 + layer, k_scale=3.0)
        with hfp.HipForwardPass(c, 700) as fp:
            _run(fp, c, 700, d, layer, 650, 0, f"gemma2-like layer {layer} (softcap, scale, window, NoPE)")


def test_consecutive_decode_steps_match_sequential_oracle():
    c = hfp.ModelConfig(16, 8, 128, 2, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6, norm_eps=1e-6)
    rng = np.random.default_rng(55)
    max_seq, p0, steps = 2048, 1500, 12
    base = dc.make_layer(c, max_seq, p0, seed=56, qk_norm=True)
    kc, vc = base.kc.copy(), base.vc.copy()
    with hfp.HipForwardPass(c, max_seq, qk_norm=[base.qk_norm] * 2) as fp:
        fp.kv.write(1, 0, kc, vc)
        for i in range(steps):
            pos = p0 + i
            d = dc.LayerData(kc, vc, rng.standard_normal(c.q_dim, dtype=np.float32),
                             rng.standard_normal(c.kv_dim, dtype=np.float32),
                             rng.standard_normal(c.kv_dim, dtype=np.float32), base.qk_norm)
            dc.log(f"[gpu] decode step {i} pos {pos}")
            st = hfp.InferenceState.create(c)
            st.q[:], st.k[:], st.v[:] = d.q, d.k, d.v
            fp.forwardAttentionOnly(st, 1, pos)
            out, kc, vc = dc.oracle_call(c, max_seq, d, 1, pos)
            dc.compare_out(st.xb2, out, f"step {i}")
        dc.compare_cache(fp, 1, kc, vc, "after decode steps")


def test_error_codes():
    c = hfp.ModelConfig(8, 2, 64, 2, rope_freq_base=1e4)
    with hfp.HipForwardPass(c, 128) as fp:
        h = fp.kv.handle
        args = (fp.gpuQ.ptr, fp.gpuK.ptr, fp.gpuV.ptr, fp.gpuXb2.ptr)
        assert _lib.status("llmp_attn_decode", h, 0, 128, *args, 0, 0) == 2   # pos >= max_seq
        assert _lib.status("llmp_attn_decode", h, 0, -1, *args, 0, 0) == 2
        assert _lib.status("llmp_attn_decode", h, 2, 5, *args, 0, 0) == 2     # bad layer
        assert _lib.status("llmp_attn_decode", h, 0, 5, *args, 2000, 0) == 1  # splits > max
        assert _lib.status("llmp_attn_decode", h + 999, 0, 5, *args, 0, 0) == 8
        with pytest.raises(_lib.LlmpError) as ei:
            fp.forwardAttentionPart(0, 128)
        assert ei.value.code == 2 and "position 128" in ei.value.message
        k = np.zeros((4, c.kv_dim), np.float32)
        with pytest.raises(_lib.LlmpError):
            fp.kv.write(0, 126, k, k)                                          # rows past the end
        # a layer never configured
        kv = hfp.KvCache(1, 16, 2, 64)
        try:
            assert _lib.status("llmp_attn_decode", kv.handle, 0, 1, *args, 0, 0) == 1
        finally:
            kv.destroy()
        # unsupported shapes
        hd = C.c_uint64()
        assert _lib.status("llmp_kv_create", 1, 16, 2, 112, 0, C.byref(hd)) == 6
        assert _lib.status("llmp_kv_create", 1, 16, 2, 96, 1, C.byref(hd)) == 6   # Q8_0 at 96
        assert _lib.status("llmp_layer_config", h, 0, 9, 2, 64, 0, 0, 0, 1, 0.0, 0.0, 1e-5,
                           None, None) == 1   # 9 query heads over 2 KV heads
        # group 9 runs as 3 groups of 3 per KV head (any group has a divisor with a kernel)
        assert _lib.status("llmp_layer_config", h, 0, 18, 2, 64, 0, 0, 0, 1, 0.0, 0.0, 1e-5,
                           None, None) == 0
        # an allocation beyond HBM is refused before touching the device
        assert _lib.status("llmp_kv_create", 4096, 1 << 20, 64, 128, 0, C.byref(hd)) == 5


def test_split_merge_in_the_split_kernel():
    """Plans whose splits the split kernel merges itself (its last workgroup per KV head, through
    agent-scope atomic partials and a per-head counter): C1 at pos 511 (16 splits of 2-wave
    workgroups) and C3 at 32k (24 splits of 8 waves): no combine launch, the oracle's output,
    and the counters re-armed (a second call, another layer, agrees too)."""
    for c, n, seed in ((hfp.ModelConfig(32, 8, 64, 2, rope_freq_base=500000.0), 512, 41),
                       (hfp.ModelConfig(24, 8, 128, 2, rope_freq_base=500000.0), 32768, 42)):
        d = dc.make_layer(c, n, n - 1, seed=seed, k_scale=0.5)
        with hfp.HipForwardPass(c, n) as fp:
            plan = fp.decodePlan(0, n - 1)
            assert plan["waves"] in (2, 8), plan
            _lib.call("llmp_profile_enable", fp.kv.handle, 1)
            out, kc, vc = dc.oracle_call(c, n, d, 0, n - 1)
            for layer in (0, 1, 0):
                _run(fp, c, n, d, layer, n - 1, 0, f"merged in the split kernel, layer {layer}",
                     check_cache=False, oracle=(out, kc, vc))
            cnt, ms = C.c_int(), C.c_double()
            _lib.call("llmp_profile_read", fp.kv.handle, _lib.LLMP_PROF_DECODE_REDUCE, C.byref(cnt), C.byref(ms))
            assert cnt.value == 0


def test_profile_counters_count_launches():
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    d = dc.make_layer(c, 4096, 4095, seed=9, k_scale=0.5)
    with hfp.HipForwardPass(c, 4096) as fp:
        fp.kv.write(0, 0, d.kc, d.vc)
        fp.uploadQKV(d.q, d.k, d.v)
        _lib.call("llmp_profile_enable", fp.kv.handle, 1)
        for _ in range(5):
            fp.forwardAttentionPart(0, 4095, 32)     # split kernel + combine kernel
        for _ in range(2):
            # 8 splits of 4-wave workgroups: the combine kernel too (the split kernel merges
            # its splits itself only with 2- or 8-wave workgroups)
            fp.forwardAttentionPart(0, 4095, 8)
        for _ in range(3):
            fp.forwardAttentionPart(0, 4095, 1)      # one split: no combine kernel
        cnt, ms = C.c_int(), C.c_double()
        _lib.call("llmp_profile_read", fp.kv.handle, _lib.LLMP_PROF_DECODE_SPLIT, C.byref(cnt), C.byref(ms))
        assert cnt.value == 10 and ms.value > 0
        _lib.call("llmp_profile_read", fp.kv.handle, _lib.LLMP_PROF_DECODE_REDUCE, C.byref(cnt), C.byref(ms))
        assert cnt.value == 7
        _lib.call("llmp_profile_reset", fp.kv.handle)
        _lib.call("llmp_profile_read", fp.kv.handle, 0, C.byref(cnt), C.byref(ms))
        assert cnt.value == 0


@pytest.mark.parametrize("splits", [0, 1, 1000])
def test_graph_replay_matches_eager(splits):
    """Decode calls captured into a HIP graph (llmp_graph_*) give the eager results on every
    replay, with other eager work and synchronisations between replays."""
    c = hfp.ModelConfig(24, 8, 128, 3, rope_freq_base=500000.0)
    d = dc.make_layer(c, 4096, 4095, seed=77, k_scale=0.5)
    with hfp.HipForwardPass(c, 4096) as fp:
        for layer in range(3):
            fp.kv.write(layer, 0, d.kc, d.vc)
        fp.uploadQKV(d.q, d.k, d.v)
        fp.forwardAttentionPart(0, 4095, splits)
        eager = fp.downloadXb2()
        out, _, _ = dc.oracle_call(c, 4096, d, 0, 4095)
        dc.compare_out(eager, out, "eager before capture")
        g = C.c_uint64()
        _lib.call("llmp_graph_begin", 0)
        fp.forwardAttentionPart(1, 4095, splits)
        fp.forwardAttentionPart(0, 4095, splits)
        _lib.call("llmp_graph_end", 0, C.byref(g))
        try:
            for rep in range(4):
                dc.log(f"[gpu] graph replay {rep} splits={splits}")
                fp.forwardAttentionPart(2, 4095, splits)       # eager work between replays
                fp.sync()
                _lib.call("llmp_graph_launch", g.value, 0)
                fp.sync()
                got = fp.downloadXb2()
                assert np.array_equal(got, eager), f"replay {rep} differs from eager"
        finally:
            _lib.call("llmp_graph_destroy", g.value)
        dc.compare_cache(fp, 0, *dc.oracle_call(c, 4096, d, 0, 4095)[1:], "cache after replays")


# ------------------------------------------------- device-side position (reference graph mode)
def test_device_position_matches_oracle_and_host_position():
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    d = dc.make_layer(c, 4096, 3000, seed=88, k_scale=0.5)
    out, kc, vc = dc.oracle_call(c, 4096, d, 0, 3000)
    with hfp.HipForwardPass(c, 4096) as fp:
        fp.kv.write(0, 0, d.kc, d.vc)
        fp.uploadQKV(d.q, d.k, d.v)
        fp.updateTokenParams(3000)
        dc.log("[gpu] device-position decode at 3000")
        fp.forwardAttentionPartDevicePosition(0)
        dc.compare_out(fp.downloadXb2(), out, "device position")
        dc.compare_cache(fp, 0, kc, vc, "device position")


def test_graph_of_device_position_decode_replays_across_tokens():
    """One capture of two layers' decode calls replayed for 10 consecutive tokens: the
    positions and q/k/v change between replays (uploaded outside the graph, as the reference's
    uploadXAndUpdateParams does before cuGraphLaunch)."""
    c = hfp.ModelConfig(16, 8, 128, 2, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6,
                        norm_eps=1e-6)
    max_seq, p0, steps = 2048, 1000, 10
    rng = np.random.default_rng(89)
    base = [dc.make_layer(c, max_seq, p0, seed=90 + l, qk_norm=True) for l in range(2)]
    caches = [(b.kc.copy(), b.vc.copy()) for b in base]
    with hfp.HipForwardPass(c, max_seq, qk_norm=[b.qk_norm for b in base]) as fp:
        for l in range(2):
            fp.kv.write(l, 0, *caches[l])
        outs = [hfp.DeviceBuffer(c.q_dim * 4) for _ in range(2)]
        g = C.c_uint64()
        _lib.call("llmp_graph_begin", 0)
        for l in range(2):
            _lib.call("llmp_attn_decode_devpos", fp.kv.handle, l, fp.gpuTokenParams.ptr,
                      fp.gpuQ.ptr, fp.gpuK.ptr, fp.gpuV.ptr, outs[l].ptr, 0, 0)
        _lib.call("llmp_graph_end", 0, C.byref(g))
        try:
            for i in range(steps):
                pos = p0 + i
                q = rng.standard_normal(c.q_dim, dtype=np.float32)
                k = rng.standard_normal(c.kv_dim, dtype=np.float32)
                v = rng.standard_normal(c.kv_dim, dtype=np.float32)
                fp.uploadQKV(q, k, v)
                fp.updateTokenParams(pos)
                dc.log(f"[gpu] graph replay at position {pos}")
                _lib.call("llmp_graph_launch", g.value, 0)
                fp.sync()
                for l in range(2):
                    d = dc.LayerData(caches[l][0], caches[l][1], q, k, v, base[l].qk_norm)
                    want, kc, vc = dc.oracle_call(c, max_seq, d, l, pos)
                    caches[l] = (kc, vc)
                    dc.compare_out(outs[l].download(np.float32, c.q_dim), want,
                                   f"graph replay layer {l} pos {pos}")
        finally:
            _lib.call("llmp_graph_destroy", g.value)
            for b in outs:
                b.free()
        for l in range(2):
            dc.compare_cache(fp, l, *caches[l], f"cache layer {l} after graph replays")


def test_device_position_outside_cache_is_a_no_op():
    c = hfp.ModelConfig(8, 2, 64, 1, rope_freq_base=1e4)
    d = dc.make_layer(c, 64, 63, seed=91)
    with hfp.HipForwardPass(c, 64) as fp:
        fp.kv.write(0, 0, d.kc, d.vc)
        fp.uploadQKV(d.q, d.k, d.v)
        sentinel = np.full(c.q_dim, 7.0, np.float32)
        fp.gpuXb2.upload(sentinel)
        for bad in (64, 1000, -1):
            fp.updateTokenParams(bad)
            fp.forwardAttentionPartDevicePosition(0, splits=4)
            fp.sync()
            assert np.array_equal(fp.downloadXb2(), sentinel)
        k_after, v_after = fp.kv.read(0, 0, 64)
        assert np.array_equal(k_after, d.kc) and np.array_equal(v_after, d.vc)
