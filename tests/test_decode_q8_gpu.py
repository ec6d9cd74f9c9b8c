"""GPU parity of decode attention over a Q8_0 KV cache (KVCache.Mode.Q8_0: int8 quants plus
one fp32 scale per 32 values, KVCache.java:11-28) against the CPU oracle's Q8_0 mode, under
both contracts the JVM can run: the scalar one (LLMP_KV_Q8_0: quantizeBlocksScalar /
dotQ8BlockScalar / saxpyQ8BlockScalar, KVCache.java:218-282) and the 8-lane SIMD one
(LLMP_KV_Q8_0_TRUNC: SimdQ8KvOps.java:37-117, truncating quantizer).

Bar: attention output max-abs <= 1e-4 (and <= 1e-4 + 1e-3*|ref|) versus the oracle; the
appended row's quants and scales, and every other row, bit-identical to the oracle's."""
import ctypes as C

import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from oracle import oracle as orc
from tests import decode_cases as dc

pytestmark = pytest.mark.gpu

MODES = [(_lib.LLMP_KV_Q8_0, orc.Q8_SCALAR), (_lib.LLMP_KV_Q8_0_TRUNC, orc.Q8_SIMD8)]
MODE_IDS = ["round", "trunc"]


@pytest.fixture(params=MODES, ids=MODE_IDS)
def mode(request):
    return request.param


def _open(c, max_seq, mode, qk=None):
    return hfp.HipForwardPass(c, max_seq, qk_norm=qk, kv_dtype=mode[0])


def _run(fp, c, max_seq, d, layer, pos, splits, what, mode, check_cache=True, oracle=None):
    dc.log(f"[gpu] Q8 {what}: mode={mode[0]} layer={layer} pos={pos} splits={splits}")
    fp.kv.write_q8(layer, 0, d.kq, d.ks, d.vq, d.vs)
    st = hfp.InferenceState.create(c)
    st.q[:], st.k[:], st.v[:] = d.q, d.k, d.v
    fp.forwardAttentionOnly(st, layer, pos, splits)
    out, cache = oracle if oracle is not None else dc.oracle_call_q8(c, max_seq, d, layer, pos,
                                                                      mode=mode[1])
    err = dc.compare_out(st.xb2, out, "Q8 " + what)
    dc.compare_cache_q8(fp, layer, cache, "Q8 " + what,
                        rows=None if check_cache else (pos, pos + 1))
    dc.log(f"[gpu] Q8 {what}: ok, max abs err {err:.2e}")
    return out, cache


@pytest.mark.parametrize("splits", [0, 1, 3, 16, 64])
def test_q8_c1_llama1b_pos511(splits, mode):
    c = hfp.ModelConfig(32, 8, 64, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    d = dc.make_layer_q8(c, 512, 511, seed=101, mode=mode[1])
    with _open(c, 512, mode) as fp:
        _run(fp, c, 512, d, 0, 511, splits, "C1 Llama-3.2-1B pos 511", mode)


@pytest.fixture(scope="module", params=[(n, m) for n in (4096, 32768) for m in MODES],
                ids=[f"ctx{n // 1024}k-{i}" for n in (4096, 32768) for i in MODE_IDS])
def c3q8(request):
    n, m = request.param
    c = hfp.ModelConfig(24, 8, 128, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    d = dc.make_layer_q8(c, n, n - 1, seed=303, k_scale=0.5, mode=m[1])
    ref = dc.oracle_call_q8(c, n, d, 0, n - 1, n_threads=16, mode=m[1])
    fp = _open(c, n, m)
    yield c, n, d, ref, fp, m
    fp.close()


@pytest.mark.parametrize("splits", [0, 16, 128, 1000])
def test_q8_c3_llama3b_split_sweep(c3q8, splits):
    c, n, d, ref, fp, m = c3q8
    _run(fp, c, n, d, 0, n - 1, splits, f"C3 Llama-3.2-3B ctx {n}", m,
         check_cache=(splits == 0), oracle=ref)


def test_q8_c2_qwen3_qknorm(mode):
    c = hfp.ModelConfig(16, 8, 128, 28, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6,
                        norm_eps=1e-6)
    layers = (0, 13, 27)
    datas = {l: dc.make_layer_q8(c, 4096, 4095, seed=2000 + l, qk_norm=True, mode=mode[1])
             for l in layers}
    qk = [datas[l].qk_norm if l in datas else (np.ones(128, np.float32),) * 2 for l in range(28)]
    with _open(c, 4096, mode, qk) as fp:
        for l in layers:
            _run(fp, c, 4096, datas[l], l, 4095, 0, "C2 Qwen3-0.6B ctx 4096", mode)


def test_q8_c4_gemma3_local_and_global_layers(mode):
    c = hfp.ModelConfig(4, 1, 256, 6, architecture=hfp.ARCH_GEMMA3, rope_freq_base=1e6,
                        norm_eps=1e-6, sliding_window=512)
    with _open(c, 2048, mode, [None] * 6) as fp:
        for layer in (0, 5):
            d = dc.make_layer_q8(c, 2048, 1500, seed=400 + layer, mode=mode[1])
            _run(fp, c, 2048, d, layer, 1500, 0, f"C4 Gemma-3-1B layer {layer}", mode)


SHAPES = [(8, 8, 64), (48, 8, 64), (64, 8, 64), (16, 8, 128), (48, 8, 128), (64, 8, 128),
          (4, 4, 256), (12, 4, 256), (24, 4, 256), (32, 4, 256), (4, 1, 256)]


@pytest.mark.parametrize("hq,hkv,dim", SHAPES, ids=[f"{a}-{b}-{c}" for a, b, c in SHAPES])
def test_q8_every_group_and_head_dim(hq, hkv, dim, mode):
    c = hfp.ModelConfig(hq, hkv, dim, 1, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6,
                        norm_eps=1e-6)
    d = dc.make_layer_q8(c, 1200, 999, seed=hq * 1000 + hkv * 10 + dim, qk_norm=True,
                         mode=mode[1])
    with _open(c, 1200, mode, [d.qk_norm]) as fp:
        for splits in (0, 1, 7):
            _run(fp, c, 1200, d, 0, 999, splits, f"shape {hq}/{hkv}/{dim}", mode)


RAGGED = [(8, 8, 64), (24, 8, 128), (16, 4, 256)]


@pytest.mark.parametrize("hq,hkv,dim", RAGGED, ids=[f"{a}-{b}-{c}" for a, b, c in RAGGED])
def test_q8_short_and_ragged_rows(hq, hkv, dim, mode):
    """GQA groups 1, 3 and 4 (the int8-MFMA score path) at positions 0 to 100: a partial first
    16-key tile, exact tile boundaries, and row `pos` alone in its split, at several split
    counts."""
    c = hfp.ModelConfig(hq, hkv, dim, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    with _open(c, 128, mode) as fp:
        for pos in (0, 1, 15, 16, 17, 31, 32, 33, 100):
            d = dc.make_layer_q8(c, 128, pos, seed=700 + pos, mode=mode[1])
            for splits in (0, 1, 2, 7):
                _run(fp, c, 128, d, 0, pos, splits, f"{hq}/{hkv}/{dim} pos {pos}", mode,
                     check_cache=(splits == 0))


@pytest.mark.parametrize("q_scale", [1e-3, 1.0, 30.0])
def test_q8_query_magnitudes_and_special_blocks(q_scale, mode):
    """The query's int8 parts (per head and 32-dim block: q = s*(Q1 + (Q2 + Q3/254)/254)) at
    small and large magnitudes, with an all-zero block (scale 0) and a block with one dominant
    element next to small ones (the parts must carry the small ones to fp32 precision)."""
    c = hfp.ModelConfig(24, 8, 128, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    d = dc.make_layer_q8(c, 1024, 1000, seed=810, mode=mode[1])
    d.q[:] *= np.float32(q_scale)
    d.q[32:64] = 0.0                                     # head 0, block 1
    d.q[128 + 64:128 + 96] *= np.float32(1e-3)           # head 1, block 2: small values ...
    d.q[128 + 70] = np.float32(8.0 * q_scale)            # ... and one dominant element
    with _open(c, 1024, mode) as fp:
        for splits in (0, 1, 5):
            _run(fp, c, 1024, d, 0, 1000, splits, f"q scale {q_scale}", mode,
                 check_cache=(splits == 0))


@pytest.mark.parametrize("rope_type,rope_dim", [(_lib.LLMP_ROPE_NEOX, 0), (_lib.LLMP_ROPE_NEOX, 64),
                                                (_lib.LLMP_ROPE_NORMAL, 64)])
def test_q8_neox_and_partial_rope(rope_type, rope_dim, mode):
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=1e4, rope_type=rope_type,
                        rope_dim_count=rope_dim)
    d = dc.make_layer_q8(c, 1024, 777, seed=31 + rope_dim, mode=mode[1])
    with _open(c, 1024, mode) as fp:
        _run(fp, c, 1024, d, 0, 777, 0, f"rope {rope_type} dims {rope_dim or 128}", mode)


def test_q8_nope_softcap_custom_scale(mode):
    c = hfp.ModelConfig(16, 4, 128, 4, architecture=hfp.ARCH_GEMMA2, rope_freq_base=1e4,
                        attn_logit_soft_cap=50.0, attention_scale=0.125, sliding_window=300,
                        no_rope_layer_interval=4)
    for layer in (0, 3):
        d = dc.make_layer_q8(c, 700, 650, seed=90 + layer, k_scale=3.0, mode=mode[1])
        with _open(c, 700, mode) as fp:
            _run(fp, c, 700, d, layer, 650, 0, f"gemma2-like layer {layer}", mode)


def test_q8_append_rounding_and_zero_blocks(mode):
    """The appended row on a NoPE layer without QK-norm is quantized from k/v as given: blocks
    with max |x| = 127 (scale 1, so x*inv is x exactly) holding x.5 values, one all-zero block
    (scale 0 -> quants 0), and values whose rounding reaches -128/127."""
    c = hfp.ModelConfig(8, 2, 64, 1, rope_freq_base=1e4, no_rope_layer_interval=1)
    d = dc.make_layer_q8(c, 64, 40, seed=5, mode=mode[1])
    k = np.zeros(c.kv_dim, np.float32)
    k[0:32] = np.array([127.0, -127.0] + [x + 0.5 for x in range(-15, 15)], np.float32)
    k[32:64] = 0.0                                    # zero block
    k[64:96] = np.linspace(-127.0, 127.0, 32, dtype=np.float32)
    k[96:128] = np.array([-127.0] + [-2.5, -1.5, -0.5, 0.5, 1.5, 2.5] * 5 + [126.5], np.float32)
    v = k[::-1].copy()
    d.k, d.v = k, v
    with _open(c, 64, mode) as fp:
        _, cache = _run(fp, c, 64, d, 0, 40, 0, "append rounding", mode)
    kq = cache[0][40]
    if mode[1] == orc.Q8_SCALAR:   # Math.round: ties toward +inf
        assert kq[2] == -14 and kq[3] == -13 and kq[17] == 1 and kq[127] == 127
    else:                          # F2I: toward zero
        assert kq[2] == -14 and kq[3] == -13 and kq[17] == 0 and kq[127] == 126
    assert (kq[32:64] == 0).all() and (cache[1][40][1] == 0.0)


def test_q8_consecutive_steps_and_device_position(mode):
    c = hfp.ModelConfig(16, 8, 128, 1, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6,
                        norm_eps=1e-6)
    rng = np.random.default_rng(77)
    max_seq, p0, steps = 2048, 1500, 8
    base = dc.make_layer_q8(c, max_seq, p0, seed=78, qk_norm=True, mode=mode[1])
    cache = (base.kq.copy(), base.ks.copy(), base.vq.copy(), base.vs.copy())
    with _open(c, max_seq, mode, [base.qk_norm]) as fp:
        fp.kv.write_q8(0, 0, *cache)
        for i in range(steps):
            pos = p0 + i
            d = dc.LayerDataQ8(*cache, rng.standard_normal(c.q_dim, dtype=np.float32),
                               rng.standard_normal(c.kv_dim, dtype=np.float32),
                               rng.standard_normal(c.kv_dim, dtype=np.float32), base.qk_norm)
            dc.log(f"[gpu] Q8 decode step {i} pos {pos} (device position: {i % 2 == 1})")
            fp.uploadQKV(d.q, d.k, d.v)
            if i % 2:
                fp.updateTokenParams(pos)
                fp.forwardAttentionPartDevicePosition(0)
            else:
                fp.forwardAttentionPart(0, pos)
            got = fp.downloadXb2()
            out, cache = dc.oracle_call_q8(c, max_seq, d, 0, pos, mode=mode[1])
            dc.compare_out(got, out, f"Q8 step {i}")
        dc.compare_cache_q8(fp, 0, cache, "Q8 after decode steps")


def test_q8_cache_rejects_fp32_row_access_and_round_trips_layout(mode):
    c = hfp.ModelConfig(8, 2, 64, 2, rope_freq_base=1e4)
    with _open(c, 64, mode) as fp:
        h = fp.kv.handle
        k = np.zeros((4, c.kv_dim), np.float32)
        kp = k.ctypes.data_as(C.POINTER(C.c_float))
        assert _lib.status("llmp_kv_read", h, 0, 0, 4, kp, kp) == 6
        assert _lib.status("llmp_kv_write", h, 0, 0, 4, kp, None) == 6
        assert _lib.status("llmp_kv_read_q8", h, 0, 62, 4, None, None, None, None) == 2
        # Round trip of both layers' quants and scales through the reference layout.
        rng = np.random.default_rng(1)
        for layer in range(2):
            kq = rng.integers(-128, 128, (64, c.kv_dim), dtype=np.int8)
            vq = rng.integers(-128, 128, (64, c.kv_dim), dtype=np.int8)
            ks = rng.random((64, c.kv_dim // 32), dtype=np.float32)
            vs = rng.random((64, c.kv_dim // 32), dtype=np.float32)
            fp.kv.write_q8(layer, 0, kq, ks, vq, vs)
            got = fp.kv.read_q8(layer, 0, 64)
            for g, w in zip(got, (kq, ks, vq, vs)):
                assert np.array_equal(g, w)
            kq0, ks0, _, _ = fp.kv.read_q8(layer, 10, 5)
            assert np.array_equal(kq0, kq[10:15]) and np.array_equal(ks0, ks[10:15])
    with hfp.HipForwardPass(c, 64) as fp:
        assert _lib.status("llmp_kv_read_q8", fp.kv.handle, 0, 0, 1, None, None, None, None) == 6


def test_q8_graph_of_device_position_decode_replays_across_tokens(mode):
    """One capture of a Q8_0 layer's device-position decode (the int8-MFMA score kernel, GQA
    group 3) replayed for 8 consecutive tokens: q/k/v and the position are uploaded between
    replays, outside the graph (uploadXAndUpdateParams before cuGraphLaunch in the
    reference); every replay against the oracle, the cache after the last one bit-exact."""
    c = hfp.ModelConfig(24, 8, 128, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    max_seq, p0, steps = 2048, 1500, 8
    rng = np.random.default_rng(95)
    d0 = dc.make_layer_q8(c, max_seq, p0, seed=96, mode=mode[1])
    cache = (d0.kq.copy(), d0.ks.copy(), d0.vq.copy(), d0.vs.copy())
    with _open(c, max_seq, mode) as fp:
        fp.kv.write_q8(0, 0, *cache)
        out = hfp.DeviceBuffer(c.q_dim * 4)
        g = C.c_uint64()
        _lib.call("llmp_graph_begin", 0)
        _lib.call("llmp_attn_decode_devpos", fp.kv.handle, 0, fp.gpuTokenParams.ptr,
                  fp.gpuQ.ptr, fp.gpuK.ptr, fp.gpuV.ptr, out.ptr, 0, 0)
        _lib.call("llmp_graph_end", 0, C.byref(g))
        try:
            for i in range(steps):
                pos = p0 + i
                q = rng.standard_normal(c.q_dim, dtype=np.float32)
                k = rng.standard_normal(c.kv_dim, dtype=np.float32)
                v = rng.standard_normal(c.kv_dim, dtype=np.float32)
                fp.uploadQKV(q, k, v)
                fp.updateTokenParams(pos)
                dc.log(f"[gpu] Q8 graph replay at position {pos}, mode {mode[0]}")
                _lib.call("llmp_graph_launch", g.value, 0)
                fp.sync()
                d = dc.LayerDataQ8(*cache, q, k, v, None)
                want, cache = dc.oracle_call_q8(c, max_seq, d, 0, pos, mode=mode[1])
                dc.compare_out(out.download(np.float32, c.q_dim), want, f"Q8 graph replay pos {pos}")
        finally:
            _lib.call("llmp_graph_destroy", g.value)
            out.free()
        dc.compare_cache_q8(fp, 0, cache, "Q8 cache after graph replays")
