"""HIP-graph replay of the multi-token attention (llmp_attn_prefill, llmp_attn_prefill_f32): a
call captured once and replayed gives, on every replay, the eager call's output and cache bit
for bit.  The inputs stay fixed, so every replay recomputes the same appends and attention;
the output buffer is cleared before each replay, and an eager call with its own check runs
between the replays.  Cases: a C5 prompt of 512 tokens (bf16 inputs; tile images), C3
speculative verification of 16 tokens after 4000 rows (fp32 inputs; split-K partials and
their combine), and the same verification over a Q8_0 cache."""
import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from tests import decode_cases as dc

pytestmark = pytest.mark.gpu
F32 = np.float32


def _check_replays(fp, fn, out, n_out, n_rows, q8, what):
    import ctypes as C
    fn()
    _lib.call("llmp_stream_sync", 0)
    want = out.download(np.float32, n_out)

    def cache():
        if q8:
            kq, ks, vq, vs = fp.kv.read_q8(0, 0, n_rows)
            return [kq.view(np.uint8), ks.view(np.uint32), vq.view(np.uint8), vs.view(np.uint32)]
        k, v = fp.kv.read(0, 0, n_rows)
        return [k.view(np.uint32), v.view(np.uint32)]
    want_cache = cache()
    zeros = np.zeros(n_out, np.float32)
    g = C.c_uint64()
    _lib.call("llmp_graph_begin", 0)
    fn()
    _lib.call("llmp_graph_end", 0, C.byref(g))
    try:
        for rep in range(1, 5):
            dc.log(f"[gpu] {what}: replay {rep}")
            out.upload(zeros)
            _lib.call("llmp_graph_launch", g.value, 0)
            _lib.call("llmp_stream_sync", 0)
            got = out.download(np.float32, n_out)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{what}: replay {rep} output"
            assert all(np.array_equal(a, b) for a, b in zip(cache(), want_cache)), f"{what}: replay {rep} cache"
            out.upload(zeros)
            fn()   # eager work between the replays
            _lib.call("llmp_stream_sync", 0)
            got = out.download(np.float32, n_out)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{what}: eager call {rep}"
    finally:
        _lib.call("llmp_graph_destroy", g.value)


def test_prefill_bf16_graph_replays():
    c = hfp.ModelConfig(32, 8, 64, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    P = 512
    rng = np.random.default_rng(61)
    with hfp.HipForwardPass(c, P) as fp:
        arrs = [hfp.to_bf16(rng.standard_normal((P, n), dtype=np.float32)) for n in (c.q_dim, c.kv_dim, c.kv_dim)]
        bufs = []
        try:
            for a in arrs:
                b = hfp.DeviceBuffer(a.nbytes)
                b.upload(a)
                bufs.append(b)
            out = hfp.DeviceBuffer(P * c.q_dim * 4)
            bufs.append(out)
            h = fp.kv.handle
            fn = lambda: _lib.call("llmp_attn_prefill", h, 0, 0, P, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr,
                                   out.ptr, 0)
            _check_replays(fp, fn, out, P * c.q_dim, P, False, "C5 prefill P=512")
        finally:
            for b in bufs:
                b.free()


@pytest.mark.parametrize("q8", [False, True], ids=["f32_cache", "q8_0_cache"])
def test_verification_graph_replays(q8):
    c = hfp.ModelConfig(24, 8, 128, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    K, rows = 16, 4000
    max_seq = rows + K
    rng = np.random.default_rng(62)
    with hfp.HipForwardPass(c, max_seq, kv_dtype=_lib.LLMP_KV_Q8_0 if q8 else _lib.LLMP_KV_F32) as fp:
        if q8:
            fp.kv.write_q8(0, 0, rng.integers(-127, 128, (rows, c.kv_dim), dtype=np.int8),
                           np.full((rows, c.kv_dim // 32), 1.2 / 127, np.float32),
                           rng.integers(-127, 128, (rows, c.kv_dim), dtype=np.int8),
                           np.full((rows, c.kv_dim // 32), 2.4 / 127, np.float32))
        else:
            fp.kv.write(0, 0, rng.standard_normal((rows, c.kv_dim), dtype=np.float32) * F32(0.5),
                        rng.standard_normal((rows, c.kv_dim), dtype=np.float32))
        arrs = [rng.standard_normal((K, n), dtype=np.float32) for n in (c.q_dim, c.kv_dim, c.kv_dim)]
        bufs = []
        try:
            for a in arrs:
                b = hfp.DeviceBuffer(a.nbytes)
                b.upload(a)
                bufs.append(b)
            out = hfp.DeviceBuffer(K * c.q_dim * 4)
            bufs.append(out)
            h = fp.kv.handle
            fn = lambda: _lib.call("llmp_attn_prefill_f32", h, 0, rows, K, bufs[0].ptr, bufs[1].ptr,
                                   bufs[2].ptr, 0, out.ptr, 0)
            _check_replays(fp, fn, out, K * c.q_dim, rows + K, q8,
                           f"C3 verification of 16 tokens ({'Q8_0' if q8 else 'fp32'} cache)")
        finally:
            for b in bufs:
                b.free()
