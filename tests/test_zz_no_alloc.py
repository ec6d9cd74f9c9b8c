"""GPU check of llmp_attn_prefill_f32_static, the multi-token entry point that allocates nothing
(its workspace is the library's static device array): on the same inputs its outputs and
cache rows are bit-identical to llmp_attn_prefill_f32's, for two calls in a row on one
handle pair, the second with a smaller input (and another workspace use: split-K partials
instead of key-tile images).  A call whose workspace would not fit is refused."""
import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from tests import decode_cases as dc

pytestmark = pytest.mark.gpu


def _call(entry, fp, layer, pos0, q, k, v):
    c = fp.config
    P = q.shape[0]
    bufs = [hfp.DeviceBuffer(a.nbytes) for a in (q, k, v)] + [hfp.DeviceBuffer(P * c.q_dim * 4)]
    try:
        for b, a in zip(bufs, (q, k, v)):
            b.upload(a)
        _lib.call(entry, fp.kv.handle, layer, pos0, P, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, 0,
                  bufs[3].ptr, 0)
        return bufs[3].download(np.float32, P * c.q_dim).reshape(P, c.q_dim)
    finally:
        for b in bufs:
            b.free()


def _same(a, b, what):
    if not np.array_equal(a.view(np.uint32), b.view(np.uint32)):
        bad = np.argwhere(a != b)
        raise AssertionError(f"{what}: {len(bad)} values differ, first {bad[:3].tolist()}")


def test_static_prefill_matches_the_allocating_entry_point_twice():
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    max_seq = 4200
    rng = np.random.default_rng(77)
    with hfp.HipForwardPass(c, max_seq) as ref, hfp.HipForwardPass(c, max_seq) as st:
        # Call 1: a 2048-token prompt from position 0 (key-tile images in the scratch).
        P1 = 2048
        q = rng.standard_normal((P1, c.q_dim), dtype=np.float32)
        k = rng.standard_normal((P1, c.kv_dim), dtype=np.float32) * np.float32(0.5)
        v = rng.standard_normal((P1, c.kv_dim), dtype=np.float32)
        dc.log("[gpu] no-alloc prefill: call 1, 2048 tokens at position 0")
        want = _call("llmp_attn_prefill_f32", ref, 0, 0, q, k, v)
        got = _call("llmp_attn_prefill_f32_static", st, 0, 0, q, k, v)
        _same(got, want, "call 1 output")
        # Rows up to 4000 for the second call's prefix (the same rows in both caches).
        fill_k = rng.standard_normal((4000 - P1, c.kv_dim), dtype=np.float32) * np.float32(0.5)
        fill_v = rng.standard_normal((4000 - P1, c.kv_dim), dtype=np.float32)
        for fp in (ref, st):
            fp.kv.write(0, P1, fill_k, fill_v)
        # Call 2: 16 draft tokens after 4000 rows (split-K partials in the scratch).
        P2 = 16
        q2 = rng.standard_normal((P2, c.q_dim), dtype=np.float32)
        k2 = rng.standard_normal((P2, c.kv_dim), dtype=np.float32) * np.float32(0.5)
        v2 = rng.standard_normal((P2, c.kv_dim), dtype=np.float32)
        dc.log("[gpu] no-alloc prefill: call 2, 16 tokens at position 4000")
        want2 = _call("llmp_attn_prefill_f32", ref, 0, 4000, q2, k2, v2)
        got2 = _call("llmp_attn_prefill_f32_static", st, 0, 4000, q2, k2, v2)
        _same(got2, want2, "call 2 output")
        ka, va = ref.kv.read(0, 0, 4000 + P2)
        kb, vb = st.kv.read(0, 0, 4000 + P2)
        _same(kb, ka, "K cache")
        _same(vb, va, "V cache")
        dc.log("[gpu] no-alloc prefill: both calls bit-identical to llmp_attn_prefill_f32")


def test_static_prefill_refuses_a_workspace_beyond_the_array():
    # 4096 tokens at 8 KV heads x head_dim 128 need 64 key tiles x 8 heads x 69,632 B = 35.7 MB
    # of images, more than the 32 MiB array; the call fails before any launch.
    c = hfp.ModelConfig(8, 8, 128, 1, rope_freq_base=500000.0)
    with hfp.HipForwardPass(c, 4096) as fp:
        b = hfp.DeviceBuffer(4096 * c.q_dim * 4)
        try:
            rc = _lib.status("llmp_attn_prefill_f32_static", fp.kv.handle, 0, 0, 4096, b.ptr,
                             b.ptr, b.ptr, 0, b.ptr, 0)
            assert rc == 1, rc
            assert "static scratch" in _lib.last_error()
        finally:
            b.free()
