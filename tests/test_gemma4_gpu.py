"""GPU parity of the Gemma 4 attention half (Gemma4InferenceEngine.forwardLayer steps 2-4,
Gemma4InferenceEngine.java:295-420) against the CPU oracle (orc.forward_gemma4).

Covered: 256-dim sliding-window layers and 512-dim full-attention layers (RoPE frequency
factors), QK-norm and the weightless V-norm in RMSNorm.apply's sequential order (appended K/V
rows bit-identical), attention scale 1.0, and shared-KV layers that attend to an earlier
layer's cache without appending (kvSourceLayer, :171-180), by decode and by prefill.

Bar: output max-abs <= 1e-4 (and <= 1e-4 + 1e-3*|ref|); cache rows bit-identical."""
import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from oracle import oracle as orc
from tests import decode_cases as dc

pytestmark = pytest.mark.gpu

HQ, HKV, D_SWA, D_FULL, EPS = 8, 2, 256, 512, 1e-6


def _config(L, pattern, shared, window, max_factors=True):
    ff = np.linspace(1.0, 6.0, D_FULL // 2).astype(np.float32) if max_factors else None
    return hfp.ModelConfig(HQ, HKV, D_SWA, L, architecture=hfp.ARCH_GEMMA4,
                           rope_freq_base=1e6, rope_freq_base_swa=1e4, norm_eps=EPS,
                           sliding_window=window, sliding_window_pattern=pattern,
                           key_length=D_FULL, shared_kv_layers=shared, rope_freq_factors=ff)


class _OracleModel:
    """The reference's per-layer float caches and Gemma 4 attention, one layer-call at a time."""

    def __init__(self, c, max_seq, fp):
        self.c, self.max_seq, self.fp = c, max_seq, fp
        self.cache = {}
        for layer in range(c.block_count):
            if fp.hasOwnKv(layer):
                D = fp.head_size(fp.isSwaLayer(layer))
                self.cache[layer] = (np.zeros((max_seq, HKV * D), np.float32),
                                     np.zeros((max_seq, HKV * D), np.float32))
        self.tables = {}
        for t in (True, False):
            D = fp.head_size(t)
            theta = c.rope_freq_base_swa if t else c.rope_freq_base
            self.tables[t] = orc.rope_tables(D, max_seq, theta,
                                             freq_factors=None if t else c.rope_freq_factors)

    def call(self, layer, pos, q, k, v, qk, n_threads=16):
        t = self.fp.isSwaLayer(layer)
        D = self.fp.head_size(t)
        cfg = orc.OracleConfig(HQ, HKV, D, self.max_seq, rope_type=0, norm_eps=EPS,
                               sliding_window=self.c.sliding_window)
        kc, vc = self.cache[self.fp.kvSourceLayer(layer)]
        cs, sn = self.tables[t]
        own = self.fp.hasOwnKv(layer)
        out, _, _, _ = orc.forward_gemma4(cfg, kc, vc, q, k if own else None, v if own else None,
                                          pos, t, qnorm_w=qk[0], knorm_w=qk[1], rope_cos=cs,
                                          rope_sin=sn, n_threads=n_threads)
        return out


def _make_qk(c, L, rng):
    pat = c.sliding_window_pattern
    ws = []
    for layer in range(L):
        D = D_SWA if pat[layer] else D_FULL
        ws.append((rng.uniform(0.5, 1.5, D).astype(np.float32),
                   rng.uniform(0.05, 0.3, D).astype(np.float32)))   # Gemma 4 K-norm ~0.13
    return ws


def _compare_own_cache(fp, om, layer, rows):
    kv, slot = fp.kv_cache(layer)
    k, v = kv.read(slot, 0, rows)
    wk, wv = om.cache[layer]
    for name, g, w in (("K", k, wk[:rows]), ("V", v, wv[:rows])):
        if not np.array_equal(g.view(np.uint32), w.view(np.uint32)):
            bad = np.argwhere(g != w)
            raise AssertionError(f"gemma4 layer {layer} {name} cache differs at {len(bad)} "
                                 f"elements, first {tuple(bad[0])}: {g[tuple(bad[0])]!r} vs "
                                 f"{w[tuple(bad[0])]!r}")


@pytest.mark.parametrize("splits", [0, 1, 5, 64])
def test_gemma4_swa_and_full_layer_decode_after_a_prefix(splits):
    """One 256-dim window layer and one 512-dim full layer at position 300 over a random
    prefix: output parity and the appended rows (QK-norm, V-norm, RoPE) bit for bit."""
    L, S, pos = 2, 320, 300
    c = _config(L, [True, False], 0, 64)
    rng = np.random.default_rng(400 + splits)
    qk = _make_qk(c, L, rng)
    with hfp.Gemma4HipForwardPass(c, S, qk_norm=qk) as fp:
        om = _OracleModel(c, S, fp)
        for layer in range(L):
            kc, vc = om.cache[layer]
            kc[:pos] = rng.standard_normal(kc[:pos].shape, dtype=np.float32) * np.float32(0.3)
            vc[:pos] = rng.standard_normal(vc[:pos].shape, dtype=np.float32)
            kv, slot = fp.kv_cache(layer)
            kv.write(slot, 0, kc, vc)
        st = fp.createState()
        for layer in range(L):
            D = fp.head_size(fp.isSwaLayer(layer))
            q = rng.standard_normal(HQ * D, dtype=np.float32) * np.float32(3)
            k = rng.standard_normal(HKV * D, dtype=np.float32) * np.float32(3)
            v = rng.standard_normal(HKV * D, dtype=np.float32) * np.float32(3)
            st.q[:q.size], st.k[:k.size], st.v[:v.size] = q, k, v
            dc.log(f"[gpu] gemma4 layer {layer} (D={D}) decode at {pos}, splits={splits}")
            fp.forwardAttentionOnly(st, layer, pos, splits)
            want = om.call(layer, pos, q, k, v, qk[layer])
            err = dc.compare_out(st.xb2[:HQ * D], want, f"gemma4 layer {layer} D={D}")
            _compare_own_cache(fp, om, layer, S)
            dc.log(f"[gpu] gemma4 layer {layer}: ok, max abs err {err:.2e}")


def test_gemma4_model_decode_with_shared_kv_layers():
    """8 layers (SWA x4, full, then shared SWA x2 and shared full): 40 tokens decoded one
    layer-call at a time, every output against the oracle, caches compared at the end."""
    L, S, T, W = 8, 64, 40, 16
    pattern = [True, True, True, True, False, True, True, False]
    c = _config(L, pattern, 3, W)
    rng = np.random.default_rng(410)
    qk = _make_qk(c, L, rng)
    with hfp.Gemma4HipForwardPass(c, S, qk_norm=qk) as fp:
        assert [fp.kvSourceLayer(l) for l in range(L)] == [0, 1, 2, 3, 4, 3, 3, 4]
        om = _OracleModel(c, S, fp)
        st = fp.createState()
        worst = 0.0
        for pos in range(T):
            for layer in range(L):
                D = fp.head_size(fp.isSwaLayer(layer))
                q = rng.standard_normal(HQ * D, dtype=np.float32) * np.float32(2)
                k = rng.standard_normal(HKV * D, dtype=np.float32) * np.float32(2)
                v = rng.standard_normal(HKV * D, dtype=np.float32) * np.float32(2)
                st.q[:q.size], st.k[:k.size], st.v[:v.size] = q, k, v
                fp.forwardAttentionOnly(st, layer, pos)
                want = om.call(layer, pos, q, k, v, qk[layer], n_threads=8)
                worst = max(worst, dc.compare_out(st.xb2[:HQ * D], want,
                                                  f"gemma4 model pos {pos} layer {layer}"))
        for layer in range(5):
            _compare_own_cache(fp, om, layer, T)
        dc.log(f"[gpu] gemma4 model: {T} tokens x {L} layers ok, max abs err {worst:.2e}")


def test_gemma4_prefill_own_and_shared_window_layers():
    """Prefill of an own-KV window layer (QK-norm, V-norm appended bit-exact) and of a shared
    window layer reading it, against the oracle's token-by-token loop."""
    L, S, W, pos0, P = 8, 200, 48, 30, 120
    pattern = [True, True, True, True, False, True, True, False]
    c = _config(L, pattern, 3, W)
    rng = np.random.default_rng(420)
    qk = _make_qk(c, L, rng)
    with hfp.Gemma4HipForwardPass(c, S, qk_norm=qk) as fp:
        om = _OracleModel(c, S, fp)
        kc, vc = om.cache[3]
        kc[:pos0] = rng.standard_normal(kc[:pos0].shape, dtype=np.float32) * np.float32(0.3)
        vc[:pos0] = rng.standard_normal(vc[:pos0].shape, dtype=np.float32)
        kv, slot = fp.kv_cache(3)
        kv.write(slot, 0, kc, vc)
        for layer in (3, 5):    # layer 5 is shared: source layer 3
            q16 = hfp.to_bf16(rng.standard_normal((P, HQ * D_SWA), dtype=np.float32) * np.float32(3))
            k16 = hfp.to_bf16(rng.standard_normal((P, HKV * D_SWA), dtype=np.float32) * np.float32(3))
            v16 = hfp.to_bf16(rng.standard_normal((P, HKV * D_SWA), dtype=np.float32) * np.float32(3))
            dc.log(f"[gpu] gemma4 prefill layer {layer}: pos0={pos0} P={P}")
            got = fp.prefill(layer, pos0, q16, k16, v16)
            q, k, v = hfp.from_bf16(q16), hfp.from_bf16(k16), hfp.from_bf16(v16)
            want = np.stack([om.call(layer, pos0 + i, q[i], k[i], v[i], qk[layer])
                             for i in range(P)])
            err = dc.compare_out(got.reshape(-1), want.reshape(-1), f"gemma4 prefill layer {layer}")
            _compare_own_cache(fp, om, 3, S)
            dc.log(f"[gpu] gemma4 prefill layer {layer}: ok, max abs err {err:.2e}")


def test_gemma4_full_layer_prefill_is_unsupported_and_bad_sources_rejected():
    c = _config(2, [True, False], 0, 32)
    with hfp.Gemma4HipForwardPass(c, 64) as fp:
        full = fp.kv[False]
        b = fp.gpuXb2.ptr
        # 512-dim heads: decode only (checked before any launch)
        assert _lib.status("llmp_attn_prefill", full.handle, 0, 0, 4, b, b, b, b, 0) == 6
        assert _lib.status("llmp_attn_decode_shared", full.handle, 0, 3, 5, 0, b, 0, b, 0, 0) == 2
        assert _lib.status("llmp_attn_decode_shared", full.handle, 0, -1, 5, 0, b, 0, b, 0, 0) == 2
        assert _lib.status("llmp_layer_norm_mode", full.handle, 0, 4) == 1
        assert _lib.status("llmp_layer_norm_mode", full.handle, 2, 1) == 2
