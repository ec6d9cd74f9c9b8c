"""GPU parity of the attention variants on the same kernels, against the CPU oracle:

- GPT-OSS attention sinks (Qwen3MoEInferenceEngine.java:295-313, softmaxWithSink :562-575),
  with the engine's alternating window (even layers windowed, :280-286) and a YaRN-style
  custom scale; decode (fp32 and Q8_0 caches, host and device positions) and prefill.
- Qwen3.5 attention output gate (Qwen35InferenceEngine.java:580-583): out *= sigmoid(gate);
  decode and prefill.

Bar: output max-abs <= 1e-4 (and <= 1e-4 + 1e-3*|ref|); cache rows bit-identical."""
import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from oracle import oracle as orc
from tests import decode_cases as dc

pytestmark = pytest.mark.gpu


def _gptoss(max_layers=2, window=128):
    # GPT-OSS-20B attention: 64 query heads, 8 KV heads, head_dim 64, window 128 (ISWA).
    return hfp.ModelConfig(64, 8, 64, max_layers, architecture=hfp.ARCH_GPT_OSS,
                           rope_freq_base=150000.0, sliding_window=window, expert_count=32,
                           attention_scale=float(np.float32(1.3 * 1.3 / 8.0)))


def _sinks(c, seed):
    return [np.random.default_rng(seed + l).uniform(-1.0, 3.0, c.head_count).astype(np.float32)
            for l in range(c.block_count)]


@pytest.mark.parametrize("pos", [0, 100, 127, 128, 129, 1000, 4095])
@pytest.mark.parametrize("splits", [0, 1, 7])
def test_gptoss_sinks_decode_both_window_kinds(pos, splits):
    c = _gptoss()
    sinks = _sinks(c, 10)
    with hfp.HipForwardPass(c, 4096, sinks=sinks) as fp:
        for layer in (0, 1):
            d = dc.make_layer(c, 4096, pos, seed=1000 * layer + pos)
            dc.log(f"[gpu] gpt-oss sinks decode layer {layer} pos {pos} splits {splits}")
            fp.kv.write(layer, 0, d.kc, d.vc)
            st = hfp.InferenceState.create(c)
            st.q[:], st.k[:], st.v[:] = d.q, d.k, d.v
            fp.forwardAttentionOnly(st, layer, pos, splits)
            want, kc, vc = dc.oracle_call(c, 4096, d, layer, pos, n_threads=16, sinks=sinks[layer])
            dc.compare_out(st.xb2, want, f"gpt-oss sinks layer {layer} pos {pos}")
            dc.compare_cache(fp, layer, kc, vc, "gpt-oss sinks cache", rows=(0, pos + 1))


@pytest.mark.parametrize("pos", [5, 300, 3000])
def test_gptoss_yarn_tables_and_mscale_scale(pos):
    """GPT-OSS with its YaRN RoPE (factor 32 over a 4096-token original context) as the MoE
    engine builds it: the host mirror makes the tables with llmp_rope_table_yarn and sets the
    layer scale to mscale^2/sqrt(headSize) (Qwen3MoEInferenceEngine.java:60-66, 277-279); the
    oracle builds its own (orc_rope_tables_yarn)."""
    c = hfp.ModelConfig(64, 8, 64, 2, architecture=hfp.ARCH_GPT_OSS, rope_freq_base=150000.0,
                        sliding_window=128, expert_count=32, rope_scaling_factor=32.0,
                        rope_orig_context_length=4096, yarn_log_multiplier=0.0)
    sinks = _sinks(c, 40)
    with hfp.HipForwardPass(c, 4096, sinks=sinks) as fp:
        assert abs(float(fp.mscale) - (1.0 + 0.1 * np.log(32.0))) < 2e-6
        for layer in (0, 1):
            d = dc.make_layer(c, 4096, pos, seed=400 + layer + pos)
            dc.log(f"[gpu] gpt-oss yarn decode layer {layer} pos {pos}")
            fp.kv.write(layer, 0, d.kc, d.vc)
            st = hfp.InferenceState.create(c)
            st.q[:], st.k[:], st.v[:] = d.q, d.k, d.v
            fp.forwardAttentionOnly(st, layer, pos)
            want, kc, vc = dc.oracle_call(c, 4096, d, layer, pos, n_threads=16, sinks=sinks[layer])
            dc.compare_out(st.xb2, want, f"gpt-oss yarn layer {layer} pos {pos}")
            dc.compare_cache(fp, layer, kc, vc, "gpt-oss yarn cache", rows=(0, pos + 1))


def test_sinks_can_be_removed_and_q8_cache_and_device_position():
    c = _gptoss(window=0)
    sinks = _sinks(c, 20)
    pos = 2000
    for mode in (_lib.LLMP_KV_Q8_0, _lib.LLMP_KV_Q8_0_TRUNC):
        omode = orc.Q8_SCALAR if mode == _lib.LLMP_KV_Q8_0 else orc.Q8_SIMD8
        d = dc.make_layer_q8(c, 2048, pos, seed=21, mode=omode)
        with hfp.HipForwardPass(c, 2048, sinks=sinks, kv_dtype=mode) as fp:
            for use_sinks in (True, False):
                if not use_sinks:
                    fp.set_sinks(0, None)
                fp.kv.write_q8(0, 0, d.kq, d.ks, d.vq, d.vs)
                fp.uploadQKV(d.q, d.k, d.v)
                fp.updateTokenParams(pos)
                dc.log(f"[gpu] Q8 mode {mode} sinks={use_sinks} device position {pos}")
                fp.forwardAttentionPartDevicePosition(0)
                want, cache = dc.oracle_call_q8(c, 2048, d, 0, pos, n_threads=16, mode=omode,
                                                sinks=sinks[0] if use_sinks else None)
                dc.compare_out(fp.downloadXb2(), want, f"Q8 sinks={use_sinks}")
                dc.compare_cache_q8(fp, 0, cache, "Q8 sinks cache", rows=(pos, pos + 1))


@pytest.mark.parametrize("pos0,P", [(0, 300), (200, 77), (1000, 8)])
def test_gptoss_sinks_prefill_then_decode(pos0, P):
    c = _gptoss()
    sinks = _sinks(c, 30)
    max_seq = pos0 + P + 4
    rng = np.random.default_rng(31 + pos0)
    with hfp.HipForwardPass(c, max_seq, sinks=sinks) as fp:
        for layer in (0, 1):
            kc = np.zeros((max_seq, c.kv_dim), np.float32)
            vc = np.zeros((max_seq, c.kv_dim), np.float32)
            kc[:pos0] = rng.standard_normal((pos0, c.kv_dim), dtype=np.float32)
            vc[:pos0] = rng.standard_normal((pos0, c.kv_dim), dtype=np.float32)
            q16 = hfp.to_bf16(rng.standard_normal((P, c.q_dim), dtype=np.float32))
            k16 = hfp.to_bf16(rng.standard_normal((P, c.kv_dim), dtype=np.float32))
            v16 = hfp.to_bf16(rng.standard_normal((P, c.kv_dim), dtype=np.float32))
            fp.kv.write(layer, 0, kc, vc)
            dc.log(f"[gpu] gpt-oss sinks prefill layer {layer} pos0 {pos0} P {P}")
            got = fp.prefill(layer, pos0, q16, k16, v16)
            oc = dc.oracle_config(c, max_seq, sinks[layer])
            cs, sn = dc.oracle_tables(c, max_seq, layer)
            want = orc.prefill_sequential(oc, kc, vc, hfp.from_bf16(q16), hfp.from_bf16(k16),
                                          hfp.from_bf16(v16), layer, pos0, rope_cos=cs,
                                          rope_sin=sn, n_threads=16)
            dc.compare_out(got.reshape(-1), want.reshape(-1), f"gpt-oss sinks prefill layer {layer}")
            dc.compare_cache(fp, layer, kc, vc, "gpt-oss prefill cache", rows=(0, pos0 + P))
            d = dc.LayerData(kc, vc, rng.standard_normal(c.q_dim, dtype=np.float32),
                             rng.standard_normal(c.kv_dim, dtype=np.float32),
                             rng.standard_normal(c.kv_dim, dtype=np.float32))
            st = hfp.InferenceState.create(c)
            st.q[:], st.k[:], st.v[:] = d.q, d.k, d.v
            fp.forwardAttentionOnly(st, layer, pos0 + P)
            out, _, _ = dc.oracle_call(c, max_seq, d, layer, pos0 + P, n_threads=16,
                                       sinks=sinks[layer])
            dc.compare_out(st.xb2, out, "decode after sinks prefill")


def _qwen35(rope_dim):
    # Qwen3.5 full-attention layer shape: 16 query heads, 2 KV heads, head_dim 256, QK-norm,
    # NEOX rotary on the first rope_dim dims.
    return hfp.ModelConfig(16, 2, 256, 1, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e7,
                           rope_dim_count=rope_dim, norm_eps=1e-6)


@pytest.mark.parametrize("rope_dim", [64, 256])
@pytest.mark.parametrize("splits", [0, 1, 5])
def test_qwen35_gated_decode(rope_dim, splits):
    c = _qwen35(rope_dim)
    d = dc.make_layer(c, 3000, 2500, seed=40 + rope_dim, qk_norm=True)
    gate = np.random.default_rng(41).uniform(-6, 6, c.q_dim).astype(np.float32)
    with hfp.HipForwardPass(c, 3000, qk_norm=[d.qk_norm]) as fp:
        fp.kv.write(0, 0, d.kc, d.vc)
        st = hfp.InferenceState.create(c)
        st.q[:], st.k[:], st.v[:] = d.q, d.k, d.v
        dc.log(f"[gpu] qwen3.5 gated decode rope_dim {rope_dim} splits {splits}")
        fp.forwardAttentionOnly(st, 0, 2500, splits, gate=gate)
        want, kc, vc = dc.oracle_call(c, 3000, d, 0, 2500, n_threads=16, gate=gate)
        dc.compare_out(st.xb2, want, "qwen3.5 gated decode")
        dc.compare_cache(fp, 0, kc, vc, "qwen3.5 gated cache", rows=(2500, 2501))
        # the ungated call on the same inputs is the plain attention
        fp.kv.write(0, 0, d.kc, d.vc)
        fp.forwardAttentionOnly(st, 0, 2500, splits)
        plain, _, _ = dc.oracle_call(c, 3000, d, 0, 2500, n_threads=16)
        dc.compare_out(st.xb2, plain, "qwen3.5 ungated decode")


def test_qwen35_gated_prefill_and_sinks_together():
    c = _qwen35(256)
    rng = np.random.default_rng(50)
    max_seq, pos0, P = 512, 64, 200
    qk = (rng.uniform(0.5, 1.5, 256).astype(np.float32), rng.uniform(0.5, 1.5, 256).astype(np.float32))
    sinks = rng.uniform(-1, 2, c.head_count).astype(np.float32)
    kc = np.zeros((max_seq, c.kv_dim), np.float32)
    vc = np.zeros((max_seq, c.kv_dim), np.float32)
    kc[:pos0] = rng.standard_normal((pos0, c.kv_dim), dtype=np.float32)
    vc[:pos0] = rng.standard_normal((pos0, c.kv_dim), dtype=np.float32)
    q16 = hfp.to_bf16(rng.standard_normal((P, c.q_dim), dtype=np.float32))
    k16 = hfp.to_bf16(rng.standard_normal((P, c.kv_dim), dtype=np.float32))
    v16 = hfp.to_bf16(rng.standard_normal((P, c.kv_dim), dtype=np.float32))
    gate = rng.uniform(-5, 5, (P, c.q_dim)).astype(np.float32)
    with hfp.HipForwardPass(c, max_seq, qk_norm=[qk], sinks=[sinks]) as fp:
        fp.kv.write(0, 0, kc, vc)
        dc.log("[gpu] qwen3.5 gated prefill with sinks")
        got = fp.prefill(0, pos0, q16, k16, v16, gate=gate)
        oc = dc.oracle_config(c, max_seq, sinks)
        cs, sn = dc.oracle_tables(c, max_seq, 0)
        want = orc.prefill_sequential(oc, kc, vc, hfp.from_bf16(q16), hfp.from_bf16(k16),
                                      hfp.from_bf16(v16), 0, pos0, qnorm_w=qk[0], knorm_w=qk[1],
                                      rope_cos=cs, rope_sin=sn, n_threads=16, gate=gate)
        dc.compare_out(got.reshape(-1), want.reshape(-1), "gated prefill with sinks")
        dc.compare_cache(fp, 0, kc, vc, "gated prefill cache", rows=(0, pos0 + P))


def test_variant_entry_point_errors():
    c = _gptoss()
    with hfp.HipForwardPass(c, 64) as fp:
        h = fp.kv.handle
        bad = np.array([1.0] * 63 + [np.inf], np.float32)
        assert _lib.status("llmp_layer_sinks", h, 0, bad.ctypes.data_as(_lib.C.POINTER(_lib.C.c_float))) == 1
        assert _lib.status("llmp_layer_sinks", h, 5, None) == 2
        b = fp.gpuXb2.ptr
        assert _lib.status("llmp_attn_decode_ex", h, 0, 3, 0, b, b, b, b + 2, b, 0, 0) == 1
        assert _lib.status("llmp_attn_decode_ex", h, 0, 3, b + 2, b, b, b, 0, b, 0, 0) == 1
