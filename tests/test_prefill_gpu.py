"""GPU parity of the prefill attention path (llmp_attn_prefill, MFMA) against the CPU oracle.

The reference has no batched prefill (the prompt is P sequential single-token forwards,
InferenceEngine.java:374-381), so the oracle is P sequential decode calls
(orc.prefill_sequential) on the fp32 widenings of the bf16 inputs.  Bar: output max-abs
<= 1e-4 (and <= 1e-4 + 1e-3*|ref|); cache rows bit-identical after the prefill and after the
decode steps that follow it."""
import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from oracle import oracle as orc
from tests import decode_cases as dc

pytestmark = pytest.mark.gpu


def _bf16_inputs(rng, P, qd, kvd, k_scale=1.0):
    q = hfp.to_bf16(rng.standard_normal((P, qd), dtype=np.float32))
    k = hfp.to_bf16(rng.standard_normal((P, kvd), dtype=np.float32) * np.float32(k_scale))
    v = hfp.to_bf16(rng.standard_normal((P, kvd), dtype=np.float32))
    return q, k, v


def _oracle_prefill(c, max_seq, layer, pos0, kc, vc, q16, k16, v16, qk=None):
    oc = dc.oracle_config(c, max_seq)
    cs, sn = dc.oracle_tables(c, max_seq, layer)
    qw, kw = qk if qk is not None else (None, None)
    return orc.prefill_sequential(oc, kc, vc, hfp.from_bf16(q16), hfp.from_bf16(k16),
                                  hfp.from_bf16(v16), layer, pos0, qnorm_w=qw, knorm_w=kw,
                                  rope_cos=cs, rope_sin=sn, n_threads=16)


def _run_prefill_case(c, max_seq, layer, pos0, P, seed, qk=None, k_scale=1.0, decode_steps=0,
                      what="prefill"):
    rng = np.random.default_rng(seed)
    kv = c.kv_dim
    kc = np.zeros((max_seq, kv), np.float32)
    vc = np.zeros((max_seq, kv), np.float32)
    kc[:pos0] = rng.standard_normal((pos0, kv), dtype=np.float32) * np.float32(k_scale)
    vc[:pos0] = rng.standard_normal((pos0, kv), dtype=np.float32)
    q16, k16, v16 = _bf16_inputs(rng, P, c.q_dim, kv, k_scale)
    qk_list = None
    if qk is not None:
        qk_list = [qk] * c.block_count
    with hfp.HipForwardPass(c, max_seq, qk_norm=qk_list) as fp:
        fp.kv.write(layer, 0, kc, vc)
        dc.log(f"[gpu] {what}: layer={layer} pos0={pos0} P={P}")
        got = fp.prefill(layer, pos0, q16, k16, v16)
        want = _oracle_prefill(c, max_seq, layer, pos0, kc, vc, q16, k16, v16, qk)
        err = dc.compare_out(got.reshape(-1), want.reshape(-1), what)
        dc.compare_cache(fp, layer, kc, vc, what + " cache", rows=(0, pos0 + P))
        dc.log(f"[gpu] {what}: ok, max abs err {err:.2e}")
        for s in range(decode_steps):
            pos = pos0 + P + s
            d = dc.LayerData(kc, vc, rng.standard_normal(c.q_dim, dtype=np.float32),
                             rng.standard_normal(kv, dtype=np.float32),
                             rng.standard_normal(kv, dtype=np.float32), qk)
            st = hfp.InferenceState.create(c)
            st.q[:], st.k[:], st.v[:] = d.q, d.k, d.v
            fp.forwardAttentionOnly(st, layer, pos)
            out, kc, vc = dc.oracle_call(c, max_seq, d, layer, pos, n_threads=16)
            dc.compare_out(st.xb2, out, f"{what}: decode step {s} after prefill")
        if decode_steps:
            dc.compare_cache(fp, layer, kc, vc, what + " cache after decode",
                             rows=(0, pos0 + P + decode_steps))
            dc.log(f"[gpu] {what}: {decode_steps} decode steps after prefill ok")


# ----------------------------------------------------------- C5: Llama-3.2-1B prefill (MFMA)
@pytest.mark.parametrize("P", [512, 2048])
def test_c5_llama1b_prefill_then_128_decode_steps(P):
    c = hfp.ModelConfig(32, 8, 64, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    _run_prefill_case(c, P + 128, 0, 0, P, seed=500 + P, decode_steps=128,
                      what=f"C5 prefill P={P}")


# Long prompts in one round of workgroups: C5 at P = 1024 (16-token query blocks), P = 1100
# (a ragged last block), 2048 after a 300-row prefix, and GQA group 2 at 2048.
@pytest.mark.parametrize("hq,pos0,P", [(32, 0, 1024), (32, 0, 1100), (32, 300, 2048), (16, 0, 2048)])
def test_prefill_long_prompts(hq, pos0, P):
    c = hfp.ModelConfig(hq, 8, 64, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    _run_prefill_case(c, pos0 + P + 4, 0, pos0, P, seed=900 + P + pos0, decode_steps=2,
                      what=f"long prefill {hq}/8/64 pos0={pos0} P={P}")


SHAPES = [(8, 8, 64), (16, 8, 64), (24, 8, 64), (32, 8, 64), (48, 8, 64), (64, 8, 64),
          (8, 8, 128), (16, 8, 128), (24, 8, 128), (32, 8, 128), (48, 8, 128), (64, 8, 128),
          (4, 4, 256), (8, 4, 256), (12, 4, 256), (16, 4, 256), (24, 4, 256), (32, 4, 256),
          (4, 1, 256)]


@pytest.mark.parametrize("hq,hkv,dim", SHAPES, ids=[f"{a}-{b}-{c}" for a, b, c in SHAPES])
def test_prefill_every_group_and_head_dim_with_prefix_and_qknorm(hq, hkv, dim):
    c = hfp.ModelConfig(hq, hkv, dim, 1, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6,
                        norm_eps=1e-6)
    rng = np.random.default_rng(hq * 100 + dim)
    qk = (rng.uniform(0.5, 1.5, dim).astype(np.float32), rng.uniform(0.5, 1.5, dim).astype(np.float32))
    _run_prefill_case(c, 400, 0, 37, 101, seed=hq + hkv + dim, qk=qk,
                      what=f"prefill shape {hq}/{hkv}/{dim}")


@pytest.mark.parametrize("P", [1, 2, 15, 16, 17, 63, 64, 65])
def test_prefill_ragged_lengths(P):
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    _run_prefill_case(c, 256, 0, 100, P, seed=P, k_scale=0.5, decode_steps=2,
                      what=f"ragged prefill P={P}")


def test_prefill_gemma3_window_local_and_global():
    c = hfp.ModelConfig(4, 1, 256, 6, architecture=hfp.ARCH_GEMMA3, rope_freq_base=1e6,
                        norm_eps=1e-6, sliding_window=64)
    rng = np.random.default_rng(3)
    qk = (rng.uniform(0.5, 1.5, 256).astype(np.float32), rng.uniform(0.5, 1.5, 256).astype(np.float32))
    for layer in (0, 5):
        _run_prefill_case(c, 512, layer, 30, 200, seed=40 + layer, qk=qk, decode_steps=3,
                          what=f"gemma3 window prefill layer {layer}")


def test_prefill_softcap_custom_scale_nope():
    c = hfp.ModelConfig(16, 4, 128, 4, architecture=hfp.ARCH_GEMMA2, rope_freq_base=1e4,
                        attn_logit_soft_cap=50.0, attention_scale=0.125, sliding_window=90,
                        no_rope_layer_interval=4)
    for layer in (0, 1, 3):
        _run_prefill_case(c, 300, layer, 20, 150, seed=60 + layer, k_scale=3.0,
                          what=f"gemma2-like prefill layer {layer}")


def test_prefill_error_codes():
    c = hfp.ModelConfig(8, 2, 64, 1, rope_freq_base=1e4)
    with hfp.HipForwardPass(c, 64) as fp:
        h = fp.kv.handle
        b = fp.gpuXb2.ptr
        assert _lib.status("llmp_attn_prefill", h, 0, 60, 8, b, b, b, b, 0) == 2   # past max_seq
        assert _lib.status("llmp_attn_prefill", h, 0, 0, 0, b, b, b, b, 0) == 2    # no tokens
        assert _lib.status("llmp_attn_prefill", h, 1, 0, 4, b, b, b, b, 0) == 2    # bad layer
        assert _lib.status("llmp_attn_prefill", h, 0, 0, 4, b, b, b, b + 4, 0) == 1  # misaligned out


# ------------------------------------- short chunks after a long prefix (split-K over key tiles)
@pytest.mark.parametrize("P", [1, 4, 8, 16])
def test_speculative_verification_shape_c3(P):
    """K draft tokens verified in one call after a 4000-token prefix (LLMEngine.java:1019-1033
    runs them as K sequential forwards); the launch splits the prefix's key tiles."""
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    _run_prefill_case(c, 4000 + P + 2, 0, 4000, P, seed=900 + P, k_scale=0.5, decode_steps=2,
                      what=f"spec-verify C3 P={P} after 4000")


def test_chunked_prefill_after_long_prefix_c5():
    c = hfp.ModelConfig(32, 8, 64, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    _run_prefill_case(c, 8200, 0, 8000, 100, seed=901, decode_steps=1,
                      what="C5 shape: 100 tokens after 8000")


def test_chunk_after_prefix_with_window_and_qknorm():
    c = hfp.ModelConfig(4, 1, 256, 6, architecture=hfp.ARCH_GEMMA3, rope_freq_base=1e6,
                        norm_eps=1e-6, sliding_window=512)
    rng = np.random.default_rng(902)
    qk = (rng.uniform(0.5, 1.5, 256).astype(np.float32), rng.uniform(0.5, 1.5, 256).astype(np.float32))
    for layer in (0, 5):   # local (window 512) and global
        _run_prefill_case(c, 3100, layer, 3000, 64, seed=903 + layer, qk=qk, decode_steps=1,
                          what=f"gemma3 chunk after 3000, layer {layer}")
