"""GPU parity of multi-token attention on fp32 projections (llmp_attn_prefill_f32) against the
CPU oracle, with no bf16 step anywhere.

The reference runs a prompt, and every speculative verification, as sequential fp32 forwards
(InferenceEngine.java:374-381, LLMEngine.java:1019-1033): each token's fp32 k/v row is
normalised, rotated and stored (Attention.java:284-367, KVCache.java:164-179) before the next
token attends.  The oracle is exactly that (orc.prefill_sequential / prefill_sequential_q8 on
the same fp32 arrays the GPU receives).

Bar: output max-abs <= 1e-4 (and <= 1e-4 + 1e-3*|ref|); every cache row bit-identical to the
oracle's after the multi-token call and after the decode steps that follow it."""
import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from oracle import oracle as orc
from tests import decode_cases as dc

pytestmark = pytest.mark.gpu


def _f32_inputs(rng, P, qd, kvd, k_scale=1.0):
    q = rng.standard_normal((P, qd), dtype=np.float32)
    k = rng.standard_normal((P, kvd), dtype=np.float32) * np.float32(k_scale)
    v = rng.standard_normal((P, kvd), dtype=np.float32)
    return q, k, v


def _decode_steps_f32(fp, c, max_seq, layer, kc, vc, pos, steps, qk, rng, what):
    for s in range(steps):
        d = dc.LayerData(kc, vc, rng.standard_normal(c.q_dim, dtype=np.float32),
                         rng.standard_normal(c.kv_dim, dtype=np.float32),
                         rng.standard_normal(c.kv_dim, dtype=np.float32), qk)
        st = hfp.InferenceState.create(c)
        st.q[:], st.k[:], st.v[:] = d.q, d.k, d.v
        fp.forwardAttentionOnly(st, layer, pos + s)
        out, kc, vc = dc.oracle_call(c, max_seq, d, layer, pos + s, n_threads=16)
        dc.compare_out(st.xb2, out, f"{what}: decode step {s}")
    return kc, vc


def run_f32_case(c, max_seq, layer, pos0, P, seed, qk=None, k_scale=1.0, decode_steps=0,
                 what="f32 prefill"):
    rng = np.random.default_rng(seed)
    kvd = c.kv_dim
    kc = np.zeros((max_seq, kvd), np.float32)
    vc = np.zeros((max_seq, kvd), np.float32)
    kc[:pos0] = rng.standard_normal((pos0, kvd), dtype=np.float32) * np.float32(k_scale)
    vc[:pos0] = rng.standard_normal((pos0, kvd), dtype=np.float32)
    q, k, v = _f32_inputs(rng, P, c.q_dim, kvd, k_scale)
    qk_list = [qk] * c.block_count if qk is not None else None
    with hfp.HipForwardPass(c, max_seq, qk_norm=qk_list) as fp:
        fp.kv.write(layer, 0, kc, vc)
        dc.log(f"[gpu] {what}: fp32 inputs, layer={layer} pos0={pos0} P={P}")
        got = fp.prefill(layer, pos0, q, k, v)
        oc = dc.oracle_config(c, max_seq)
        cs, sn = dc.oracle_tables(c, max_seq, layer)
        qw, kw = qk if qk is not None else (None, None)
        want = orc.prefill_sequential(oc, kc, vc, q, k, v, layer, pos0, qnorm_w=qw, knorm_w=kw,
                                      rope_cos=cs, rope_sin=sn, n_threads=16)
        err = dc.compare_out(got.reshape(-1), want.reshape(-1), what)
        dc.compare_cache(fp, layer, kc, vc, what + " cache", rows=(0, pos0 + P))
        dc.log(f"[gpu] {what}: ok, max abs err {err:.2e}")
        if decode_steps:
            kc, vc = _decode_steps_f32(fp, c, max_seq, layer, kc, vc, pos0 + P, decode_steps,
                                       qk, rng, what)
            dc.compare_cache(fp, layer, kc, vc, what + " cache after decode",
                             rows=(0, pos0 + P + decode_steps))
            dc.log(f"[gpu] {what}: {decode_steps} decode steps after it ok")
    return err


# ------------------------------------------- C5 shape (Llama-3.2-1B) as a prompt of fp32 rows
@pytest.mark.parametrize("P", [512, 2048])
def test_c5_shape_f32_prompt_then_128_decode_steps(P):
    c = hfp.ModelConfig(32, 8, 64, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    run_f32_case(c, P + 128, 0, 0, P, seed=1500 + P, decode_steps=128,
                 what=f"C5 shape fp32 P={P}")


# --------------------------- C3 speculative verification: K fp32 draft rows after 4000 rows
@pytest.mark.parametrize("K", [1, 4, 8, 16])
def test_c3_verification_f32_then_128_decode_steps(K):
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    run_f32_case(c, 4000 + K + 128, 0, 4000, K, seed=1900 + K, k_scale=0.5, decode_steps=128,
                 what=f"C3 verify fp32 K={K} after 4000")


SHAPES = [(32, 8, 64), (24, 8, 128), (16, 8, 128), (64, 8, 128), (8, 4, 256), (4, 1, 256)]


@pytest.mark.parametrize("hq,hkv,dim", SHAPES, ids=[f"{a}-{b}-{c}" for a, b, c in SHAPES])
def test_f32_prompt_qknorm_neox_with_prefix(hq, hkv, dim):
    c = hfp.ModelConfig(hq, hkv, dim, 1, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6,
                        norm_eps=1e-6)
    rng = np.random.default_rng(hq * 10 + dim)
    qk = (rng.uniform(0.5, 1.5, dim).astype(np.float32), rng.uniform(0.5, 1.5, dim).astype(np.float32))
    run_f32_case(c, 400, 0, 37, 101, seed=2000 + hq + dim, qk=qk, decode_steps=2,
                 what=f"fp32 prompt {hq}/{hkv}/{dim} qk-norm neox")


def test_f32_gemma3_window_local_and_global():
    c = hfp.ModelConfig(4, 1, 256, 6, architecture=hfp.ARCH_GEMMA3, rope_freq_base=1e6,
                        norm_eps=1e-6, sliding_window=64)
    rng = np.random.default_rng(2100)
    qk = (rng.uniform(0.5, 1.5, 256).astype(np.float32), rng.uniform(0.5, 1.5, 256).astype(np.float32))
    for layer in (0, 5):
        run_f32_case(c, 512, layer, 30, 200, seed=2101 + layer, qk=qk, decode_steps=3,
                     what=f"fp32 gemma3 window layer {layer}")


@pytest.mark.parametrize("P", [1, 17, 64, 65])
def test_f32_ragged_lengths(P):
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    run_f32_case(c, 256, 0, 100, P, seed=2200 + P, k_scale=0.5, decode_steps=1,
                 what=f"fp32 ragged P={P}")


def test_f32_prompt_matches_decode_calls_bit_for_bit_in_the_cache():
    """The rows a fp32 multi-token call appends equal those of P llmp_attn_decode calls on the
    same inputs, read back from two caches of the library itself."""
    c = hfp.ModelConfig(16, 8, 128, 1, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6,
                        norm_eps=1e-6)
    rng = np.random.default_rng(2300)
    qk = (rng.uniform(0.5, 1.5, 128).astype(np.float32), rng.uniform(0.5, 1.5, 128).astype(np.float32))
    P = 40
    q, k, v = _f32_inputs(rng, P, c.q_dim, c.kv_dim)
    with hfp.HipForwardPass(c, 64, qk_norm=[qk]) as a, hfp.HipForwardPass(c, 64, qk_norm=[qk]) as b:
        a.prefill(0, 0, q, k, v)
        for i in range(P):
            st = hfp.InferenceState.create(c)
            st.q[:], st.k[:], st.v[:] = q[i], k[i], v[i]
            b.forwardAttentionOnly(st, 0, i)
        ka, va = a.kv.read(0, 0, P)
        kb, vb = b.kv.read(0, 0, P)
        assert np.array_equal(ka.view(np.uint32), kb.view(np.uint32))
        assert np.array_equal(va.view(np.uint32), vb.view(np.uint32))


# ------------------------------------------------------------------ Q8_0 cache, fp32 inputs
Q8_MODES = [(_lib.LLMP_KV_Q8_0, orc.Q8_SCALAR), (_lib.LLMP_KV_Q8_0_TRUNC, orc.Q8_SIMD8)]


@pytest.mark.parametrize("mode", Q8_MODES, ids=["round", "trunc"])
@pytest.mark.parametrize("pos0,P", [(0, 512), (4000, 16)], ids=["prompt512", "verify16"])
def test_f32_inputs_over_q8_cache(mode, pos0, P):
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    max_seq = pos0 + P + 4
    rng = np.random.default_rng(2400 + pos0 + P)
    kvd = c.kv_dim
    kf = np.zeros((max_seq, kvd), np.float32)
    vf = np.zeros((max_seq, kvd), np.float32)
    kf[:pos0] = rng.standard_normal((pos0, kvd), dtype=np.float32) * np.float32(0.5)
    vf[:pos0] = rng.standard_normal((pos0, kvd), dtype=np.float32)
    kq, ks = dc.quantize_rows(kf, mode[1])
    vq, vs = dc.quantize_rows(vf, mode[1])
    kq[pos0:] = 0; ks[pos0:] = 0; vq[pos0:] = 0; vs[pos0:] = 0
    q, k, v = _f32_inputs(rng, P, c.q_dim, kvd, 0.5)
    what = f"fp32 inputs over Q8_0 ({mode[0]}) pos0={pos0} P={P}"
    with hfp.HipForwardPass(c, max_seq, kv_dtype=mode[0]) as fp:
        fp.kv.write_q8(0, 0, kq, ks, vq, vs)
        dc.log(f"[gpu] {what}")
        got = fp.prefill(0, pos0, q, k, v)
        oc = dc.oracle_config(c, max_seq)
        cs, sn = dc.oracle_tables(c, max_seq, 0)
        want = orc.prefill_sequential_q8(oc, kq, ks, vq, vs, q, k, v, 0, pos0, rope_cos=cs,
                                         rope_sin=sn, n_threads=16, mode=mode[1])
        err = dc.compare_out(got.reshape(-1), want.reshape(-1), what)
        dc.compare_cache_q8(fp, 0, (kq, ks, vq, vs), what + " cache")
        dc.log(f"[gpu] {what}: ok, max abs err {err:.2e}")


def test_f32_entry_point_errors():
    c = hfp.ModelConfig(8, 2, 64, 1, rope_freq_base=1e4)
    with hfp.HipForwardPass(c, 64) as fp:
        h = fp.kv.handle
        b = fp.gpuXb2.ptr
        assert _lib.status("llmp_attn_prefill_f32", h, 0, 0, 4, b + 2, b, b, 0, b, 0) == 1  # q 2 B
        assert _lib.status("llmp_attn_prefill_f32", h, 0, 60, 8, b, b, b, 0, b, 0) == 2     # rows
        with pytest.raises(TypeError):
            fp.prefill(0, 0, np.zeros((2, c.q_dim), np.float64), np.zeros((2, c.kv_dim), np.float64),
                       np.zeros((2, c.kv_dim), np.float64))
        with pytest.raises(TypeError):
            fp.prefill(0, 0, np.zeros((2, c.q_dim), np.float32), hfp.to_bf16(np.zeros((2, c.kv_dim))),
                       np.zeros((2, c.kv_dim), np.float32))


@pytest.mark.parametrize("arch,rope_dim", [(hfp.ARCH_QWEN3, 32), (hfp.ARCH_QWEN3, 64),
                                           (hfp.ARCH_LLAMA, 64)],
                         ids=["neox32", "neox64", "normal64"])
def test_f32_prompt_partial_rope(arch, rope_dim):
    """Partial RoPE (rotated dims < head_dim, ModelConfig.ropeDimensionCount) in the append and
    in the query fragments: NEOX pairs (i, i + R/2) cross lanes of the MFMA layout."""
    c = hfp.ModelConfig(16, 8, 128, 1, architecture=arch, rope_freq_base=1e6, norm_eps=1e-6,
                        rope_dim_count=rope_dim)
    rng = np.random.default_rng(2500 + rope_dim)
    qk = (rng.uniform(0.5, 1.5, 128).astype(np.float32), rng.uniform(0.5, 1.5, 128).astype(np.float32))
    run_f32_case(c, 300, 0, 20, 90, seed=2510 + rope_dim, qk=qk, decode_steps=2,
                 what=f"fp32 partial rope {arch} R={rope_dim}")
