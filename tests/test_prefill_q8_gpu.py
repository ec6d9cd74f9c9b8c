"""GPU parity of prefill attention over a Q8_0 KV cache against the CPU oracle.

The reference's prefill is P sequential single-token forwards (InferenceEngine.java:374-381);
over a Q8_0 cache each token's K/V rows are quantised as it appends them (KVCache.storeK /
storeV, KVCache.java:164-179, 218-243) and later tokens attend to the quantised rows
(dotQ8 / saxpyQ8, KVCache.java:244-282).  The oracle (orc.prefill_sequential_q8) runs exactly
that under either JVM contract (rounding LLMP_KV_Q8_0, or the truncating 8-lane SIMD one,
LLMP_KV_Q8_0_TRUNC).

Bar: output max-abs <= 1e-4 (and <= 1e-4 + 1e-3*|ref|); appended quants and scales, and every
other row, bit-identical to the oracle's, after the prefill and after decode steps that follow."""
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


def _run_q8_prefill(c, max_seq, layer, pos0, P, seed, mode, qk=None, k_scale=1.0,
                    decode_steps=0, what="Q8 prefill"):
    rng = np.random.default_rng(seed)
    kv = c.kv_dim
    kf = np.zeros((max_seq, kv), np.float32)
    vf = np.zeros((max_seq, kv), np.float32)
    kf[:pos0] = rng.standard_normal((pos0, kv), dtype=np.float32) * np.float32(k_scale)
    vf[:pos0] = rng.standard_normal((pos0, kv), dtype=np.float32)
    kq, ks = dc.quantize_rows(kf, mode[1])
    vq, vs = dc.quantize_rows(vf, mode[1])
    kq[pos0:] = 0; ks[pos0:] = 0; vq[pos0:] = 0; vs[pos0:] = 0
    q16 = hfp.to_bf16(rng.standard_normal((P, c.q_dim), dtype=np.float32))
    k16 = hfp.to_bf16(rng.standard_normal((P, kv), dtype=np.float32) * np.float32(k_scale))
    v16 = hfp.to_bf16(rng.standard_normal((P, kv), dtype=np.float32))
    qk_list = [qk] * c.block_count if qk is not None else None
    with hfp.HipForwardPass(c, max_seq, qk_norm=qk_list, kv_dtype=mode[0]) as fp:
        fp.kv.write_q8(layer, 0, kq, ks, vq, vs)
        dc.log(f"[gpu] {what}: mode={mode[0]} layer={layer} pos0={pos0} P={P}")
        got = fp.prefill(layer, pos0, q16, k16, v16)
        oc = dc.oracle_config(c, max_seq)
        cs, sn = dc.oracle_tables(c, max_seq, layer)
        qw, kw = qk if qk is not None else (None, None)
        want = orc.prefill_sequential_q8(oc, kq, ks, vq, vs, hfp.from_bf16(q16),
                                         hfp.from_bf16(k16), hfp.from_bf16(v16), layer, pos0,
                                         qnorm_w=qw, knorm_w=kw, rope_cos=cs, rope_sin=sn,
                                         n_threads=16, mode=mode[1])
        err = dc.compare_out(got.reshape(-1), want.reshape(-1), what)
        dc.compare_cache_q8(fp, layer, (kq, ks, vq, vs), what + " cache")
        dc.log(f"[gpu] {what}: ok, max abs err {err:.2e}")
        cache = (kq, ks, vq, vs)
        for s in range(decode_steps):
            pos = pos0 + P + s
            d = dc.LayerDataQ8(*cache, rng.standard_normal(c.q_dim, dtype=np.float32),
                               rng.standard_normal(kv, dtype=np.float32),
                               rng.standard_normal(kv, dtype=np.float32), qk)
            st = hfp.InferenceState.create(c)
            st.q[:], st.k[:], st.v[:] = d.q, d.k, d.v
            fp.forwardAttentionOnly(st, layer, pos)
            out, cache = dc.oracle_call_q8(c, max_seq, d, layer, pos, n_threads=16, mode=mode[1])
            dc.compare_out(st.xb2, out, f"{what}: decode step {s} after prefill")
        if decode_steps:
            dc.compare_cache_q8(fp, layer, cache, what + " cache after decode")
            dc.log(f"[gpu] {what}: {decode_steps} decode steps after prefill ok")


@pytest.mark.parametrize("P", [512, 2048])
def test_q8_c5_llama1b_prefill_then_decode(P, mode):
    c = hfp.ModelConfig(32, 8, 64, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    _run_q8_prefill(c, P + 16, 0, 0, P, seed=700 + P, mode=mode, decode_steps=16,
                    what=f"Q8 C5 prefill P={P}")


SHAPES = [(32, 8, 64), (24, 8, 128), (16, 4, 256), (4, 1, 256)]


@pytest.mark.parametrize("hq,hkv,dim", SHAPES, ids=[f"{a}-{b}-{c}" for a, b, c in SHAPES])
def test_q8_prefill_head_dims_with_prefix_and_qknorm(hq, hkv, dim, mode):
    c = hfp.ModelConfig(hq, hkv, dim, 1, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6,
                        norm_eps=1e-6)
    rng = np.random.default_rng(hq * 10 + dim)
    qk = (rng.uniform(0.5, 1.5, dim).astype(np.float32), rng.uniform(0.5, 1.5, dim).astype(np.float32))
    _run_q8_prefill(c, 400, 0, 37, 101, seed=hq + dim, mode=mode, qk=qk,
                    what=f"Q8 prefill shape {hq}/{hkv}/{dim}")


@pytest.mark.parametrize("P", [1, 17, 65])
def test_q8_prefill_ragged_lengths(P, mode):
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    _run_q8_prefill(c, 256, 0, 100, P, seed=80 + P, mode=mode, k_scale=0.5, decode_steps=2,
                    what=f"Q8 ragged prefill P={P}")


def test_q8_prefill_gemma3_window_local_and_global(mode):
    c = hfp.ModelConfig(4, 1, 256, 6, architecture=hfp.ARCH_GEMMA3, rope_freq_base=1e6,
                        norm_eps=1e-6, sliding_window=64)
    rng = np.random.default_rng(5)
    qk = (rng.uniform(0.5, 1.5, 256).astype(np.float32), rng.uniform(0.5, 1.5, 256).astype(np.float32))
    for layer in (0, 5):
        _run_q8_prefill(c, 512, layer, 30, 200, seed=90 + layer, mode=mode, qk=qk,
                        decode_steps=2, what=f"Q8 gemma3 window prefill layer {layer}")


@pytest.mark.parametrize("P", [4, 16])
def test_q8_speculative_verification_after_long_prefix(P, mode):
    """Short chunks after a 4000-token prefix split the key tiles and stage straight from the
    Q8_0 cache (no tile images)."""
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    _run_q8_prefill(c, 4000 + P + 2, 0, 4000, P, seed=950 + P, mode=mode, k_scale=0.5,
                    decode_steps=2, what=f"Q8 spec-verify C3 P={P} after 4000")
