"""Randomised GPU parity sweep of decode attention against the CPU oracle.

Each case draws, from a fixed seed (so every run checks the same cases):
- an architecture: Llama (NORMAL RoPE), Qwen3 (NEOX RoPE, QK-norm), Gemma 3 (sliding window,
  local and global layers, QK-norm), Gemma 2-like (soft-cap, custom scale, window, NoPE
  layers);
- a GQA group, a KV head count, a head dim, a position, a split count;
- a KV cache type: fp32, or Q8_0 under either JVM contract.

The combinations cross the kernel paths: the fp32 split kernel, the int8-MFMA score kernel for
Q8_0 groups up to 4, the VALU Q8_0 kernel for groups of 6 and 8, the register and LDS query
prologues, and partial tiles and short splits.  The bar is the one of the other decode tests:
output within 1e-4 (and 1e-4 + 1e-3*|ref|) of the oracle, and the appended row bit-identical
(KVCache.storeK/storeV, Attention.java:284-367)."""
import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from oracle import oracle as orc
from tests import decode_cases as dc

pytestmark = pytest.mark.gpu

MAX_SEQ = 1536
ARCHS = ("llama", "qwen3", "gemma3", "gemma2")
KV_TYPES = ((_lib.LLMP_KV_F32, None), (_lib.LLMP_KV_Q8_0, orc.Q8_SCALAR),
            (_lib.LLMP_KV_Q8_0_TRUNC, orc.Q8_SIMD8))


def _draw(rng):
    arch = ARCHS[int(rng.integers(len(ARCHS)))]
    group = int(rng.choice([1, 2, 3, 4, 6, 8]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    dim = int(rng.choice([64, 128, 256]))
    pos = int(rng.integers(0, MAX_SEQ))
    splits = int(rng.choice([0, 1, int(rng.integers(2, 200))]))
    kv = int(rng.integers(len(KV_TYPES)))
    layer = int(rng.integers(0, 6))
    return arch, group * hkv, hkv, dim, pos, splits, kv, layer


CASES = [_draw(np.random.default_rng(20261202 + i)) for i in range(36)]


def _config(arch, hq, hkv, dim):
    if arch == "llama":
        return hfp.ModelConfig(hq, hkv, dim, 6, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    if arch == "qwen3":
        return hfp.ModelConfig(hq, hkv, dim, 6, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6,
                               norm_eps=1e-6)
    if arch == "gemma3":
        return hfp.ModelConfig(hq, hkv, dim, 6, architecture=hfp.ARCH_GEMMA3, rope_freq_base=1e6,
                               norm_eps=1e-6, sliding_window=512)
    return hfp.ModelConfig(hq, hkv, dim, 6, architecture=hfp.ARCH_GEMMA2, rope_freq_base=1e4,
                           attn_logit_soft_cap=50.0, attention_scale=0.125, sliding_window=300,
                           no_rope_layer_interval=4)


@pytest.mark.parametrize("case", CASES, ids=[f"{a}-{hq}/{hkv}/{d}-p{p}-s{s}-kv{k}-l{l}"
                                             for a, hq, hkv, d, p, s, k, l in CASES])
def test_decode_random_case(case):
    arch, hq, hkv, dim, pos, splits, kv, layer = case
    c = _config(arch, hq, hkv, dim)
    qk = arch in ("qwen3", "gemma3")
    kv_dtype, q8_mode = KV_TYPES[kv]
    what = f"random {arch} {hq}/{hkv}/{dim} pos {pos} splits {splits} kv {kv_dtype} layer {layer}"
    dc.log(f"[gpu] {what}")
    seed = 5000 + hq * 97 + dim + pos
    if q8_mode is None:
        d = dc.make_layer(c, MAX_SEQ, pos, seed=seed, k_scale=0.5, qk_norm=qk)
    else:
        d = dc.make_layer_q8(c, MAX_SEQ, pos, seed=seed, k_scale=0.5, qk_norm=qk, mode=q8_mode)
    with hfp.HipForwardPass(c, MAX_SEQ, qk_norm=[d.qk_norm] * 6, kv_dtype=kv_dtype) as fp:
        st = hfp.InferenceState.create(c)
        st.q[:], st.k[:], st.v[:] = d.q, d.k, d.v
        if q8_mode is None:
            fp.kv.write(layer, 0, d.kc, d.vc)
            fp.forwardAttentionOnly(st, layer, pos, splits)
            out, kc, vc = dc.oracle_call(c, MAX_SEQ, d, layer, pos)
            dc.compare_out(st.xb2, out, what)
            dc.compare_cache(fp, layer, kc, vc, what, rows=(pos, pos + 1))
        else:
            fp.kv.write_q8(layer, 0, d.kq, d.ks, d.vq, d.vs)
            fp.forwardAttentionOnly(st, layer, pos, splits)
            out, cache = dc.oracle_call_q8(c, MAX_SEQ, d, layer, pos, mode=q8_mode)
            dc.compare_out(st.xb2, out, what)
            dc.compare_cache_q8(fp, layer, cache, what, rows=(pos, pos + 1))
    dc.log(f"[gpu] {what}: ok")
