"""Randomised GPU parity sweep of the attention half of a layer (llmp_attn_block and
llmp_attn_block_batch) against the oracle's block (orc.attn_block).

Each case draws, from a fixed seed (so every run checks the same cases):
- the projection formats: one of the 18 GGUF types for q, k, v and o, or a K-quant mix
  (Q4_K_M, Q3_K_L, Q5_K_M);
- a head shape: GQA group 1-8 or 16 over 1-4 KV heads, head_dim 64 or 128, and an embedding
  width of 1024-3072;
- the architecture features: q/k/v/o biases, pre-norm or none, post-norm, merged QKV (one
  format), Granite's residual scale, per-head QK-norm (Qwen3, NEOX RoPE);
- the call: single-token steps after a cached prefix or one K-token call of 1-20 tokens, on
  the fp32 or the Q8_1 input.

The combinations cross the projection kernels' format pairs and round counts, the input
modes and the token-batched path with the decode and multi-token attention kernels.  The bars
are those of test_block_gpu.py (single-token calls) and test_block_batch_gpu.py (K-token
calls)."""
import zlib

import numpy as np
import pytest

from llmplayer_amd import hip_forward_pass as hfp
from tests import ggml_pack as gp
from tests import test_block_batch_gpu as tbb
from tests import test_block_gpu as tbg

pytestmark = pytest.mark.gpu

MIXES = {"q4_k_m": (gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K),
         "q3_k_l": (gp.GGML_Q3_K, gp.GGML_Q3_K, gp.GGML_Q5_K, gp.GGML_Q5_K),
         "q5_k_m": (gp.GGML_Q5_K, gp.GGML_Q5_K, gp.GGML_Q6_K, gp.GGML_Q5_K)}


def _draw(rng):
    if rng.random() < 0.25:
        mix = list(MIXES)[int(rng.integers(len(MIXES)))]
        types, tname = MIXES[mix], mix
    else:
        t = tbg.TYPES[int(rng.integers(len(tbg.TYPES)))]
        types, tname = (t,) * 4, tbg.NAMES[t]
    superblock = any(t in (gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q3_K, gp.GGML_Q5_K, gp.GGML_IQ4_XS,
                           gp.GGML_Q2_K, gp.GGML_IQ3_XXS, gp.GGML_IQ3_S, gp.GGML_IQ2_S) for t in types)
    while True:   # super-block formats need q_dim (the output projection's width) in whole 256s
        hkv = int(rng.choice([1, 2, 4]))
        group = int(rng.choice([1, 2, 3, 4, 5, 8, 16]))
        if group == 16:
            hkv = min(hkv, 2)
        d = int(rng.choice([64, 128]))
        if not superblock or (hkv * group * d) % 256 == 0:
            break
    dim = int(rng.choice([1024, 2048, 3072]))
    flags = {
        "bias": bool(rng.random() < 0.3),
        "post": bool(rng.random() < 0.25),
        "pre": bool(rng.random() < 0.9),
        "merged": bool(len(set(types)) == 1 and rng.random() < 0.25),
        "rscale": 0.3 if rng.random() < 0.2 else 0.0,
        "qk": bool(rng.random() < 0.3),
    }
    batched = bool(rng.random() < 0.4)
    q8 = bool(rng.random() < 0.35)
    pos0 = int(rng.integers(0, 300))
    k = int(rng.integers(1, 21))
    return types, tname, hkv * group, hkv, d, dim, flags, batched, q8, pos0, k


CASES = [_draw(np.random.default_rng(20261203 + i)) for i in range(28)]


def _id(case):
    types, tname, hq, hkv, d, dim, flags, batched, q8, pos0, k = case
    on = "".join(c for c, f in (("b", flags["bias"]), ("p", flags["post"]), ("n", flags["pre"]),
                                ("m", flags["merged"]), ("r", flags["rscale"] > 0), ("q", flags["qk"])) if f)
    call = (f"batch{k}" if batched else "tok") + ("-q8_1" if q8 else "")
    return f"{tname}-{hq}/{hkv}/{d}-dim{dim}-{on or 'none'}-{call}-p{pos0}"


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_block_random(case):
    types, tname, hq, hkv, d, dim, flags, batched, q8, pos0, k = case
    seed = zlib.crc32(_id(case).encode())
    qk = None
    if flags["qk"]:
        c = hfp.ModelConfig(hq, hkv, d, 1, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6,
                            norm_eps=1e-6)
        rng = np.random.default_rng(seed)
        qk = (rng.uniform(0.5, 1.5, d).astype(np.float32), rng.uniform(0.5, 1.5, d).astype(np.float32))
    else:
        c = hfp.ModelConfig(hq, hkv, d, 1, architecture=hfp.ARCH_LLAMA, rope_freq_base=500000.0)
    common = dict(merged=flags["merged"], bias=flags["bias"], post=flags["post"], pre=flags["pre"],
                  rscale=flags["rscale"], qk=qk)
    if batched:
        tbb._run_batch(c, dim, pos0 + k + 8, pos0, k, types, seed=seed, what=_id(case), q8=q8, **common)
    else:
        tbg._run(c, dim, pos0 + 10, pos0, 2, types, seed=seed, what=_id(case), q8=q8, **common)
