"""Randomised GPU parity sweep of prefill (llmp_attn_prefill) against the CPU oracle's P
sequential decode calls.

Each case draws, from a fixed seed:
- an architecture: Llama; Qwen3 with QK-norm; Gemma 3 with window, local/global layers and
  QK-norm; Gemma 2-like with soft-cap, custom scale, window and NoPE layers;
- a GQA group, a KV head count, a head dim, a cached prefix length pos0 and a chunk length P;
- a KV cache type: fp32, or Q8_0 under either JVM contract.

Short chunks after long prefixes take the split-K path with direct staging; long chunks take
the tile-image path.  The bar is that of the other prefill tests: output within 1e-4 (and
1e-4 + 1e-3*|ref|) of the oracle, and the cache rows bit-identical after the chunk
(InferenceEngine.prefill, InferenceEngine.java:374-381)."""
import numpy as np
import pytest

from llmplayer_amd import _lib
from oracle import oracle as orc
from tests.test_decode_random_gpu import _config
from tests.test_prefill_gpu import _run_prefill_case
from tests.test_prefill_q8_gpu import _run_q8_prefill

pytestmark = pytest.mark.gpu

ARCHS = ("llama", "qwen3", "gemma3", "gemma2")
KV_TYPES = (None, (_lib.LLMP_KV_Q8_0, orc.Q8_SCALAR), (_lib.LLMP_KV_Q8_0_TRUNC, orc.Q8_SIMD8))


def _draw(rng):
    arch = ARCHS[int(rng.integers(len(ARCHS)))]
    group = int(rng.choice([1, 2, 3, 4, 6, 8]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    dim = int(rng.choice([64, 128, 256]))
    pos0 = int(rng.choice([0, int(rng.integers(1, 1000))]))
    P = int(rng.choice([int(rng.integers(1, 17)), int(rng.integers(17, 200))]))
    kv = int(rng.integers(len(KV_TYPES)))
    layer = int(rng.integers(0, 6))
    return arch, group * hkv, hkv, dim, pos0, P, kv, layer


CASES = [_draw(np.random.default_rng(77000 + i)) for i in range(24)]


@pytest.mark.parametrize("case", CASES, ids=[f"{a}-{hq}/{hkv}/{d}-p{p}-P{n}-kv{k}-l{l}"
                                             for a, hq, hkv, d, p, n, k, l in CASES])
def test_prefill_random_case(case):
    arch, hq, hkv, dim, pos0, P, kv, layer = case
    c = _config(arch, hq, hkv, dim)
    qk = None
    if arch in ("qwen3", "gemma3"):
        rng = np.random.default_rng(hq * 131 + dim)
        qk = (rng.uniform(0.5, 1.5, dim).astype(np.float32),
              rng.uniform(0.5, 1.5, dim).astype(np.float32))
    max_seq = pos0 + P + 8
    what = f"random prefill {arch} {hq}/{hkv}/{dim} pos0 {pos0} P {P} kv {kv} layer {layer}"
    seed = 9000 + hq * 31 + dim + pos0 + P
    if KV_TYPES[kv] is None:
        _run_prefill_case(c, max_seq, layer, pos0, P, seed, qk=qk, k_scale=0.5, what=what)
    else:
        _run_q8_prefill(c, max_seq, layer, pos0, P, seed, KV_TYPES[kv], qk=qk, k_scale=0.5,
                        what=what)
