"""HIP-graph replay of the attention half of a layer (llmp_attn_block, llmp_attn_block_batch).

A call captured once (llmp_graph_begin / llmp_graph_end) and replayed must leave, on every
replay, the state that the same call made eagerly on a twin handle leaves: the residual rows
and the cache rows bit for bit (the same kernels on the same inputs).  The single-token block
reads its position from device memory (the reference's graph mode: CudaForwardPass.java:
1760-1812, tokenParams updated between replays), so its replays step through positions; the
K-token call (fp32 or Q8_1 input) repeats at a fixed position, its residual rows changing
from replay to replay.
Eager calls run between the replays, and every replay is checked."""
import ctypes as C

import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from tests import decode_cases as dc
from tests import ggml_pack as gp
from tests import test_block_gpu as tbg

pytestmark = pytest.mark.gpu
F32 = np.float32


def _twins(c, dim, max_seq, pos0, types, seed, K, q8=False):
    """Two handles with the same cache prefix, weights and residual rows (q8: the Q8_1 input
    mode)."""
    rng = np.random.default_rng(seed)
    lw, _ = tbg._weights(c, dim, types, rng, bias=True)
    kc = rng.standard_normal((pos0, c.kv_dim)).astype(F32)
    vc = rng.standard_normal((pos0, c.kv_dim)).astype(F32)
    x = (rng.standard_normal((K, dim)) * 2).astype(F32)
    fps = []
    for _ in range(2):
        fp = hfp.HipForwardPass(c, max_seq)
        fp.kv.write(0, 0, kc, vc)
        fp.setBlockConfig(dim, 0.0, _lib.LLMP_INPUT_Q8_1 if q8 else _lib.LLMP_INPUT_F32)
        fp.uploadLayerWeights(0, lw)
        fps.append(fp)
    return fps, x


def _same(fa, fb, a, b, n_rows, what):
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{what}: residual rows differ"
    ka, va = fa.kv.read(0, 0, n_rows)
    kb, vb = fb.kv.read(0, 0, n_rows)
    assert np.array_equal(ka.view(np.uint32), kb.view(np.uint32)), f"{what}: K rows differ"
    assert np.array_equal(va.view(np.uint32), vb.view(np.uint32)), f"{what}: V rows differ"


@pytest.mark.parametrize("types", [(gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K),
                                   (gp.GGML_IQ3_S,) * 4], ids=["q4_k_m", "iq3_s"])
def test_block_graph_at_device_positions_matches_eager_calls(types):
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    pos0 = 200
    (graphed, eager), x = _twins(c, 1024, 256, pos0, types, 41, 1)
    try:
        for fp in (graphed, eager):
            fp.uploadX(x[0])
            fp.updateTokenParams(pos0)
            fp.forwardAttentionBlock(0, pos0, device_position=True)   # sizes every workspace
        _lib.call("llmp_stream_sync", 0)
        g = C.c_uint64()
        _lib.call("llmp_graph_begin", 0)
        graphed.forwardAttentionBlock(0, pos0, device_position=True)
        _lib.call("llmp_graph_end", 0, C.byref(g))
        try:
            for rep in range(1, 6):
                pos = pos0 + rep
                dc.log(f"[gpu] block graph {types[0]}: replay {rep} at position {pos}")
                graphed.updateTokenParams(pos)
                _lib.call("llmp_graph_launch", g.value, 0)
                _lib.call("llmp_stream_sync", 0)
                eager.updateTokenParams(pos)   # the same launch plan (planned for max_seq - 1)
                eager.forwardAttentionBlock(0, pos, device_position=True)
                _lib.call("llmp_stream_sync", 0)
                _same(graphed, eager, graphed.downloadX(), eager.downloadX(), pos + 1, f"replay {rep}")
        finally:
            _lib.call("llmp_graph_destroy", g.value)
    finally:
        graphed.close()
        eager.close()


@pytest.mark.parametrize("types,K,q8", [((gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K), 8, False),
                                        ((gp.GGML_Q2_K,) * 4, 16, False), ((gp.GGML_F32,) * 4, 20, False),
                                        ((gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K), 16, True)],
                         ids=["q4_k_m-8", "q2_k-16", "f32-20", "q4_k_m-16-q8_1"])
def test_block_batch_graph_matches_eager_calls(types, K, q8):
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    pos0 = 150
    (graphed, eager), x = _twins(c, 1024, 256, pos0, types, 43, K, q8)
    try:
        for fp in (graphed, eager):
            fp.uploadXBatch(x)
            fp.forwardAttentionBlockBatch(0, pos0, K)   # sizes every workspace
        _lib.call("llmp_stream_sync", 0)
        g = C.c_uint64()
        _lib.call("llmp_graph_begin", 0)
        graphed.forwardAttentionBlockBatch(0, pos0, K)
        _lib.call("llmp_graph_end", 0, C.byref(g))
        try:
            for rep in range(1, 5):
                dc.log(f"[gpu] block batch graph {types[0]} K={K}: replay {rep}")
                _lib.call("llmp_graph_launch", g.value, 0)
                _lib.call("llmp_stream_sync", 0)
                eager.forwardAttentionBlockBatch(0, pos0, K)
                _lib.call("llmp_stream_sync", 0)
                _same(graphed, eager, graphed.downloadXBatch(K), eager.downloadXBatch(K), pos0 + K,
                      f"replay {rep}")
        finally:
            _lib.call("llmp_graph_destroy", g.value)
    finally:
        graphed.close()
        eager.close()
