"""GPU parity of the attention half for K tokens in one call (llmp_attn_block_batch: the
projections of all K tokens on the matrix cores, the multi-token attention on fp32 projections,
the output projection and residual) against K sequential calls of the oracle's restatement of
TransformerBlock.forward / Attention.forward (orc.attn_block), the reference's per-token
forwards (LLMEngine.forwardBatch, LLMEngine.java:1019-1033).

Bar: every token's residual after the block within 1e-4 + 1e-3*|ref| elementwise of the
oracle, and max-abs <= max(1e-4, 2^-17 * max|ref|): the projections sum in another order than
the CPU path, and a reordered fp32 sum of n terms moves by ~sqrt(n)/2 units of the last place of
its partial sums, which passes 1e-4 once outputs reach ~30 (the single-token block meets the
same bar and no tighter one there); below |ref| = 13 the bar is the plain 1e-4.  Q4_K weights are
drawn centred (_centered_q4_k) so the residual stays at a real model's scale.  The K appended
K/V rows meet the standard bar; every other cache row is unchanged.  The oracle appends its own
rows as it goes, so later tokens attend to the oracle's rows, as in the reference."""
import ctypes as C

import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from oracle import oracle as orc
from tests import decode_cases as dc
from tests import ggml_pack as gp
from tests.test_block_gpu import NAMES
from tests import test_block_gpu as tbg

pytestmark = pytest.mark.gpu

F32 = np.float32


def _centered_q4_k(rows, cols, rng, scale=0.05):
    """Q4_K weights whose sub-block mins cancel their mean, as a quantiser's are (dmin = 8d,
    m = round(7.5 sc / 8): d*sc*q - dmin*m ~ d*sc*(q - 7.5)).  The shared generator draws scales
    and mins independently, which gives every weight a positive mean and residuals of ~50; with
    centred weights the residual stays at the scale of real models."""
    ns = cols // 256
    d = rng.uniform(0.5, 1.5, (rows, ns)) * scale / 256
    sc = rng.integers(16, 64, (rows, ns, 8))
    mn = np.rint(sc * 7.5 / 8).astype(np.int64)
    wb, _ = gp.pack_q4_k(gp._f16_bits(d), gp._f16_bits(d * 8), sc, mn, rng.integers(0, 16, (rows, cols)))
    return wb


def _weights(c, dim, types, rng, merged=False, bias=False, post=False, pre=True):
    """The block weights of tests.test_block_gpu, with Q4_K tensors drawn centred."""
    lw, bw = tbg._weights(c, dim, types, rng, merged, bias, post, pre)
    if not merged:
        for name, attr_t, rows, cols in (("wq", "wq_type", c.q_dim, dim), ("wk", "wk_type", c.kv_dim, dim),
                                         ("wv", "wv_type", c.kv_dim, dim), ("wo", "wo_type", dim, c.q_dim)):
            if getattr(bw, attr_t) == gp.GGML_Q4_K:
                wb = _centered_q4_k(rows, cols, rng)
                setattr(lw, name, hfp.GgufTensor(gp.GGML_Q4_K, rows, cols, wb.reshape(-1)))
                setattr(bw, name, wb)
    return lw, bw


def _compare_block(got, want, what):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = dc.ATOL + dc.RTOL * np.abs(want.astype(np.float64))
    cap = max(dc.ATOL, 2.0 ** -17 * float(np.abs(want).max()))
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert (err <= bound).all() and err.max() <= cap, (
        f"{what}: max abs err {err.max():.3e} (bar {cap:.2e}); {int((err > bound).sum())} "
        f"elements above {dc.ATOL} + {dc.RTOL}*|ref|")
    return float(err.max())


def _run_batch(c, dim, max_seq, pos0, K, types, seed, what, merged=False, bias=False,
               post=False, pre=True, rscale=0.0, qk=None, q8=False, sinks=None, layer=0,
               rounds=1, batched=False, per_token=False, single_tail=False):
    """`rounds` batched calls of K tokens each, from position pos0 on layer `layer` of c, each
    token checked against sequential orc.attn_block calls.  per_token: check that the calls ran
    one single-token decode per token.  batched: also check that the calls
    took the matrix-core path (no single-token decode launch: the profile counters)."""
    rng = np.random.default_rng(seed)
    lw, bw = _weights(c, dim, types, rng, merged, bias, post, pre)
    bw.residual_scale = rscale
    bw.q8_1_input = q8
    kv = c.kv_dim
    kc = np.zeros((max_seq, kv), F32)
    vc = np.zeros((max_seq, kv), F32)
    kc[:pos0] = rng.standard_normal((pos0, kv)).astype(F32)
    vc[:pos0] = rng.standard_normal((pos0, kv)).astype(F32)
    qk_list = [qk] * c.block_count if qk is not None else None
    oc = dc.oracle_config(c, max_seq, sinks)
    cs, sn = dc.oracle_tables(c, max_seq, layer)
    qw, kw = qk if qk is not None else (None, None)
    sink_list = [sinks] * c.block_count if sinks is not None else None
    with hfp.HipForwardPass(c, max_seq, qk_norm=qk_list, sinks=sink_list) as fp:
        fp.kv.write(layer, 0, kc, vc)
        fp.setBlockConfig(dim, rscale, _lib.LLMP_INPUT_Q8_1 if q8 else _lib.LLMP_INPUT_F32)
        fp.uploadLayerWeights(layer, lw)
        if batched or per_token or single_tail:
            _lib.call("llmp_profile_enable", fp.kv.handle, 1)
        worst = 0.0
        p0 = pos0
        for r in range(rounds):
            x = (rng.standard_normal((K, dim)) * 2).astype(F32)
            dc.log(f"[gpu] block batch {what}: round {r}, {K} tokens at pos {p0}")
            fp.uploadXBatch(x)
            fp.forwardAttentionBlockBatch(layer, p0, K)
            got = fp.downloadXBatch(K)
            want = np.empty_like(got)
            attn = []
            ok, ov = kc.copy(), vc.copy()
            for t in range(K):
                want[t], a_t = orc.attn_block(oc, bw, ok, ov, x[t], layer, p0 + t, qnorm_w=qw, knorm_w=kw,
                                              rope_cos=cs, rope_sin=sn, n_threads=16, return_attn=True)
                attn.append(a_t)
            gk, gv = fp.kv.read(layer, 0, p0 + K)
            assert np.array_equal(gk[:p0], kc[:p0]) and np.array_equal(gv[:p0], vc[:p0])
            dc.compare_out(gk[p0:p0 + K], ok[p0:p0 + K], f"block batch {what} appended K rows")
            dc.compare_out(gv[p0:p0 + K], ov[p0:p0 + K], f"block batch {what} appended V rows")
            for t in range(K):
                if q8 and orc.q8_1_routed(bw.wo_type):   # near-tie allowance of Wo's int8 input
                    worst = max(worst, tbg._compare_q8_output(got[t], want[t], attn[t], bw, rscale,
                                                              f"block batch {what} token {t}"))
                else:
                    worst = max(worst, _compare_block(got[t], want[t], f"block batch {what} token {t}"))
            # continue from the device's rows
            kc[p0:p0 + K], vc[p0:p0 + K] = gk[p0:p0 + K], gv[p0:p0 + K]
            p0 += K
        if per_token:
            n, ms = C.c_int(), C.c_double()
            _lib.call("llmp_profile_read", fp.kv.handle, _lib.LLMP_PROF_DECODE_SPLIT, C.byref(n), C.byref(ms))
            assert n.value == rounds * K, f"{what}: {n.value} single-token decode launches"
        if single_tail:   # groups of 16 batched, a last group of one token single
            n, ms = C.c_int(), C.c_double()
            _lib.call("llmp_profile_read", fp.kv.handle, _lib.LLMP_PROF_DECODE_SPLIT, C.byref(n), C.byref(ms))
            assert n.value == rounds * (K % 16 == 1), f"{what}: {n.value} single-token decode launches"
            _lib.call("llmp_profile_read", fp.kv.handle, _lib.LLMP_PROF_PREFILL_ATTN, C.byref(n), C.byref(ms))
            assert n.value >= rounds * (K // 16), f"{what}: {n.value} multi-token attention launches"
        if batched:
            n, ms = C.c_int(), C.c_double()
            _lib.call("llmp_profile_read", fp.kv.handle, _lib.LLMP_PROF_DECODE_SPLIT, C.byref(n), C.byref(ms))
            assert n.value == 0, f"{what}: {n.value} single-token decode launches"
            _lib.call("llmp_profile_read", fp.kv.handle, _lib.LLMP_PROF_PREFILL_ATTN, C.byref(n), C.byref(ms))
            assert n.value >= rounds, f"{what}: {n.value} multi-token attention launches"
        dc.log(f"[gpu] block batch {what}: ok, max abs err {worst:.2e}")


TYPES = tbg.TYPES


@pytest.mark.parametrize("t", TYPES, ids=[NAMES[t] for t in TYPES])
def test_block_batch_every_weight_format(t):
    """Each format's matrix-core path: 5 tokens (a partial token tile) after a 40-row prefix,
    then 5 more."""
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    if t in tbg.PER_TOKEN:
        _run_batch(c, 1024, 64, 40, 5, (t, t, t, t), seed=1600 + t, what=NAMES[t], rounds=2,
                   per_token=True)
        return
    _run_batch(c, 1024, 64, 40, 5, (t, t, t, t), seed=1600 + t, what=NAMES[t], rounds=2, batched=True)


@pytest.mark.parametrize("mix", ["q3_k_l", "q5_k_m"])
def test_block_batch_c3_q3_k_l_and_q5_k_m(mix):
    """The C3 shape with the Q3_K_L mix (Q3_K q, k; Q5_K v, o) and the Q5_K_M mix (Q5_K q, k, o;
    Q6_K v): their two-format launches on the matrix cores, 8 tokens after 4000 rows."""
    types = {"q3_k_l": (gp.GGML_Q3_K, gp.GGML_Q3_K, gp.GGML_Q5_K, gp.GGML_Q5_K),
             "q5_k_m": (gp.GGML_Q5_K, gp.GGML_Q5_K, gp.GGML_Q6_K, gp.GGML_Q5_K)}[mix]
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    _run_batch(c, 3072, 4096, 4000, 8, types, seed=1650 + len(mix), what=f"C3 {mix}", batched=True)


@pytest.mark.parametrize("t", [gp.GGML_IQ3_XXS, gp.GGML_IQ3_S, gp.GGML_IQ2_S, gp.GGML_Q2_K],
                         ids=["iq3_xxs", "iq3_s", "iq2_s", "q2_k"])
def test_block_batch_c3_codebook_formats_and_q2_k(t):
    """The C3 shape with q, k, v and o in a codebook format (the codebook in LDS) or Q2_K (scale
    and min per 16 columns): 16 tokens after 1000 rows, each wave over three 128-column chunks
    (both halves of the super-blocks)."""
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    _run_batch(c, 3072, 1100, 1000, 16, (t, t, t, t), seed=1670 + t, what=f"C3 {NAMES[t]}", batched=True)


@pytest.mark.parametrize("t", [gp.GGML_Q4_K, gp.GGML_IQ2_S], ids=["q4_k", "iq2_s"])
def test_block_batch_at_the_widest_embedding(t):
    """dim 16384: the token-batched projections stage 64 KB of norm weights in LDS (with
    IQ2_S's codebook and tables beside them)."""
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    _run_batch(c, 16384, 64, 40, 6, (t, t, t, t), seed=1690 + t, what=f"{NAMES[t]} width 16384", batched=True)


@pytest.mark.parametrize("K,ctx", [(4, 4096), (16, 4096), (4, 32768), (16, 32768)])
def test_block_batch_c3_q4_k_m(K, ctx):
    """C3 shape (24/8/128, dim 3072) with the Q4_K_M mix (Q4_K q, k, o; Q6_K v): K draft
    tokens verified after ctx - K cached rows."""
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    _run_batch(c, 3072, ctx, ctx - K, K, (gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K),
               seed=1700 + K, what=f"C3 Q4_K_M K={K} ctx {ctx}")


def test_block_batch_more_than_16_tokens():
    """20 tokens: a full group of 16, then 4 that attend to the first 16's appended rows."""
    c = hfp.ModelConfig(16, 4, 64, 1, rope_freq_base=10000.0)
    _run_batch(c, 2048, 256, 100, 20, (gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q8_0),
               seed=1710, what="20 tokens")


@pytest.mark.parametrize("dim", [1024, 4096, 8192])
def test_block_batch_widths(dim):
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    _run_batch(c, dim, 64, 30, 8, (gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K),
               seed=1720 + dim // 1024, what=f"Q4_K_M dim {dim}")


def test_block_batch_merged_qkv_biases_post_norm_scale():
    """Merged F16 QKV (Phi-3), biases, Gemma post-norm and the Granite residual scale."""
    c = hfp.ModelConfig(16, 16, 64, 1, rope_freq_base=10000.0)
    _run_batch(c, 1024, 64, 20, 6, (gp.GGML_F16,) * 4, seed=1730, what="merged f16 + post-norm",
               merged=True, bias=True, post=True, rscale=0.25)


def test_block_batch_qwen2_biases_q8_0_no_prenorm():
    c = hfp.ModelConfig(12, 2, 128, 1, architecture="qwen2", rope_freq_base=1e6)
    _run_batch(c, 1536, 64, 30, 7, (gp.GGML_Q8_0,) * 4, seed=1740, what="qwen2 bias q8_0",
               bias=True)
    c2 = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=1e6)
    _run_batch(c2, 1024, 64, 10, 3, (gp.GGML_Q4_0,) * 4, seed=1741, what="olmo2 post only",
               pre=False, post=True)


def test_block_batch_gpt_oss_shape():
    """GPT-OSS-20B attention: dim 2880 (not a multiple of 128: a partial last chunk) against
    q_dim 4096, Q8_0 with biases, sinks, the even-layer window across its edge."""
    c = hfp.ModelConfig(64, 8, 64, 2, architecture=hfp.ARCH_GPT_OSS, rope_freq_base=150000.0,
                        sliding_window=128, expert_count=32,
                        attention_scale=float(np.float32(1.3 * 1.3 / 8.0)))
    sinks = (np.random.default_rng(5).standard_normal(64) * 2).astype(F32)
    _run_batch(c, 2880, 256, 120, 12, (gp.GGML_Q8_0,) * 4, seed=1750, what="gpt-oss", bias=True,
               sinks=sinks, layer=0)


def test_block_batch_qk_norm_qwen3():
    c = hfp.ModelConfig(16, 8, 128, 1, architecture="qwen3", rope_freq_base=1e6, norm_eps=1e-6)
    rng = np.random.default_rng(77)
    qk = (rng.uniform(0.5, 1.5, 128).astype(F32), rng.uniform(0.5, 1.5, 128).astype(F32))
    _run_batch(c, 1024, 128, 50, 9, (gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K),
               seed=1760, what="qwen3 qk-norm", qk=qk)


@pytest.mark.parametrize("q8", [False, True], ids=["fp32", "q8_1"])
def test_block_batch_of_one_token_is_the_single_token_call(q8):
    """A group of one token runs the single-token launches (faster than the batched ones for one
    token): one-token llmp_attn_block_batch equals llmp_attn_block bit for bit, and 17 tokens
    take one batched group of 16 and one single-token call."""
    from tests.test_block_graph_gpu import _twins, _same
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    types = (gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K)
    (a, b), x = _twins(c, 1024, 256, 100, types, 51, 1, q8)
    try:
        a.uploadXBatch(x)
        a.forwardAttentionBlockBatch(0, 100, 1)
        b.uploadX(x[0])
        b.forwardAttentionBlock(0, 100)
        _same(a, b, a.downloadXBatch(1)[0], b.downloadX(), 101, "one-token batch")
    finally:
        a.close()
        b.close()
    _run_batch(c, 1024, 256, 60, 17, types, seed=1790 + int(q8), what=f"17 tokens ({'q8_1' if q8 else 'fp32'})",
               q8=q8, single_tail=True)


Q8_1_BATCH = [gp.GGML_Q4_K, gp.GGML_Q8_0, gp.GGML_Q5_0, gp.GGML_Q3_K, gp.GGML_Q5_K, gp.GGML_IQ4_NL,
              gp.GGML_IQ4_XS, gp.GGML_Q6_K]


@pytest.mark.parametrize("t", Q8_1_BATCH, ids=[NAMES[t] for t in Q8_1_BATCH])
def test_block_batch_q8_1_input_formats(t):
    """The Q8_1 input mode (the reference GPU's int8 matvecs) for K tokens: the routed types on
    the staged int8 quants of each token (tok_q8_kernel), exact integer block dots on the matrix
    cores; Q6_K on the fp32 input.  Against K sequential Q8_1-mode orc_attn_block calls."""
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    _run_batch(c, 1024, 64, 40, 5, (t, t, t, t), seed=1770 + t, what=f"q8_1 {NAMES[t]}", rounds=2,
               batched=True, q8=True)


@pytest.mark.parametrize("mix", ["q4_k_m", "q3_k_l", "q5_k_m"])
def test_block_batch_q8_1_c3_mixes(mix):
    """C3 with the K-quant mixes in the Q8_1 mode: one launch over an int8 format and Q6_K (or
    two int8 formats), 16 tokens after 1000 rows, then Wo on the quantised attention output."""
    types = {"q4_k_m": (gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K),
             "q3_k_l": (gp.GGML_Q3_K, gp.GGML_Q3_K, gp.GGML_Q5_K, gp.GGML_Q5_K),
             "q5_k_m": (gp.GGML_Q5_K, gp.GGML_Q5_K, gp.GGML_Q6_K, gp.GGML_Q5_K)}[mix]
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    _run_batch(c, 3072, 1100, 1000, 16, types, seed=1780 + len(mix), what=f"q8_1 C3 {mix}",
               batched=True, q8=True)


def test_block_batch_errors():
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    with hfp.HipForwardPass(c, 64) as fp:
        fp.setBlockConfig(1024)
        fp.uploadXBatch(np.zeros((4, 1024), F32))
        # no weights uploaded
        assert _lib.status("llmp_attn_block_batch", fp.kv.handle, 0, 0, 4, fp.gpuXBatch.ptr, 0) == 1
        rng = np.random.default_rng(3)
        lw, _ = _weights(c, 1024, (gp.GGML_Q4_K,) * 4, rng)
        fp.uploadLayerWeights(0, lw)
        # rows past the cache, a bad layer, zero tokens
        assert _lib.status("llmp_attn_block_batch", fp.kv.handle, 0, 62, 4, fp.gpuXBatch.ptr, 0) == 2
        assert _lib.status("llmp_attn_block_batch", fp.kv.handle, 1, 0, 4, fp.gpuXBatch.ptr, 0) == 2
        assert _lib.status("llmp_attn_block_batch", fp.kv.handle, 0, 0, 0, fp.gpuXBatch.ptr, 0) == 2
        assert _lib.status("llmp_attn_block_batch", fp.kv.handle, 0, 0, 4, fp.gpuXBatch.ptr + 4, 0) == 1
