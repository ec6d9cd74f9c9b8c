"""GPU parity of the attention half of a layer (llmp_attn_block: pre-norm, Q/K/V projections over
GGUF-format weights, the attention core, output projection, post-norm, residual) against the
oracle's restatement of TransformerBlock.forward / Attention.forward (orc.attn_block).

Weights come from tests/ggml_pack.py (packed from each format's layout).  Bar: the residual
after the block max-abs <= 1e-4 (and <= 1e-4 + 1e-3*|ref|) against the oracle; the appended
K/V row to the same bar (the projections sum in another order than the CPU path, so the row
is not bit-identical here; bit-exact appends are pinned by the from-projection entry points)
and every other cache row unchanged."""
import numpy as np
import pytest

from llmplayer_amd import _lib
from llmplayer_amd import hip_forward_pass as hfp
from oracle import oracle as orc
from tests import decode_cases as dc
from tests import ggml_pack as gp

pytestmark = pytest.mark.gpu

F32 = np.float32
TYPES = [gp.GGML_F32, gp.GGML_F16, gp.GGML_BF16, gp.GGML_Q8_0, gp.GGML_Q4_0, gp.GGML_Q4_K,
         gp.GGML_Q6_K, gp.GGML_Q5_0, gp.GGML_Q3_K, gp.GGML_Q5_K, gp.GGML_IQ4_NL, gp.GGML_IQ4_XS,
         gp.GGML_MXFP4, gp.GGML_Q5_1, gp.GGML_Q2_K, gp.GGML_IQ3_XXS, gp.GGML_IQ3_S, gp.GGML_IQ2_S]
NAMES = {0: "f32", 1: "f16", 30: "bf16", 8: "q8_0", 2: "q4_0", 12: "q4_k", 14: "q6_k", 6: "q5_0",
         11: "q3_k", 13: "q5_k", 20: "iq4_nl", 23: "iq4_xs", 39: "mxfp4", 7: "q5_1", 10: "q2_k",
         18: "iq3_xxs", 21: "iq3_s", 22: "iq2_s"}
# formats with no token-batched kernel, whose K-token calls run their tokens one by one: none
PER_TOKEN = ()


def _tensor(t, rows, cols, rng, scale=0.05):
    wb, vals = gp.random_weights(t, rows, cols, rng, scale)
    return hfp.GgufTensor(t, rows, cols, wb.reshape(-1)), wb


def _weights(c, dim, types, rng, merged=False, bias=False, post=False, pre=True, qkv_scale=0.05):
    """types: (tq, tk, tv, to); qkv_scale: the Q/K/V weights' magnitude.  Returns
    (TransformerLayerWeights, orc.BlockWeights)."""
    qd, kvd = c.q_dim, c.kv_dim
    tq, tk, tv, to = types
    lw = hfp.TransformerLayerWeights()
    bw = orc.BlockWeights(dim)
    if merged:
        t, wb = _tensor(tq, qd + 2 * kvd, dim, rng, qkv_scale)
        lw.wqkv, bw.wqkv, bw.wqkv_type = t, wb, tq
    else:
        lw.wq, bw.wq = _tensor(tq, qd, dim, rng, qkv_scale)
        lw.wk, bw.wk = _tensor(tk, kvd, dim, rng, qkv_scale)
        lw.wv, bw.wv = _tensor(tv, kvd, dim, rng, qkv_scale)
        bw.wq_type, bw.wk_type, bw.wv_type = tq, tk, tv
    lw.wo, bw.wo = _tensor(to, dim, qd, rng)
    bw.wo_type = to
    if pre:
        lw.attnNorm = bw.attn_norm = rng.uniform(0.5, 1.5, dim).astype(F32)
    if post:
        lw.postAttnNorm = bw.post_attn_norm = rng.uniform(0.5, 1.5, dim).astype(F32)
    if bias:
        lw.qBias = bw.q_bias = (rng.standard_normal(qd) * 0.1).astype(F32)
        lw.kBias = bw.k_bias = (rng.standard_normal(kvd) * 0.1).astype(F32)
        lw.vBias = bw.v_bias = (rng.standard_normal(kvd) * 0.1).astype(F32)
        lw.woBias = bw.o_bias = (rng.standard_normal(dim) * 0.1).astype(F32)
    return lw, bw


def _run(c, dim, max_seq, pos0, steps, types, seed, what, merged=False, bias=False, post=False,
         pre=True, rscale=0.0, qk=None, splits=0, devpos=False, q8=False, sinks=None, layer=0,
         weights=None):
    """`steps` block calls at positions pos0.. on layer `layer` of c (its window, RoPE table
    and sinks), each checked against orc.attn_block.  weights: a prepared (layer weights, oracle
    weights) pair in place of random ones of `types`."""
    rng = np.random.default_rng(seed)
    lw, bw = weights if weights is not None else _weights(c, dim, types, rng, merged, bias, post, pre)
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
        worst = 0.0
        for s in range(steps):
            pos = pos0 + s
            x = (rng.standard_normal(dim) * 2).astype(F32)
            dc.log(f"[gpu] block {what}: step {s} pos {pos}")
            fp.uploadX(x)
            if devpos:
                fp.updateTokenParams(pos)
            fp.forwardAttentionBlock(layer, pos, splits, device_position=devpos)
            got = fp.downloadX()
            want, attn = orc.attn_block(oc, bw, kc, vc, x, layer, pos, qnorm_w=qw, knorm_w=kw,
                                        rope_cos=cs, rope_sin=sn, n_threads=16, return_attn=True)
            gk, gv = fp.kv.read(layer, 0, pos + 1)
            assert np.array_equal(gk[:pos], kc[:pos]) and np.array_equal(gv[:pos], vc[:pos])
            dc.compare_out(gk[pos], kc[pos], f"block {what} appended K row")
            dc.compare_out(gv[pos], vc[pos], f"block {what} appended V row")
            if q8 and orc.q8_1_routed(bw.wo_type):
                worst = max(worst, _compare_q8_output(got, want, attn, bw, rscale,
                                                      f"block {what} pos {pos}"))
            else:
                worst = max(worst, dc.compare_out(got, want, f"block {what} pos {pos}"))
            # continue from the device's rows so later steps attend to the same cache
            kc[pos], vc[pos] = gk[pos], gv[pos]
        dc.log(f"[gpu] block {what}: ok, max abs err {worst:.2e}")


def _compare_q8_output(got, want, attn, bw, rscale, what):
    """The residual after a Q8_1-mode block.  The attention output is computed in two orders
    (GPU, oracle), so an element within rounding of a quantisation tie may take the other
    int8 value ahead of the output projection; each such element j may move output i by
    |Wo[i, j]| * d_j (its block's scale).  The bar is the usual one plus that allowance for the
    oracle's near-tie elements (|frac(|x|*127/max) - 1/2| < 2e-3), and nothing more."""
    qd = attn.size
    a = attn.astype(np.float32).reshape(-1, 32)
    m = np.abs(a).max(axis=1)
    inv = np.where(m > 0, np.float32(127) / np.where(m > 0, m, 1), 0).astype(np.float32)
    t = np.abs(a * inv[:, None])
    near = (np.abs(t - np.floor(t) - 0.5) < 2e-3).reshape(-1)
    d = np.repeat(m / np.float32(127), 32)
    wo = orc.dequant_rows(bw.wo_type, bw.wo, bw.dim, qd).astype(np.float64)
    allow = np.abs(wo[:, near]) @ d[near].astype(np.float64) if near.any() else np.zeros(bw.dim)
    if rscale > 0:
        allow = allow * rscale
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = dc.ATOL + dc.RTOL * np.abs(want.astype(np.float64)) + 1.01 * allow
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert (err <= bound).all(), (f"{what}: {int((err > bound).sum())} elements above the bar "
                                  f"(max abs err {err.max():.3e}, {int(near.sum())} near-tie inputs)")
    dc.log(f"[gpu] {what}: max abs err {err.max():.2e}, {int(near.sum())} near-tie inputs of Wo")
    return float(err.max())


@pytest.mark.parametrize("t", TYPES, ids=[NAMES[t] for t in TYPES])
def test_block_every_weight_format(t):
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    _run(c, 1024, 64, 40, 2, (t, t, t, t), seed=600 + t, what=NAMES[t])


WIDE = [gp.GGML_F32, gp.GGML_F16, gp.GGML_BF16, gp.GGML_Q8_0, gp.GGML_Q4_0, gp.GGML_Q5_0,
        gp.GGML_IQ4_NL, gp.GGML_MXFP4, gp.GGML_Q3_K, gp.GGML_Q5_K, gp.GGML_IQ4_XS, gp.GGML_Q5_1,
        gp.GGML_Q2_K, gp.GGML_IQ3_XXS, gp.GGML_IQ3_S, gp.GGML_IQ2_S]


@pytest.mark.parametrize("t", WIDE, ids=[NAMES[t] for t in WIDE])
def test_block_weight_formats_at_width_4096(t):
    """Rows of 4096 columns: 8 unit rounds in registers and a second batch for the 4-weight
    unit formats (F32, F16, BF16, Q8_0), 8 rounds for the 8-weight units (Q4_0, Q5_0, IQ4_NL,
    MXFP4, Q5_K, IQ4_XS, IQ3_XXS, IQ2_S), 6 and a second batch for IQ3_S, 4 for Q3_K's 16-weight
    units."""
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    _run(c, 4096, 64, 33, 1, (t, t, t, t), seed=900 + t, what=f"{NAMES[t]} width 4096")


@pytest.mark.parametrize("t", [gp.GGML_F32, gp.GGML_Q8_0, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_IQ2_S],
                         ids=["f32", "q8_0", "q4_k", "q6_k", "iq2_s"])
def test_block_weight_formats_at_the_widest_embedding(t):
    """dim 16384, the widest llmp_block_config accepts: the Q/K/V projections stage 64 KB of
    input in LDS, plus the chunk sums (Q4_K), the per-row scale tables (Q4_K, Q6_K, IQ2_S) and
    the codebook (IQ2_S); F32 and Q8_0 rows take several batches of unit rounds.  The Q/K/V weights are half the usual magnitude, so that
    the 16384-term projections land at the magnitudes of the 4096-wide tests (and their fp32
    reordering error with them)."""
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    w = _weights(c, 16384, (t, t, t, t), np.random.default_rng(950 + t), qkv_scale=0.025)
    _run(c, 16384, 64, 33, 1, (t, t, t, t), seed=950 + t, what=f"{NAMES[t]} width 16384", weights=w)


@pytest.mark.parametrize("dim", [2048, 3072, 8192])
def test_block_c3_q3_k_l_and_q5_k_m_mixes(dim):
    """The Q3_K_L mix (Q3_K q and k, Q5_K v and o; q, k and v in one two-format launch) and the
    Q5_K_M mix (Q5_K q, k, o and Q6_K v), three steps after a 300-row prefix."""
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    _run(c, dim, 512, 300, 3, (gp.GGML_Q3_K, gp.GGML_Q3_K, gp.GGML_Q5_K, gp.GGML_Q5_K),
         seed=615 + dim // 1024, what=f"Q3_K_L dim {dim}")
    _run(c, dim, 512, 300, 3, (gp.GGML_Q5_K, gp.GGML_Q5_K, gp.GGML_Q6_K, gp.GGML_Q5_K),
         seed=625 + dim // 1024, what=f"Q5_K_M dim {dim}")


def test_block_iq4_xs_with_q5_k_v_and_mxfp4_extreme_exponents():
    """IQ4_XS q and k with a Q5_K v (the IQ4_XS mix at GQA 4 and above: two launches), and an
    MXFP4 output projection whose block exponents include 0, 1 and 255."""
    c = hfp.ModelConfig(16, 4, 128, 1, rope_freq_base=500000.0)
    _run(c, 2048, 256, 100, 2, (gp.GGML_IQ4_XS, gp.GGML_IQ4_XS, gp.GGML_Q5_K, gp.GGML_IQ4_XS),
         seed=670, what="IQ4_XS + Q5_K v")
    rng = np.random.default_rng(671)
    lw, bw = _weights(c, 1024, (gp.GGML_MXFP4,) * 4, rng)
    e = rng.integers(119, 124, (1024, 2048 // 32))
    e[0, :3] = (0, 1, 255)
    e[5, 7] = 1
    wb, _ = gp.pack_mxfp4(e, rng.integers(0, 16, (1024, 2048)))
    lw.wo = hfp.GgufTensor(gp.GGML_MXFP4, 1024, 2048, wb.reshape(-1))
    bw.wo = wb
    _run(c, 1024, 64, 20, 2, None, seed=672, what="MXFP4 special exponents", weights=(lw, bw))


def test_block_c3_llama3b_shape_q4_k_m_mix():
    """C3 shape (24/8/128, dim 3072) with the Q4_K_M mix: Q4_K for q, k, o and Q6_K for v
    (separate launches per weight type), four steps after a 2000-row prefix."""
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    _run(c, 3072, 2048, 2000, 4, (gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K),
         seed=610, what="C3 Q4_K_M")


@pytest.mark.parametrize("dim", [1024, 2048, 4096, 8192])
def test_block_q4_k_m_mix_widths(dim):
    """The Q4_K + Q6_K projections in one launch at widths that take 2, 4 and 8 unit rounds in
    registers and, at 8192, a second batch of rounds."""
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    _run(c, dim, 64, 30, 2, (gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K),
         seed=700 + dim // 1024, what=f"Q4_K_M mix dim {dim}")


def test_block_q6_k_q4_k_mix_swapped():
    """Q6_K for q, k and Q4_K for v (the pair in the other order, GemvSeg::fmt by type)."""
    c = hfp.ModelConfig(16, 4, 128, 1, rope_freq_base=500000.0)
    _run(c, 2048, 64, 21, 2, (gp.GGML_Q6_K, gp.GGML_Q6_K, gp.GGML_Q4_K, gp.GGML_Q6_K),
         seed=720, what="Q6_K q/k + Q4_K v", bias=True)


def test_block_merged_qkv_phi3():
    c = hfp.ModelConfig(16, 16, 64, 1, rope_freq_base=10000.0)
    _run(c, 1024, 64, 20, 2, (gp.GGML_F16,) * 4, seed=620, what="merged QKV f16", merged=True)


def test_block_qwen2_biases_q8_0():
    c = hfp.ModelConfig(12, 2, 128, 1, architecture="qwen2", rope_freq_base=1e6)   # Qwen2-1.5B shape
    _run(c, 1536, 64, 30, 2, (gp.GGML_Q8_0,) * 4, seed=630, what="qwen2 bias q8_0", bias=True)


def test_block_gemma_post_norm_bias_and_granite_scale():
    c = hfp.ModelConfig(8, 4, 256, 1, architecture=hfp.ARCH_GEMMA3, rope_freq_base=1e6,
                        norm_eps=1e-6)
    rng = np.random.default_rng(640)
    qk = (rng.uniform(0.5, 1.5, 256).astype(F32), rng.uniform(0.5, 1.5, 256).astype(F32))
    _run(c, 1536, 64, 25, 2, (gp.GGML_BF16, gp.GGML_Q6_K, gp.GGML_Q6_K, gp.GGML_BF16), seed=641,
         what="post-norm + bias + residual scale", bias=True, post=True, rscale=0.22, qk=qk)


def test_block_olmo2_post_norm_only_and_device_position():
    c = hfp.ModelConfig(16, 16, 128, 1, rope_freq_base=500000.0)
    _run(c, 2048, 80, 50, 3, (gp.GGML_Q4_K,) * 4, seed=650, what="post-norm only, device position",
         post=True, pre=False, devpos=True)


def test_block_split_settings_agree():
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    for splits in (1, 7, 64):
        _run(c, 3072, 600, 512, 1, (gp.GGML_Q8_0,) * 4, seed=660 + splits,
             what=f"C3 q8_0 splits={splits}", splits=splits)


# ---- the Q8_1 input mode (the reference GPU's int8 matvecs: Q4_K, Q8_0, Q5_0, Q3_K, Q5_K, ----
# ---- IQ4_NL, IQ4_XS; the other formats on the fp32 input) ---------------------------------
# The oracle quantises the same staged-norm floats, so the int8 operands are the GPU's; the
# outputs differ by float summation order, and by a rare quantisation tie of the attention
# output (computed in two orders) ahead of the output projection.

Q8_1_CASES = [gp.GGML_Q4_K, gp.GGML_Q8_0, gp.GGML_Q5_0, gp.GGML_Q3_K, gp.GGML_Q5_K, gp.GGML_IQ4_NL,
              gp.GGML_IQ4_XS, gp.GGML_Q6_K, gp.GGML_F16, gp.GGML_Q4_0, gp.GGML_MXFP4, gp.GGML_IQ3_S]


@pytest.mark.parametrize("t", Q8_1_CASES,
                         ids=[NAMES[t] + ("" if orc.q8_1_routed(t) else "-fp32") for t in Q8_1_CASES])
def test_block_q8_1_input_formats(t):
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    _run(c, 1024, 64, 40, 2, (t, t, t, t), seed=800 + t, what=f"q8_1 {NAMES[t]}", q8=True)


def test_block_q8_1_c3_llama3b_q4_k_m_mix():
    """The C3 shape with the Q4_K_M mix: Q4_K rows on the Q8_1 input and Q6_K rows on the
    fp32 input in one launch, Wo on the quantised attention output."""
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    _run(c, 3072, 2048, 2000, 4, (gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K),
         seed=810, what="q8_1 C3 Q4_K_M", q8=True)


@pytest.mark.parametrize("dim", [2048, 3072, 8192])
def test_block_q8_1_q3_k_l_and_q5_k_m_mixes(dim):
    """The Q3_K_L mix (Q3_K and Q5_K rows both on the Q8_1 input in one launch; 8192 columns
    take a second batch of the Q5_K side's 3 rounds) and the Q5_K_M mix (Q5_K on the Q8_1
    input next to Q6_K on the fp32 one) in the Q8_1 mode."""
    c = hfp.ModelConfig(24, 8, 128, 1, rope_freq_base=500000.0)
    _run(c, dim, 512, 300, 2, (gp.GGML_Q3_K, gp.GGML_Q3_K, gp.GGML_Q5_K, gp.GGML_Q5_K),
         seed=850 + dim // 1024, what=f"q8_1 Q3_K_L dim {dim}", q8=True)
    _run(c, dim, 512, 300, 2, (gp.GGML_Q5_K, gp.GGML_Q5_K, gp.GGML_Q6_K, gp.GGML_Q5_K),
         seed=860 + dim // 1024, what=f"q8_1 Q5_K_M dim {dim}", q8=True)


@pytest.mark.parametrize("dim", [2048, 4096, 8192])
def test_block_q8_1_widths(dim):
    """2, 4 and 8 unit rounds of the Q8_1 Q4_K side (the pair caps it at 4: a second batch at
    8192), Q8_0 rows at 4, 8 and 16 rounds (two batches)."""
    c = hfp.ModelConfig(8, 2, 128, 1, rope_freq_base=500000.0)
    _run(c, dim, 64, 30, 1, (gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K),
         seed=820 + dim // 1024, what=f"q8_1 Q4_K_M dim {dim}", q8=True)
    _run(c, dim, 64, 30, 1, (gp.GGML_Q8_0,) * 4, seed=830 + dim // 1024,
         what=f"q8_1 Q8_0 dim {dim}", q8=True)


def test_block_q8_1_merged_qkv_bias_granite_scale():
    c = hfp.ModelConfig(12, 4, 128, 1, rope_freq_base=1e6, norm_eps=1e-6)
    _run(c, 3072, 64, 20, 2, (gp.GGML_Q8_0,) * 4, seed=840, what="q8_1 merged Q8_0",
         merged=True, bias=True, rscale=0.3, q8=True)


# ---- the MoE engines' attention half (Qwen3MoEInferenceEngine.gqaAttention, :237-328) -------

@pytest.mark.parametrize("layer", [0, 1], ids=["windowed", "global"])
@pytest.mark.parametrize("q8", [False, True], ids=["f32-input", "q8_1-input"])
def test_block_gptoss_20b_attention(layer, q8):
    """GPT-OSS-20B's attention half: dim 2880 with q_dim 4096 (64 x 64), Q8_0 projections with
    biases on q, k, v and o, attention sinks, the engine's window of 128 on even layers, the
    YaRN-style scale; positions across the window edge."""
    c = hfp.ModelConfig(64, 8, 64, 2, architecture=hfp.ARCH_GPT_OSS, rope_freq_base=150000.0,
                        sliding_window=128, expert_count=32,
                        attention_scale=float(np.float32(1.3 * 1.3 / 8.0)))
    sinks = np.random.default_rng(850).uniform(-1.0, 3.0, 64).astype(np.float32)
    _run(c, 2880, 256, 126, 3, (gp.GGML_Q8_0,) * 4, seed=851 + layer, what=f"gpt-oss layer {layer}",
         bias=True, sinks=sinks, layer=layer, q8=q8)


def test_block_qwen3_30b_a3b_attention():
    """Qwen3-30B-A3B's attention half: dim 2048 with q_dim 4096 (32 x 128), 4 KV heads (GQA 8),
    per-head QK-norm, the Q4_K_M mix."""
    c = hfp.ModelConfig(32, 4, 128, 1, architecture=hfp.ARCH_QWEN3, rope_freq_base=1e6,
                        norm_eps=1e-6)
    rng = np.random.default_rng(860)
    qk = (rng.uniform(0.5, 1.5, 128).astype(F32), rng.uniform(0.5, 1.5, 128).astype(F32))
    _run(c, 2048, 1024, 900, 3, (gp.GGML_Q4_K, gp.GGML_Q4_K, gp.GGML_Q6_K, gp.GGML_Q4_K),
         seed=861, what="qwen3-30b-a3b", qk=qk)


def test_block_error_codes():
    c = hfp.ModelConfig(8, 2, 64, 1, rope_freq_base=1e4)
    with hfp.HipForwardPass(c, 32) as fp:
        h = fp.kv.handle
        assert _lib.status("llmp_layer_weight", h, 0, 1, 0, 512, 512, None, 0) == 1  # no block config
        assert _lib.status("llmp_block_config", h, 500, 0.0) == 1                     # not a multiple of 32
        assert _lib.status("llmp_block_input_mode", h, 2) == 1                        # unknown mode
        fp.setBlockConfig(512)
        x = fp.gpuX.ptr
        assert _lib.status("llmp_attn_block", h, 0, 3, 0, x, 0, 0) == 1               # no weights yet
        w = np.zeros(512 * 512 * 4, np.uint8)
        assert _lib.status("llmp_layer_weight", h, 0, _lib.LLMP_W_Q, 0, 128, 512, w.ctypes.data, 128 * 512 * 4) == 1  # rows != q_dim
        assert _lib.status("llmp_layer_weight", h, 0, _lib.LLMP_W_Q, 16, 512, 512, w.ctypes.data, 512 * 66 // 256 * 512) == 6  # IQ2_XXS: no kernel (the reference loads none either)
        assert _lib.status("llmp_layer_weight", h, 0, _lib.LLMP_W_Q, 0, 512, 512, w.ctypes.data, 100) == 1   # byte count
        assert _lib.status("llmp_layer_weight", h, 0, 11, 0, 1, 512, w.ctypes.data, 2048) == 1  # bad slot
        assert _lib.status("llmp_layer_weight", h, 0, _lib.LLMP_W_ATTN_NORM, 8, 1, 512, w.ctypes.data, 2048) == 1  # vector not fp32
