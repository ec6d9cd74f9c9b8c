"""Pins the CPU restatement (oracle/attn_oracle.c) before it is trusted as the checker.

The reference ships no tests or golden vectors for this path and its Java cannot run here,
so each oracle function is pinned by what the mathematics fixes: closed forms, invariants,
special cases that reduce to a textbook routine, and float64 brute force on small shapes.
Each check is chosen so that a plausible slip (dropped FMA, wrong pair index, eps in the
wrong place, wrong GQA mapping, off-by-one window) fails it.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests import refmath as rm

F32 = np.float32


# ---------------------------------------------------------------- SimdVectorOps.dot / saxpy
def test_dot_integer_closed_form():
    for n in (1, 7, 8, 9, 16, 64, 100, 128, 256):
        a = np.arange(1, n + 1, dtype=F32)
        assert orc.dot(a, np.ones(n, F32)) == F32(n * (n + 1) / 2)
        assert orc.dot(a, a) == F32(n * (n + 1) * (2 * n + 1) / 6)


def test_dot_uses_fma_on_lanes_and_plain_mul_add_on_tail():
    # x*x with x = 1 + 2^-12 is 1 + 2^-11 + 2^-24, which is not a float: a fused
    # multiply-add keeps the 2^-24, an unfused one rounds it away (Vector.fma vs a*b+c).
    x = F32(1 + 2.0 ** -12)
    m = F32(-(1 + 2.0 ** -11))
    a = np.zeros(16, F32); b = np.zeros(16, F32)
    a[0], b[0] = m, F32(1)          # lane 0 first term
    a[8], b[8] = x, x               # lane 0 second term -> fma keeps 2^-24
    assert orc.dot(a, b) == F32(2.0 ** -24)
    # tail element (index 8 of a 9-vector) uses a separate multiply and add
    a9 = np.zeros(9, F32); b9 = np.zeros(9, F32)
    a9[0], b9[0] = m, F32(1)
    a9[8], b9[8] = x, x
    assert orc.dot(a9, b9) == F32(0.0)


def test_dot_matches_float64():
    rng = np.random.default_rng(1)
    for n in (64, 128, 256, 77):
        a = rng.standard_normal(n).astype(F32)
        b = rng.standard_normal(n).astype(F32)
        want = float(a.astype(np.float64) @ b.astype(np.float64))
        assert abs(float(orc.dot(a, b)) - want) < 1e-5 * n


def test_saxpy_fused_on_lanes():
    x = np.full(8, F32(1 + 2.0 ** -12), F32)
    y = np.full(8, F32(-(1 + 2.0 ** -11)), F32)
    out = orc.saxpy(F32(1 + 2.0 ** -12), x, y)
    assert np.all(out == F32(2.0 ** -24))
    out9 = orc.saxpy(F32(1 + 2.0 ** -12), np.full(9, x[0], F32), np.full(9, y[0], F32))
    assert out9[8] == F32(0.0) and out9[0] == F32(2.0 ** -24)


# ------------------------------------------------------------------------- softmax
def test_softmax_closed_forms():
    assert np.all(orc.softmax(np.zeros(10, F32)) == F32(0.1))
    assert orc.softmax(np.array([3.5], F32))[0] == F32(1.0)
    rng = np.random.default_rng(2)
    x = rng.standard_normal(1000).astype(F32) * 4
    got = orc.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max())
    np.testing.assert_allclose(got, e / e.sum(), rtol=2e-6, atol=1e-9)
    assert abs(got.astype(np.float64).sum() - 1) < 1e-5
    # argmax kept, ordering kept
    assert np.argmax(got) == np.argmax(x)
    assert np.all(np.diff(got[np.argsort(x)]) >= 0)


# --------------------------------------------------------------------- QK-norm
def test_per_head_norm_constant_vector_is_sign():
    D = 128
    x = np.concatenate([np.full(D, 3.0, F32), np.full(D, -0.25, F32)])
    out = orc.per_head_norm(x, np.ones(D, F32), 2, D, 0.0)
    np.testing.assert_allclose(out[:D], 1.0, rtol=2e-7)
    np.testing.assert_allclose(out[D:], -1.0, rtol=2e-7)


def test_per_head_norm_power_of_two_scale_invariance_is_exact():
    rng = np.random.default_rng(3)
    D = 128
    x = rng.standard_normal(4 * D).astype(F32)
    w = rng.uniform(0.5, 1.5, D).astype(F32)
    base = orc.per_head_norm(x, w, 4, D, 0.0)
    for k in (-6, -1, 3, 10):
        assert np.array_equal(orc.per_head_norm(x * F32(2.0 ** k), w, 4, D, 0.0), base)


def test_per_head_norm_matches_float64_with_eps_and_weights():
    rng = np.random.default_rng(4)
    for D, H, eps in ((128, 16, 1e-6), (256, 4, 1e-6), (64, 3, 0.5)):
        x = (rng.standard_normal(H * D) * rng.uniform(0.01, 3, H).repeat(D)).astype(F32)
        w = rng.uniform(0.5, 1.5, D).astype(F32)
        got = orc.per_head_norm(x, w, H, D, eps)
        want = rm.rms_norm_heads(x, w, H, D, eps)
        np.testing.assert_allclose(got, want, rtol=3e-6, atol=1e-7)


# ------------------------------------------------------------------------ RoPE
@pytest.mark.parametrize("R,theta", [(64, 5e5), (128, 1e6), (256, 1e4), (128, 5e5)])
def test_rope_tables_match_angle_definition(R, theta):
    S = 2048
    cos_t, sin_t = orc.rope_tables(R, S, theta)
    assert np.all(cos_t[0] == 1) and np.all(sin_t[0] == 0)
    i = np.arange(R // 2)
    freq = (1.0 / np.power(np.float64(F32(theta)), 2.0 * i / R)).astype(F32)
    ang = (np.arange(S, dtype=F32)[:, None] * freq[None, :]).astype(F32)
    # float32 angle as the reference forms it, then cos/sin in double -> float
    np.testing.assert_array_max_ulp(cos_t, np.cos(ang.astype(np.float64)).astype(F32), 1)
    np.testing.assert_array_max_ulp(sin_t, np.sin(ang.astype(np.float64)).astype(F32), 1)
    # pair 0 rotates by exactly `pos` radians
    np.testing.assert_allclose(cos_t[:, 0], np.cos(np.arange(S)), atol=2e-7)


def test_rope_freq_factors_divide_the_base_frequency():
    # RoPE.java:86-89: baseFreq = (float)(1/pow(theta, 2i/R)); baseFreq /= freqFactors[i] for
    # the pairs the factor array covers; angle = (float)(pos * freq)
    R, S, theta = 128, 600, 1e6
    ff = np.linspace(1.0, 8.0, R // 2 - 8).astype(F32)   # shorter than R/2: tail unscaled
    cos_t, sin_t = orc.rope_tables(R, S, theta, freq_factors=ff)
    i = np.arange(R // 2)
    base = (1.0 / np.power(np.float64(F32(theta)), 2.0 * i / R)).astype(F32)
    freq = base.copy()
    freq[:ff.size] = (base[:ff.size] / ff).astype(F32)
    ang = (np.arange(S, dtype=F32)[:, None] * freq[None, :]).astype(F32)
    np.testing.assert_array_max_ulp(cos_t, np.cos(ang.astype(np.float64)).astype(F32), 1)
    np.testing.assert_array_max_ulp(sin_t, np.sin(ang.astype(np.float64)).astype(F32), 1)


def test_rope_linear_scale_divides_frequencies():
    R, S = 128, 64
    c1, s1 = orc.rope_tables(R, S * 8, 1e4)
    c8, s8 = orc.rope_tables(R, S * 8, 1e4, linear_freq_scale=8.0)
    # angle(pos*8, scale 8) == angle(pos, 1) up to float rounding of freq/8
    np.testing.assert_allclose(c8[::8][:S], c1[:S], atol=2e-5)
    np.testing.assert_allclose(s8[::8][:S], s1[:S], atol=2e-5)


# ---- YaRN tables (RoPE.java:45-117): closed forms of the NTK-by-parts blend -----------------
def _yarn_dims(R, theta, L, beta_fast=32.0, beta_slow=1.0):
    """The correction dims of the YaRN paper, R*ln(L/(2*pi*beta)) / (2*ln(theta)), in float64."""
    def corr(beta):
        return R * np.log(L / (beta * 2 * np.pi)) / (2 * np.log(theta))
    return max(0.0, np.floor(corr(beta_fast))), min(R / 2 - 1, np.ceil(corr(beta_slow)))


def test_rope_yarn_factor_one_is_the_plain_table():
    c0, s0 = orc.rope_tables(64, 300, 1.5e5)
    c1, s1, ms = orc.rope_tables_yarn(64, 300, 1.5e5, 1.0, 4096, 0.1)
    assert np.array_equal(c0, c1) and np.array_equal(s0, s1) and ms == 1.0


@pytest.mark.parametrize("R,theta,s,L", [(64, 1.5e5, 32.0, 4096), (128, 1e6, 4.0, 32768),
                                         (128, 1e4, 40.0, 4096)])
def test_rope_yarn_blend_and_correction_dims(R, theta, s, L):
    """Dims up to the fast correction dim keep the base frequency (bit-identical to the plain
    table), dims from the slow one on take base/s (bit-identical to the linear-scaled table), and
    the dims between blend linearly in the dim index."""
    S = 64
    cy, sy, _ = orc.rope_tables_yarn(R, S, theta, s, L)
    c1, s1 = orc.rope_tables(R, S, theta)
    cs, ss = orc.rope_tables(R, S, theta, linear_freq_scale=s)
    low, high = _yarn_dims(R, theta, L)
    i = np.arange(R // 2)
    ext, itp = i <= low, i >= high
    assert ext.any() and itp.any() and (~ext & ~itp).any(), (low, high)
    assert np.array_equal(cy[:, ext], c1[:, ext]) and np.array_equal(sy[:, ext], s1[:, ext])
    assert np.array_equal(cy[:, itp], cs[:, itp]) and np.array_equal(sy[:, itp], ss[:, itp])
    # between: at pos 1 the angle is the frequency itself
    base = 1.0 / np.power(np.float64(F32(theta)), 2.0 * i / R)
    ramp = 1.0 - np.clip((i - low) / max(0.001, high - low), 0.0, 1.0)
    want = base * ramp + base / s * (1 - ramp)
    mid = ~ext & ~itp
    np.testing.assert_allclose(np.arcsin(sy[1, mid].astype(np.float64)), want[mid], rtol=2e-6)
    assert np.all(np.diff(np.arcsin(sy[1].astype(np.float64))) < 0)   # frequencies decrease


@pytest.mark.parametrize("s,log_mul", [(32.0, 0.0), (40.0, 0.0707), (4.0, 1.0)])
def test_rope_yarn_mscale_closed_form(s, log_mul):
    _, _, ms = orc.rope_tables_yarn(64, 4, 1e4, s, 4096, log_mul)
    attn = 0.1 * log_mul * np.log(s) + 1.0 if log_mul > 0 else 1.0
    assert abs(float(ms) - attn * (1.0 + 0.1 * np.log(s))) < 2e-6


@pytest.mark.parametrize("rope_type", [0, 2])
def test_rope_apply_identity_at_pos0_and_pairing(rope_type):
    H, D, R = 3, 64, 64
    cos_t, sin_t = orc.rope_tables(R, 16, 5e5)
    rng = np.random.default_rng(5)
    x = rng.standard_normal(H * D).astype(F32)
    assert np.array_equal(orc.rope_apply_all(x, H, D, R, rope_type, cos_t, sin_t, 0), x)
    # one-hot on the first element of each pair lands on (cos, sin) at the partner index
    half = R // 2
    for i in (0, 1, 5, half - 1):
        e = np.zeros(H * D, F32)
        i0 = 2 * i if rope_type == 0 else i
        i1 = 2 * i + 1 if rope_type == 0 else half + i
        e[D + i0] = 1.0
        out = orc.rope_apply_all(e, H, D, R, rope_type, cos_t, sin_t, 7)
        assert out[D + i0] == cos_t[7, i] and out[D + i1] == sin_t[7, i]
        out[D + i0] = 0; out[D + i1] = 0
        assert not out.any()


@pytest.mark.parametrize("rope_type", [0, 2])
def test_rope_apply_matches_rotation_and_preserves_pair_norms(rope_type):
    H, D, R, theta = 4, 128, 128, 1e6
    S = 4096
    cos_t, sin_t = orc.rope_tables(R, S, theta)
    rng = np.random.default_rng(6)
    x = rng.standard_normal(H * D).astype(F32)
    for pos in (1, 17, 4095):
        got = orc.rope_apply_all(x, H, D, R, rope_type, cos_t, sin_t, pos)
        want = rm.rope_rotate(x, H, D, R, rope_type, rm.rope_angles(R, pos, float(F32(theta))))
        np.testing.assert_allclose(got, want, atol=3e-6)
        # rotation back by the same angle (sin negated) recovers x
        back = orc.rope_apply_all(got, H, D, R, rope_type, cos_t, -sin_t, pos)
        np.testing.assert_allclose(back, x, atol=2e-6)
        half = R // 2
        xx = x.reshape(H, D); gg = got.reshape(H, D)
        if rope_type == 0:
            n0 = xx[:, 0::2] ** 2 + xx[:, 1::2] ** 2; n1 = gg[:, 0::2] ** 2 + gg[:, 1::2] ** 2
        else:
            n0 = xx[:, :half] ** 2 + xx[:, half:] ** 2; n1 = gg[:, :half] ** 2 + gg[:, half:] ** 2
        np.testing.assert_allclose(n1, n0, rtol=3e-6, atol=1e-7)


def test_partial_rope_leaves_tail_untouched():
    H, D, R = 2, 128, 64
    cos_t, sin_t = orc.rope_tables(R, 32, 1e4)
    x = np.random.default_rng(7).standard_normal(H * D).astype(F32)
    out = orc.rope_apply_all(x, H, D, R, 2, cos_t, sin_t, 9).reshape(H, D)
    assert np.array_equal(out[:, R:], x.reshape(H, D)[:, R:])


def test_global_layer_patterns():
    g3 = [orc.is_global_layer(orc.ARCH_GEMMA3, l) for l in range(26)]
    assert [l for l in range(26) if g3[l]] == [5, 11, 17, 23]
    assert [orc.is_global_layer(orc.ARCH_GEMMA2, l) for l in range(4)] == [False, True, False, True]
    assert [orc.is_global_layer(orc.ARCH_GPT_OSS, l) for l in range(4)] == [True, False, True, False]
    assert [orc.is_global_layer(orc.ARCH_COHERE2, l) for l in range(8)] == [
        False, False, False, True, False, False, False, True]
    assert all(orc.is_global_layer(orc.ARCH_OTHER, l) for l in range(8))


# ------------------------------------------------------------ full attention layer-call
def _setup(cfg, pos, seed, k_scale=1.0, theta=5e5):
    rng = np.random.default_rng(seed)
    kv = cfg.kv_dim
    kc = np.zeros((cfg.max_seq, kv), F32); vc = np.zeros((cfg.max_seq, kv), F32)
    kc[:pos] = rng.standard_normal((pos, kv)).astype(F32) * F32(k_scale)
    vc[:pos] = rng.standard_normal((pos, kv)).astype(F32)
    q = rng.standard_normal(cfg.n_heads * cfg.head_size).astype(F32)
    k = (rng.standard_normal(kv) * k_scale).astype(F32)
    v = rng.standard_normal(kv).astype(F32)
    cos_t, sin_t = orc.rope_tables(cfg.rope_dim or cfg.head_size, cfg.max_seq, theta)
    return kc, vc, q, k, v, cos_t, sin_t


def test_pos0_output_is_v0():
    # DiagnosticRunner.java:367-385: at pos=0 attention output = V directly
    cfg = orc.OracleConfig(32, 8, 64, 16)
    kc, vc, q, k, v, cs, sn = _setup(cfg, 0, 10)
    out, _, _ = orc.forward_from_projections(cfg, kc, vc, q, k, v, 0, 0, rope_cos=cs, rope_sin=sn)
    want = np.repeat(v.reshape(8, 64), 4, axis=0).reshape(-1)
    assert np.array_equal(out, want)


def test_uniform_scores_give_mean_of_v():
    cfg = orc.OracleConfig(24, 8, 128, 300)
    kc, vc, q, k, v, cs, sn = _setup(cfg, 257, 11)
    q[:] = 0
    out, _, _ = orc.forward_from_projections(cfg, kc, vc, q, k, v, 0, 257, rope_cos=cs, rope_sin=sn)
    mean = vc[:258].astype(np.float64).mean(axis=0).reshape(8, 128)
    np.testing.assert_allclose(out.reshape(24, 128), np.repeat(mean, 3, axis=0), atol=2e-6)


def test_dominant_score_selects_row_and_gqa_mapping():
    Hq, Hkv, D = 8, 2, 64
    cfg = orc.OracleConfig(Hq, Hkv, D, 64)
    kc, vc, q, k, v, cs, sn = _setup(cfg, 40, 12)
    # no RoPE so that K rows line up with q directly
    q = np.zeros(Hq * D, F32); q[::D] = 1.0  # every head looks along dim 0
    kc[:40] = 0; k[:] = 0
    kc[13, 0] = 1000.0         # kv head 0 strongly prefers t=13
    kc[29, D] = 1000.0         # kv head 1 strongly prefers t=29
    out, _, _ = orc.forward_from_projections(cfg, kc, vc, q, k, v, 0, 40)
    o = out.reshape(Hq, D)
    for h in range(Hq):
        kh = h // (Hq // Hkv)
        t = 13 if kh == 0 else 29
        np.testing.assert_allclose(o[h], vc[t, kh * D:(kh + 1) * D], atol=1e-5)


def test_gqa_heads_read_their_own_kv_head():
    Hq, Hkv, D = 12, 4, 64
    cfg = orc.OracleConfig(Hq, Hkv, D, 32)
    kc, vc, q, k, v, cs, sn = _setup(cfg, 20, 13)
    for kh in range(Hkv):
        vc[:, kh * D:(kh + 1) * D] = kh + 1
        v[kh * D:(kh + 1) * D] = kh + 1
    out, _, _ = orc.forward_from_projections(cfg, kc, vc, q, k, v, 0, 20, rope_cos=cs, rope_sin=sn)
    o = out.reshape(Hq, D)
    for h in range(Hq):
        np.testing.assert_allclose(o[h], h // 3 + 1, rtol=1e-6)


@pytest.mark.parametrize("shape", [(4, 1, 256, 2), (32, 8, 64, 4), (16, 8, 128, 0), (24, 8, 128, 0)])
@pytest.mark.parametrize("qk_norm", [False, True])
def test_layer_call_matches_float64_brute_force(shape, qk_norm):
    Hq, Hkv, D, rtype = shape
    pos = 63
    cfg = orc.OracleConfig(Hq, Hkv, D, 64, rope_type=rtype, norm_eps=1e-6)
    kc, vc, q, k, v, cs, sn = _setup(cfg, pos, 14, k_scale=0.5, theta=1e6)
    rng = np.random.default_rng(15)
    qw = rng.uniform(0.5, 1.5, D).astype(F32) if qk_norm else None
    kw = rng.uniform(0.5, 1.5, D).astype(F32) if qk_norm else None
    kc0 = kc.copy(); vc0 = vc.copy()
    out, q2, k2 = orc.forward_from_projections(cfg, kc, vc, q, k, v, 0, pos, qnorm_w=qw,
                                               knorm_w=kw, rope_cos=cs, rope_sin=sn)
    # float64 chain: norm -> rotate -> append -> softmax attention
    qq = rm.rms_norm_heads(q, qw, Hq, D, 1e-6) if qk_norm else q.astype(np.float64)
    kk = rm.rms_norm_heads(k, kw, Hkv, D, 1e-6) if qk_norm else k.astype(np.float64)
    ang = rm.rope_angles(D, pos, float(F32(1e6)))
    qq = rm.rope_rotate(qq, Hq, D, D, rtype, ang)
    kk = rm.rope_rotate(kk, Hkv, D, D, rtype, ang)
    np.testing.assert_allclose(q2, qq, atol=2e-5)
    np.testing.assert_allclose(k2, kk, atol=2e-5)
    K = kc0.astype(np.float64); V = vc0.astype(np.float64)
    K[pos] = kk; V[pos] = v
    want = rm.attention(qq, K, V, Hq, Hkv, D, 0, pos, 1 / np.sqrt(D))
    rm.assert_close(out, want, atol=2e-5, rtol=1e-4, what="oracle vs fp64")
    # append: row pos holds the rotated k / raw v bit-for-bit, nothing else changed
    assert np.array_equal(kc[pos], k2) and np.array_equal(vc[pos], v)
    kc[pos] = kc0[pos]; vc[pos] = vc0[pos]
    assert np.array_equal(kc, kc0) and np.array_equal(vc, vc0)


def test_flash_equals_two_pass():
    cfg = orc.OracleConfig(24, 8, 128, 1100)
    kc, vc, q, k, v, cs, sn = _setup(cfg, 1023, 16, k_scale=0.5)
    a, _, _ = orc.forward_from_projections(cfg, kc.copy(), vc.copy(), q, k, v, 0, 1023,
                                           rope_cos=cs, rope_sin=sn)
    b, _, _ = orc.forward_from_projections(cfg, kc.copy(), vc.copy(), q, k, v, 0, 1023,
                                           rope_cos=cs, rope_sin=sn, use_flash=True)
    np.testing.assert_allclose(a, b, atol=2e-6)


def test_threads_do_not_change_results():
    cfg = orc.OracleConfig(24, 8, 128, 600)
    kc, vc, q, k, v, cs, sn = _setup(cfg, 511, 17)
    a, _, _ = orc.forward_from_projections(cfg, kc.copy(), vc.copy(), q, k, v, 0, 511,
                                           rope_cos=cs, rope_sin=sn, n_threads=1)
    b, _, _ = orc.forward_from_projections(cfg, kc.copy(), vc.copy(), q, k, v, 0, 511,
                                           rope_cos=cs, rope_sin=sn, n_threads=4)
    assert np.array_equal(a, b)


def test_softcap_matches_float64():
    cfg = orc.OracleConfig(8, 2, 64, 100, softcap=5.0)
    kc, vc, q, k, v, cs, sn = _setup(cfg, 80, 18, k_scale=3.0)
    kc0 = kc.copy(); vc0 = vc.copy()
    out, q2, k2 = orc.forward_from_projections(cfg, kc, vc, q, k, v, 0, 80)
    K = kc0.astype(np.float64); V = vc0.astype(np.float64); K[80] = k; V[80] = v
    want = rm.attention(q, K, V, 8, 2, 64, 0, 80, 1 / 8.0, softcap=5.0)
    rm.assert_close(out, want, atol=2e-5, rtol=1e-4, what="softcap")


@pytest.mark.parametrize("pos", [100, 510, 511, 512, 513, 900])
def test_sliding_window_boundaries(pos):
    W = 512
    cfg = orc.OracleConfig(4, 1, 256, 1024, sliding_window=W, arch=orc.ARCH_GEMMA3)
    start = max(0, pos - W + 1)
    assert orc.start_pos(cfg, 0, pos) == start          # local layer
    assert orc.start_pos(cfg, 5, pos) == 0              # global layer (5 % 6 == 5)
    kc, vc, q, k, v, cs, sn = _setup(cfg, pos, 19)
    vc_poison = vc.copy(); vc_poison[:start] = 1e6       # rows outside the window
    a, _, _ = orc.forward_from_projections(cfg, kc.copy(), vc.copy(), q, k, v, 0, pos)
    b, _, _ = orc.forward_from_projections(cfg, kc.copy(), vc_poison, q, k, v, 0, pos)
    assert np.array_equal(a, b)
    K = kc.astype(np.float64); V = vc.astype(np.float64); K[pos] = k; V[pos] = v
    want = rm.attention(q, K, V, 4, 1, 256, start, pos, 1 / 16.0)
    rm.assert_close(a, want, atol=2e-5, rtol=1e-4, what="window")


def test_nope_layer_skips_rotation():
    cfg = orc.OracleConfig(8, 2, 64, 32, no_rope_interval=4)
    kc, vc, q, k, v, cs, sn = _setup(cfg, 10, 20)
    _, q3, k3 = orc.forward_from_projections(cfg, kc.copy(), vc.copy(), q, k, v, 3, 10,
                                             rope_cos=cs, rope_sin=sn)
    assert np.array_equal(q3, q) and np.array_equal(k3, k)
    _, q2, _ = orc.forward_from_projections(cfg, kc.copy(), vc.copy(), q, k, v, 2, 10,
                                            rope_cos=cs, rope_sin=sn)
    assert not np.array_equal(q2, q)


def test_prefill_equals_sequential_decode_calls():
    cfg = orc.OracleConfig(8, 2, 64, 64)
    rng = np.random.default_rng(21)
    P = 20
    q = rng.standard_normal((P, 8 * 64)).astype(F32)
    k = rng.standard_normal((P, 128)).astype(F32)
    v = rng.standard_normal((P, 128)).astype(F32)
    cs, sn = orc.rope_tables(64, 64, 5e5)
    kc1 = np.zeros((64, 128), F32); vc1 = np.zeros((64, 128), F32)
    out = orc.prefill_sequential(cfg, kc1, vc1, q, k, v, 0, 0, rope_cos=cs, rope_sin=sn)
    kc2 = np.zeros((64, 128), F32); vc2 = np.zeros((64, 128), F32)
    for i in range(P):
        o, _, _ = orc.forward_from_projections(cfg, kc2, vc2, q[i], k[i], v[i], 0, i,
                                               rope_cos=cs, rope_sin=sn)
        assert np.array_equal(out[i], o)
    assert np.array_equal(kc1, kc2) and np.array_equal(vc1, vc2)


# ----------------------------------------------------------------- Q8_0 KV cache mode
def _round_half_up_f64(y):
    """Math.round(float): floor(y + 0.5) computed exactly in float64."""
    return np.floor(np.float64(np.float32(y)) + 0.5)


def test_q8_round_half_up_matches_exact_definition():
    edges = [0.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -127.5, 0.49999997, -0.49999997,
             0.50000006, -0.50000006, 1e-30, -1e-30, 127.0, -128.0, 3.4999998, -3.4999998]
    for y in edges:
        assert orc.round_half_up(y) == _round_half_up_f64(y), y
    rng = np.random.default_rng(30)
    ys = np.concatenate([rng.uniform(-130, 130, 4000), np.arange(-128, 128) + 0.5]).astype(F32)
    got = np.array([orc.round_half_up(y) for y in ys])
    assert np.array_equal(got, _round_half_up_f64(ys))


def test_q8_quantize_closed_form_and_round_trip():
    rng = np.random.default_rng(31)
    x = (rng.standard_normal(256) * rng.uniform(0.01, 10, 8).repeat(32)).astype(F32)
    q, sc = orc.q8_quantize(x)
    xb = x.reshape(8, 32)
    want_scale = (np.abs(xb).max(axis=1) / F32(127.0)).astype(F32)     # IEEE float32 division
    assert np.array_equal(sc, want_scale)
    inv = (F32(1.0) / want_scale).astype(F32)
    y = (xb * inv[:, None]).astype(F32)
    want_q = np.clip(_round_half_up_f64(y), -128, 127).astype(np.int8).reshape(-1)
    assert np.array_equal(q, want_q)
    # every block reaches +-127 at its largest |x|; dequantisation error <= scale/2 (+ulp)
    assert np.all(np.abs(q.reshape(8, 32)).max(axis=1) == 127)
    deq = q.reshape(8, 32).astype(np.float64) * sc[:, None]
    assert np.all(np.abs(deq - xb) <= sc[:, None] * 0.5 * (1 + 1e-5))
    # an all-zero block has scale 0 and zero quants
    q0, s0 = orc.q8_quantize(np.zeros(32, F32))
    assert s0[0] == 0 and not q0.any()


def test_q8_dot_and_saxpy_match_float64_on_dequantised_values():
    rng = np.random.default_rng(32)
    for D in (64, 128, 256):
        k = rng.standard_normal(D).astype(F32)
        qv = rng.standard_normal(D).astype(F32)
        kq, ks = orc.q8_quantize(k)
        deq = kq.astype(np.float64) * np.repeat(ks, 32)
        assert abs(float(orc.q8_dot(qv, kq, ks)) - float(qv.astype(np.float64) @ deq)) < 1e-4
        out0 = rng.standard_normal(D).astype(F32)
        got = orc.q8_saxpy(0.37, kq, ks, out0)
        np.testing.assert_allclose(got, out0 + np.float32(0.37) * deq, atol=2e-6)
        # per-block unfused order: the scalar path's exact float result
        acc = np.float32(0)
        for b in range(D // 32):
            a = np.float32(0)
            for i in range(32):
                a = np.float32(a + np.float32(qv[32 * b + i] * np.float32(kq[32 * b + i])))
            acc = np.float32(acc + np.float32(a * ks[b]))
        assert orc.q8_dot(qv, kq, ks) == acc


@pytest.mark.parametrize("shape", [(32, 8, 64), (24, 8, 128), (4, 1, 256)])
def test_q8_layer_call_matches_float64_on_dequantised_cache(shape):
    Hq, Hkv, D = shape
    S, pos = 80, 70
    cfg = orc.OracleConfig(Hq, Hkv, D, S, rope_type=0)
    rng = np.random.default_rng(33)
    kv = Hkv * D
    kf = rng.standard_normal((S, kv)).astype(F32)
    vf = rng.standard_normal((S, kv)).astype(F32)
    kq = np.zeros((S, kv), np.int8); vq = np.zeros((S, kv), np.int8)
    ks = np.zeros((S, kv // 32), F32); vs = np.zeros((S, kv // 32), F32)
    for t in range(pos):
        kq[t], ks[t] = orc.q8_quantize(kf[t])
        vq[t], vs[t] = orc.q8_quantize(vf[t])
    q = rng.standard_normal(Hq * D).astype(F32)
    k = rng.standard_normal(kv).astype(F32)
    v = rng.standard_normal(kv).astype(F32)
    cs, sn = orc.rope_tables(D, S, 5e5)
    kq0, ks0, vq0, vs0 = kq.copy(), ks.copy(), vq.copy(), vs.copy()
    out, q2, k2 = orc.forward_from_projections_q8(cfg, kq, ks, vq, vs, q, k, v, 0, pos,
                                                  rope_cos=cs, rope_sin=sn)
    # the appended row is the quantisation of the rotated k and of v
    qk_row, sk_row = orc.q8_quantize(k2)
    qv_row, sv_row = orc.q8_quantize(v)
    assert np.array_equal(kq[pos], qk_row) and np.array_equal(ks[pos], sk_row)
    assert np.array_equal(vq[pos], qv_row) and np.array_equal(vs[pos], sv_row)
    kq[pos] = kq0[pos]; ks[pos] = ks0[pos]; vq[pos] = vq0[pos]; vs[pos] = vs0[pos]
    assert np.array_equal(kq, kq0) and np.array_equal(vs, vs0)
    K = (kq0.astype(np.float64).reshape(S, -1, 32) * ks0[:, :, None]).reshape(S, kv)
    V = (vq0.astype(np.float64).reshape(S, -1, 32) * vs0[:, :, None]).reshape(S, kv)
    K[pos] = (qk_row.astype(np.float64).reshape(-1, 32) * sk_row[:, None]).reshape(-1)
    V[pos] = (qv_row.astype(np.float64).reshape(-1, 32) * sv_row[:, None]).reshape(-1)
    want = rm.attention(q2, K, V, Hq, Hkv, D, 0, pos, 1 / np.sqrt(D))
    rm.assert_close(out, want, atol=2e-5, rtol=1e-4, what="q8 layer-call")
    b, _, _ = orc.forward_from_projections_q8(cfg, kq0.copy(), ks0.copy(), vq0.copy(), vs0.copy(),
                                              q, k, v, 0, pos, rope_cos=cs, rope_sin=sn,
                                              use_flash=True)
    np.testing.assert_allclose(out, b, atol=2e-6)


# ----------------------------------------- Q8_0, the 8-lane SimdQ8KvOps contract (AVX2 hosts)
def _fma32(a, b, c):
    """float32 fma: a*b + c exact in float64 (a is an int8 quant or a product of <= 32
    significant bits, magnitudes kept moderate by the callers), rounded once to float32."""
    return np.float32(np.float64(a) * np.float64(b) + np.float64(c))


def _q8_prefill_setup(Hq, Hkv, D, S, pos0, P, mode, seed):
    """A Q8_0 cache with rows [0, pos0) quantised under `mode`, plus P tokens of q/k/v."""
    rng = np.random.default_rng(seed)
    kv = Hkv * D
    kq = np.zeros((S, kv), np.int8); vq = np.zeros((S, kv), np.int8)
    ks = np.zeros((S, kv // 32), F32); vs = np.zeros((S, kv // 32), F32)
    for t in range(pos0):
        kq[t], ks[t] = orc.q8_quantize(rng.standard_normal(kv).astype(F32), mode)
        vq[t], vs[t] = orc.q8_quantize(rng.standard_normal(kv).astype(F32), mode)
    q = rng.standard_normal((P, Hq * D)).astype(F32)
    k = rng.standard_normal((P, kv)).astype(F32)
    v = rng.standard_normal((P, kv)).astype(F32)
    return kq, ks, vq, vs, q, k, v


def _dequant(quants, scales):
    n, kv = quants.shape
    return (quants.astype(np.float64).reshape(n, -1, 32) * scales[:, :, None]).reshape(n, kv)


@pytest.mark.parametrize("mode", [orc.Q8_SCALAR, orc.Q8_SIMD8])
def test_q8_prefill_first_token_output_is_its_dequantised_v(mode):
    # one attended row: weight 1, so out = scale * quant of the row just appended, exactly
    Hq, Hkv, D, S = 8, 2, 64, 16
    cfg = orc.OracleConfig(Hq, Hkv, D, S, rope_type=0)
    kq, ks, vq, vs, q, k, v = _q8_prefill_setup(Hq, Hkv, D, S, 0, 1, mode, 50)
    cs, sn = orc.rope_tables(D, S, 5e5)
    out = orc.prefill_sequential_q8(cfg, kq, ks, vq, vs, q, k, v, 0, 0, rope_cos=cs,
                                    rope_sin=sn, mode=mode)
    qv, sv = orc.q8_quantize(v[0], mode)
    row = (qv.astype(F32).reshape(-1, 32) * sv[:, None]).reshape(Hkv, D)
    assert np.array_equal(out.reshape(Hq, D), np.repeat(row, Hq // Hkv, axis=0))


@pytest.mark.parametrize("mode", [orc.Q8_SCALAR, orc.Q8_SIMD8])
def test_q8_prefill_appends_quantised_rotated_rows_at_their_positions(mode):
    Hq, Hkv, D, S, pos0, P = 8, 2, 64, 40, 9, 12
    cfg = orc.OracleConfig(Hq, Hkv, D, S, rope_type=0)
    kq, ks, vq, vs, q, k, v = _q8_prefill_setup(Hq, Hkv, D, S, pos0, P, mode, 51)
    before = [a.copy() for a in (kq, ks, vq, vs)]
    cs, sn = orc.rope_tables(D, S, 5e5)
    orc.prefill_sequential_q8(cfg, kq, ks, vq, vs, q, k, v, 0, pos0, rope_cos=cs, rope_sin=sn,
                              mode=mode)
    for i in range(P):
        kr = orc.rope_apply_all(k[i], Hkv, D, D, 0, cs, sn, pos0 + i)
        want_kq, want_ks = orc.q8_quantize(kr, mode)
        want_vq, want_vs = orc.q8_quantize(v[i], mode)
        assert np.array_equal(kq[pos0 + i], want_kq) and np.array_equal(ks[pos0 + i], want_ks)
        assert np.array_equal(vq[pos0 + i], want_vq) and np.array_equal(vs[pos0 + i], want_vs)
    for a, b in zip((kq, ks, vq, vs), before):   # rows outside [pos0, pos0 + P) untouched
        assert np.array_equal(a[:pos0], b[:pos0]) and np.array_equal(a[pos0 + P:], b[pos0 + P:])


@pytest.mark.parametrize("mode", [orc.Q8_SCALAR, orc.Q8_SIMD8])
def test_q8_prefill_uniform_scores_average_each_tokens_causal_rows(mode):
    # q = 0: every score is 0, so token i's output is the mean of dequantised V rows
    # 0 .. pos0 + i (its own row included, later rows excluded)
    Hq, Hkv, D, S, pos0, P = 6, 2, 64, 48, 17, 9
    cfg = orc.OracleConfig(Hq, Hkv, D, S, rope_type=0)
    kq, ks, vq, vs, q, k, v = _q8_prefill_setup(Hq, Hkv, D, S, pos0, P, mode, 52)
    q[:] = 0
    cs, sn = orc.rope_tables(D, S, 5e5)
    out = orc.prefill_sequential_q8(cfg, kq, ks, vq, vs, q, k, v, 0, pos0, rope_cos=cs,
                                    rope_sin=sn, mode=mode)
    V = _dequant(vq, vs)
    for i in range(P):
        mean = V[:pos0 + i + 1].mean(axis=0).reshape(Hkv, D)
        np.testing.assert_allclose(out[i].reshape(Hq, D), np.repeat(mean, Hq // Hkv, axis=0),
                                   atol=2e-6)


def test_q8_simd8_quantize_truncates_toward_zero():
    rng = np.random.default_rng(40)
    x = (rng.standard_normal(512) * rng.uniform(0.01, 10, 16).repeat(32)).astype(F32)
    q, sc = orc.q8_quantize(x, orc.Q8_SIMD8)
    qs, scs = orc.q8_quantize(x)
    assert np.array_equal(sc, scs)                                   # same scale as the scalar path
    inv = (F32(1.0) / sc).astype(F32)
    y = (x.reshape(16, 32) * inv[:, None]).astype(F32)
    assert np.array_equal(q, np.clip(np.trunc(y), -128, 127).astype(np.int8).reshape(-1))
    assert (q != qs).any()                                           # the contracts differ
    # hand cases: scale 1 (max 127), so y = x exactly
    blk = np.array([127.0, -127.0, 2.7, -2.7, 0.5, -0.5, 126.99, -126.99] + [0.0] * 24, F32)
    qb, sb = orc.q8_quantize(blk, orc.Q8_SIMD8)
    assert sb[0] == 1.0 and list(qb[:8]) == [127, -127, 2, -2, 0, 0, 126, -126]
    qr, _ = orc.q8_quantize(blk)
    assert list(qr[:8]) == [127, -127, 3, -3, 1, 0, 127, -127]       # Math.round: ties up


def test_q8_simd8_dot_and_saxpy_follow_lane_fma_order():
    rng = np.random.default_rng(41)
    for D in (64, 128, 256):
        qv = rng.standard_normal(D).astype(F32)
        kq = rng.integers(-128, 128, D).astype(np.int8)
        ks = rng.uniform(0.001, 0.05, D // 32).astype(F32)
        total = F32(0)
        for b in range(D // 32):
            lane = [F32(0)] * 8
            for c in range(0, 32, 8):
                for l in range(8):
                    i = 32 * b + c + l
                    lane[l] = _fma32(kq[i], qv[i], lane[l])
            s = lane[0]
            for l in range(1, 8):
                s = F32(s + lane[l])
            total = F32(total + F32(s * ks[b]))
        assert orc.q8_dot(qv, kq, ks, orc.Q8_SIMD8) == total
        out0 = rng.standard_normal(D).astype(F32)
        got = orc.q8_saxpy(0.37, kq, ks, out0, orc.Q8_SIMD8)
        w = np.repeat((F32(0.37) * ks).astype(F32), 32)
        want = np.array([_fma32(kq[i], w[i], out0[i]) for i in range(D)], F32)
        assert np.array_equal(got, want)
    # FMA witness: lane 0 sees quant -3 x q 1 (chunk 0), then quant 3 x q (1 + 2^-23)
    # (chunk 1).  Fused: 3*(1 + 2^-23) - 3 = 3*2^-23 exactly; an unfused product rounds
    # 3 + 3*2^-23 to a multiple of 2^-22 first, leaving 2^-22 or 2^-21.
    qv = np.zeros(32, F32)
    kq = np.zeros(32, np.int8)
    qv[0], kq[0] = 1.0, -3
    qv[8], kq[8] = F32(1 + 2.0 ** -23), 3
    assert orc.q8_dot(qv, kq, np.ones(1, F32), orc.Q8_SIMD8) == F32(3 * 2.0 ** -23)
    assert orc.q8_dot(qv, kq, np.ones(1, F32)) != F32(3 * 2.0 ** -23)   # scalar: unfused


def test_q8_simd8_layer_call():
    Hq, Hkv, D, S, pos = 24, 8, 128, 80, 70
    cfg = orc.OracleConfig(Hq, Hkv, D, S, rope_type=0)
    rng = np.random.default_rng(42)
    kv = Hkv * D
    kq = np.zeros((S, kv), np.int8); vq = np.zeros((S, kv), np.int8)
    ks = np.zeros((S, kv // 32), F32); vs = np.zeros((S, kv // 32), F32)
    for t in range(pos):
        kq[t], ks[t] = orc.q8_quantize(rng.standard_normal(kv).astype(F32), orc.Q8_SIMD8)
        vq[t], vs[t] = orc.q8_quantize(rng.standard_normal(kv).astype(F32), orc.Q8_SIMD8)
    q = rng.standard_normal(Hq * D).astype(F32)
    k = rng.standard_normal(kv).astype(F32)
    v = rng.standard_normal(kv).astype(F32)
    cs, sn = orc.rope_tables(D, S, 5e5)
    kq0, ks0, vq0, vs0 = kq.copy(), ks.copy(), vq.copy(), vs.copy()
    out, q2, k2 = orc.forward_from_projections_q8(cfg, kq, ks, vq, vs, q, k, v, 0, pos,
                                                  rope_cos=cs, rope_sin=sn, mode=orc.Q8_SIMD8)
    qk_row, sk_row = orc.q8_quantize(k2, orc.Q8_SIMD8)
    qv_row, sv_row = orc.q8_quantize(v, orc.Q8_SIMD8)
    assert np.array_equal(kq[pos], qk_row) and np.array_equal(ks[pos], sk_row)
    assert np.array_equal(vq[pos], qv_row) and np.array_equal(vs[pos], sv_row)
    K = (kq.astype(np.float64).reshape(S, -1, 32) * ks[:, :, None]).reshape(S, kv)
    V = (vq.astype(np.float64).reshape(S, -1, 32) * vs[:, :, None]).reshape(S, kv)
    want = rm.attention(q2, K, V, Hq, Hkv, D, 0, pos, 1 / np.sqrt(D))
    rm.assert_close(out, want, atol=2e-5, rtol=1e-4, what="q8 simd8 layer-call")
    # the scalar contract stores a different row for the same input
    kq1, ks1, vq1, vs1 = kq0.copy(), ks0.copy(), vq0.copy(), vs0.copy()
    orc.forward_from_projections_q8(cfg, kq1, ks1, vq1, vs1, q, k, v, 0, pos, rope_cos=cs,
                                    rope_sin=sn)
    assert not np.array_equal(kq1[pos], kq[pos])


# ------------------------------------------- attention variants: GPT-OSS sinks, Qwen3.5 gate
def test_softmax_with_sink_closed_forms():
    x = np.array([0.0, 0.0, 0.0, 0.0], F32)
    for sink in (-3.0, 0.0, 2.0):
        got = orc.softmax_with_sink(x, sink)
        want = 1.0 / (4.0 + np.exp(sink))
        np.testing.assert_allclose(got, np.full(4, want), rtol=2e-7)
    # a very negative sink is the plain softmax, bit for bit (same max, same sum order)
    rng = np.random.default_rng(50)
    y = rng.standard_normal(300).astype(F32) * F32(3)
    assert np.array_equal(orc.softmax_with_sink(y, -1e30), orc.softmax(y))
    # a dominant sink takes (almost) all the mass; weights keep their ratios
    z = orc.softmax_with_sink(y, 60.0)
    assert z.sum() < 1e-15 and np.all(z >= 0)
    w = orc.softmax_with_sink(y, 1.5)
    e = np.exp(y.astype(np.float64) - max(y.max(), 1.5))
    np.testing.assert_allclose(w, e / (e.sum() + np.exp(1.5 - max(y.max(), 1.5))), rtol=2e-6)


@pytest.mark.parametrize("shape", [(24, 8, 128), (32, 8, 64), (8, 8, 64)])
def test_sinks_layer_call_matches_float64(shape):
    Hq, Hkv, D = shape
    pos = 90
    rng = np.random.default_rng(51)
    sinks = rng.uniform(-2, 4, Hq).astype(F32)
    cfg = orc.OracleConfig(Hq, Hkv, D, 128, sinks=sinks, attention_scale=0.11)
    kc, vc, q, k, v, cs, sn = _setup(cfg, pos, 52, k_scale=0.5)
    kc0, vc0 = kc.copy(), vc.copy()
    out, q2, k2 = orc.forward_from_projections(cfg, kc, vc, q, k, v, 0, pos, rope_cos=cs,
                                               rope_sin=sn)
    K = kc0.astype(np.float64); V = vc0.astype(np.float64)
    K[pos] = k2; V[pos] = v
    want = rm.attention(q2, K, V, Hq, Hkv, D, 0, pos, float(F32(0.11)), sinks=sinks)
    rm.assert_close(out, want, atol=2e-6, rtol=1e-5, what="sinks vs fp64")
    # the sinks shrink every head's weights: without them the output differs
    cfg0 = orc.OracleConfig(Hq, Hkv, D, 128, attention_scale=0.11)
    out0, _, _ = orc.forward_from_projections(cfg0, kc0.copy(), vc0.copy(), q, k, v, 0, pos,
                                              rope_cos=cs, rope_sin=sn)
    assert np.abs(out - out0).max() > 1e-3
    # q = 0: every score is 0, so head h's output is sum(V) / (n + exp(sink_h))
    cfgz = orc.OracleConfig(Hq, Hkv, D, 128, sinks=sinks)
    outz, _, _ = orc.forward_from_projections(cfgz, kc0.copy(), vc0.copy(), np.zeros_like(q), k,
                                              v, 0, pos)
    Vh = V.reshape(-1, Hkv, D)[:pos + 1].sum(0)
    g = Hq // Hkv
    wantz = np.stack([Vh[h // g] / (pos + 1 + np.exp(float(sinks[h]))) for h in range(Hq)])
    np.testing.assert_allclose(outz.reshape(Hq, D), wantz, atol=2e-6)
    # the flash loop has no sink form in the reference: with sinks the two-pass path runs
    b, _, _ = orc.forward_from_projections(cfg, kc0.copy(), vc0.copy(), q, k, v, 0, pos,
                                           rope_cos=cs, rope_sin=sn, use_flash=True)
    assert np.array_equal(b, out)


def test_sigmoid_gate_closed_forms():
    rng = np.random.default_rng(53)
    out = rng.standard_normal(512).astype(F32)
    assert np.array_equal(orc.sigmoid_gate(out, np.zeros(512, F32)), out * F32(0.5))
    assert np.array_equal(orc.sigmoid_gate(out, np.full(512, 200.0, F32)), out)
    assert not orc.sigmoid_gate(out, np.full(512, -200.0, F32)).any()
    g = rng.uniform(-8, 8, 512).astype(F32)
    want = out.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))
    np.testing.assert_allclose(orc.sigmoid_gate(out, g), want, rtol=3e-7, atol=1e-30)


def test_gated_layer_call_is_gate_times_plain_output():
    cfg = orc.OracleConfig(16, 4, 128, 64, rope_type=orc.ROPE_NEOX, norm_eps=1e-6)
    kc, vc, q, k, v, cs, sn = _setup(cfg, 40, 54, theta=1e7)
    gate = np.random.default_rng(55).uniform(-4, 4, 16 * 128).astype(F32)
    a, _, _ = orc.forward_from_projections(cfg, kc.copy(), vc.copy(), q, k, v, 0, 40,
                                           rope_cos=cs, rope_sin=sn)
    b, _, _ = orc.forward_from_projections(cfg, kc.copy(), vc.copy(), q, k, v, 0, 40,
                                           rope_cos=cs, rope_sin=sn, gate=gate)
    assert np.array_equal(b, orc.sigmoid_gate(a, gate))
    np.testing.assert_allclose(b, a.astype(np.float64) / (1 + np.exp(-gate.astype(np.float64))),
                               rtol=1e-6, atol=1e-30)


def test_gptoss_moe_engine_windows_even_layers():
    # Qwen3MoEInferenceEngine.java:280-286: even layers attend to the last W rows, odd layers
    # to all; Attention.isGlobalLayer's GPT-OSS rule is the opposite.
    moe = orc.OracleConfig(8, 2, 64, 600, sliding_window=128, arch=orc.ARCH_GPT_OSS_MOE)
    att = orc.OracleConfig(8, 2, 64, 600, sliding_window=128, arch=orc.ARCH_GPT_OSS)
    for layer in range(4):
        even = layer % 2 == 0
        assert orc.start_pos(moe, layer, 500) == (373 if even else 0)
        assert orc.start_pos(att, layer, 500) == (0 if even else 373)
        assert orc.start_pos(moe, layer, 100) == 0
    from llmplayer_amd import hip_forward_pass as hfp
    for layer in range(4):
        assert hfp.is_global_layer(hfp.ARCH_GPT_OSS, layer, expert_count=32) == (layer % 2 == 1)
        assert hfp.is_global_layer(hfp.ARCH_GPT_OSS, layer) == (layer % 2 == 0)


# ----------------------------------------------------------------- Gemma 4 attention layer
def test_rms_norm_seq_closed_forms_and_eps_inside_the_root():
    # constant c: sum of squares D*c^2 is exact, so r = 1/(float)sqrt(c^2 + eps) exactly
    for D, cval, eps in ((256, 3.0, 1e-6), (512, -0.75, 1e-6), (256, 2.0, 0.5)):
        x = np.full(D, cval, F32)
        got = orc.rms_norm_seq(x, None, eps)
        r = F32(1.0) / F32(np.sqrt(np.float64(F32(F32(cval * cval * D) / F32(D)) + F32(eps))))
        assert np.array_equal(got, np.full(D, F32(F32(cval) * r)))
    # eps = 0: scaling by a power of two leaves the normalised vector bit-identical
    rng = np.random.default_rng(70)
    x = rng.standard_normal(512).astype(F32)
    w = rng.uniform(0.5, 1.5, 512).astype(F32)
    assert np.array_equal(orc.rms_norm_seq(x, w, 0.0), orc.rms_norm_seq(x * F32(8.0), w, 0.0))


def test_rms_norm_seq_matches_float64_and_uses_the_sequential_order():
    rng = np.random.default_rng(71)
    differs = 0
    for D in (256, 512):
        for _ in range(8):
            x = (rng.standard_normal(D) * 3).astype(F32)
            w = rng.uniform(0.5, 1.5, D).astype(F32)
            got = orc.rms_norm_seq(x, w, 1e-6)
            want = rm.rms_norm_heads(x, w, 1, D, 1e-6)
            np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-7)
            ss = F32(0.0)                      # RMSNorm.java:26-30, one float at a time
            for v in x:
                ss = F32(ss + F32(v * v))
            r = F32(1.0) / F32(np.sqrt(np.float64(F32(ss / F32(D)) + F32(1e-6))))
            assert np.array_equal(got, (x * r) * w)
            differs += not np.array_equal(got, orc.per_head_norm(x, w, 1, D, 1e-6))
    assert differs > 0   # the 8-lane FMA order of SimdVectorOps gives other last bits


def _g4_tables(D, S, theta, factors=None):
    return orc.rope_tables(D, S, theta, freq_factors=factors)


def _g4_float64(q, k, v, kcache, vcache, qw, kw, cs, sn, Hq, Hkv, D, pos, start, eps):
    """Gemma 4 attention half in float64: QK-norm, V-norm, NORMAL RoPE by the tables,
    scale-1 softmax attention over rows [start, pos] (row pos from k, v when given)."""
    def rope(x, nh):
        x = np.asarray(x, np.float64).reshape(nh, D).copy()
        c, s = cs[pos].astype(np.float64), sn[pos].astype(np.float64)
        a, b = x[:, 0::2].copy(), x[:, 1::2].copy()
        x[:, 0::2], x[:, 1::2] = a * c - b * s, a * s + b * c
        return x.reshape(-1)
    qn = rope(rm.rms_norm_heads(q, qw, Hq, D, eps), Hq)
    K = kcache.astype(np.float64).copy()
    V = vcache.astype(np.float64).copy()
    if k is not None:
        K[pos] = rope(rm.rms_norm_heads(k, kw, Hkv, D, eps), Hkv)
        V[pos] = rm.rms_norm_heads(v, np.ones(D), Hkv, D, eps)
    return rm.attention(qn, K, V, Hq, Hkv, D, start, pos, 1.0), K[pos], V[pos]


@pytest.mark.parametrize("D,is_swa", [(256, True), (512, False)])
def test_gemma4_layer_matches_float64(D, is_swa):
    Hq, Hkv, S, W, pos = 8, 2, 96, 40, 77
    cfg = orc.OracleConfig(Hq, Hkv, D, S, rope_type=0, norm_eps=1e-6, sliding_window=W)
    rng = np.random.default_rng(72 + D)
    kc = np.zeros((S, Hkv * D), F32); vc = np.zeros((S, Hkv * D), F32)
    kc[:pos] = rng.standard_normal((pos, Hkv * D)).astype(F32)
    vc[:pos] = rng.standard_normal((pos, Hkv * D)).astype(F32)
    q = rng.standard_normal(Hq * D).astype(F32) * F32(4)
    k = rng.standard_normal(Hkv * D).astype(F32) * F32(4)
    v = rng.standard_normal(Hkv * D).astype(F32) * F32(4)
    qw = rng.uniform(0.5, 1.5, D).astype(F32)
    kw = rng.uniform(0.5, 1.5, D).astype(F32)
    factors = None if is_swa else np.linspace(1.0, 4.0, D // 2).astype(F32)
    cs, sn = _g4_tables(D, S, 1e4 if is_swa else 1e6, factors)
    kc0 = kc.copy()
    out, q2, k2, v2 = orc.forward_gemma4(cfg, kc, vc, q, k, v, pos, is_swa, qnorm_w=qw,
                                         knorm_w=kw, rope_cos=cs, rope_sin=sn)
    start = pos - W + 1 if is_swa else 0
    want, krow, vrow = _g4_float64(q, k, v, kc0, vc, qw, kw, cs, sn, Hq, Hkv, D, pos, start, 1e-6)
    rm.assert_close(out, want, atol=2e-5, rtol=1e-4, what=f"gemma4 D={D}")
    np.testing.assert_allclose(kc[pos], krow, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(vc[pos], vrow, rtol=1e-5, atol=1e-6)
    assert np.array_equal(kc[pos], k2) and np.array_equal(vc[pos], v2)
    assert np.array_equal(np.delete(kc, pos, 0), np.delete(kc0, pos, 0))
    # the stored V row is the weightless sequential norm of v, K the weighted one then RoPE
    for h in range(Hkv):
        assert np.array_equal(v2[h * D:(h + 1) * D], orc.rms_norm_seq(v[h * D:(h + 1) * D], None, 1e-6))


def test_gemma4_shared_layer_reads_the_source_cache_and_appends_nothing():
    Hq, Hkv, D, S, pos = 4, 1, 256, 64, 50
    cfg = orc.OracleConfig(Hq, Hkv, D, S, rope_type=0, norm_eps=1e-6, sliding_window=20)
    rng = np.random.default_rng(73)
    kc = rng.standard_normal((S, D)).astype(F32)
    vc = rng.standard_normal((S, D)).astype(F32)
    q = rng.standard_normal(Hq * D).astype(F32)
    qw = rng.uniform(0.5, 1.5, D).astype(F32)
    cs, sn = _g4_tables(D, S, 1e4)
    kc0, vc0 = kc.copy(), vc.copy()
    out, _, _, _ = orc.forward_gemma4(cfg, kc, vc, q, None, None, pos, True, qnorm_w=qw,
                                      rope_cos=cs, rope_sin=sn)
    assert np.array_equal(kc, kc0) and np.array_equal(vc, vc0)
    want, _, _ = _g4_float64(q, None, None, kc0, vc0, qw, None, cs, sn, Hq, Hkv, D, pos,
                             pos - 19, 1e-6)
    rm.assert_close(out, want, atol=2e-5, rtol=1e-4, what="gemma4 shared layer")


@pytest.mark.parametrize("pos", [18, 19, 20, 33])
def test_gemma4_window_boundaries_by_uniform_scores(pos):
    # q = 0: every score is 0, so the output is the mean of V over the attended rows
    Hq, Hkv, D, S, W = 2, 1, 256, 40, 20
    cfg = orc.OracleConfig(Hq, Hkv, D, S, rope_type=0, norm_eps=1e-6, sliding_window=W)
    rng = np.random.default_rng(74)
    kc = rng.standard_normal((S, D)).astype(F32)
    vc = rng.standard_normal((S, D)).astype(F32)
    q = np.zeros(Hq * D, F32)
    for is_swa in (True, False):
        out, _, _, _ = orc.forward_gemma4(cfg, kc.copy(), vc.copy(), q, None, None, pos, is_swa)
        start = max(0, pos - W + 1) if is_swa else 0
        mean = vc[start:pos + 1].astype(np.float64).mean(axis=0)
        np.testing.assert_allclose(out.reshape(Hq, D), np.tile(mean, (Hq, 1)), atol=2e-6)
