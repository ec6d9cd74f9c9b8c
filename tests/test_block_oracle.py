"""Pins the oracle's attention-block restatement (oracle/block_oracle.c) before it is trusted.

Dequantisation is checked against tests/ggml_pack.py, which packs each format from its layout
in the opposite direction and computes the values in float32 independently; Float16 against
numpy; the matmul and RMSNorm against float64; the whole block against a float64 chain and
against identities a slip would break (zero output projection leaves the residual, merged
and separate QKV agree, the bias and residual scale enter once)."""
import numpy as np
import pytest

from oracle import oracle as orc
from tests import ggml_pack as gp
from tests import refmath as rm

F32 = np.float32
TYPES = [gp.GGML_F32, gp.GGML_F16, gp.GGML_BF16, gp.GGML_Q8_0, gp.GGML_Q4_0, gp.GGML_Q4_K,
         gp.GGML_Q6_K, gp.GGML_Q5_0, gp.GGML_Q3_K, gp.GGML_Q5_K, gp.GGML_IQ4_NL, gp.GGML_IQ4_XS,
         gp.GGML_MXFP4, gp.GGML_Q5_1, gp.GGML_Q2_K, gp.GGML_IQ3_XXS, gp.GGML_IQ3_S, gp.GGML_IQ2_S]
NAMES = {0: "f32", 1: "f16", 30: "bf16", 8: "q8_0", 2: "q4_0", 12: "q4_k", 14: "q6_k", 6: "q5_0",
         11: "q3_k", 13: "q5_k", 20: "iq4_nl", 23: "iq4_xs", 39: "mxfp4", 7: "q5_1", 10: "q2_k",
         18: "iq3_xxs", 21: "iq3_s", 22: "iq2_s"}
IQ_TYPES = [gp.GGML_IQ3_XXS, gp.GGML_IQ3_S, gp.GGML_IQ2_S]


def test_f16_conversion_matches_ieee_half_for_every_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(F32)
    got = np.array([orc.f16_to_f32(b) for b in bits], F32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("t", TYPES, ids=[NAMES[t] for t in TYPES])
def test_dequantised_values_match_the_packer(t):
    rng = np.random.default_rng(80 + t)
    rows, cols = 5, 512
    wb, vals = gp.random_weights(t, rows, cols, rng)
    got = orc.dequant_rows(t, wb, rows, cols)
    assert np.array_equal(got.view(np.uint32), vals.view(np.uint32))


def test_q4_0_nibbles_interleave_within_a_block():
    # Q4_0FloatTensor: element 2i is the low nibble of byte i, element 2i+1 the high nibble
    q = np.full((1, 32), 8, np.int64)
    q[0, 5] = 9                                   # element 5: byte 2, high nibble
    wb, _ = gp.pack_q4_0(np.array([[0x3C00]], np.uint16), q)   # d = 1.0
    assert wb[0, 2 + 2] == (8 | (9 << 4))
    got = orc.dequant_rows(gp.GGML_Q4_0, wb, 1, 32)[0]
    assert got[5] == 1.0 and np.count_nonzero(got) == 1


def test_q4_k_sub_block_scales_and_mins_are_distinct():
    # every sub-block gets its own (scale, min), with the top bits of sub-blocks 4..7 set, so
    # a wrong index or bit position in the 12-byte unpacking moves some value
    sc = np.array([[[1, 2, 3, 4, 49, 50, 61, 63]]])
    mn = np.array([[[5, 6, 7, 8, 33, 40, 52, 62]]])
    q = np.tile(np.arange(32) % 16, 8).reshape(1, 256)
    wb, vals = gp.pack_q4_k(np.array([[0x3C00]], np.uint16), np.array([[0x3800]], np.uint16), sc, mn, q)
    got = orc.dequant_rows(gp.GGML_Q4_K, wb, 1, 256)[0]
    assert np.array_equal(got, vals[0])
    for s in range(8):
        seg = got[32 * s:32 * s + 32]
        # d = 1, dmin = 0.5: value = sc*q - 0.5*m
        assert np.array_equal(seg, (sc[0, 0, s] * (np.arange(32) % 16) - 0.5 * mn[0, 0, s]).astype(F32))


def test_q6_k_quarters_take_their_own_scales():
    sc = np.arange(1, 17, dtype=np.int8).reshape(1, 1, 16) * np.int8(3) - np.int8(20)
    q = np.full((1, 256), 33, np.int64)           # (q - 32) = 1: value = d * scale
    wb, vals = gp.pack_q6_k(np.array([[0x3C00]], np.uint16), sc, q)
    got = orc.dequant_rows(gp.GGML_Q6_K, wb, 1, 256)[0]
    assert np.array_equal(got, vals[0])
    for e in (0, 15, 16, 31, 32, 64, 96, 127, 128, 144, 200, 255):
        h, r = divmod(e, 128)
        c, l = divmod(r, 32)
        assert got[e] == sc[0, 0, 8 * h + l // 16 + 2 * c]


def test_q5_0_split_nibbles_and_fifth_bit():
    # element i < 16: low nibble of byte i; element 16 + i: its high nibble; bit 4 of element
    # i is bit i of qh; value (q - 16) * d
    q = np.full((1, 32), 16, np.int64)
    q[0, 3] = 16 + 5                              # low nibble of byte 3, no fifth bit change
    q[0, 20] = 1                                  # high nibble of byte 4, fifth bit clear
    q[0, 31] = 31
    wb, vals = gp.pack_q5_0(np.array([[0x3C00]], np.uint16), q)
    assert wb[0, 6 + 3] == (5 | (0 << 4)) and wb[0, 6 + 4] == (0 | (1 << 4))
    qh = int.from_bytes(bytes(wb[0, 2:6]), "little")
    assert qh == (0xFFFFFFFF & ~(1 << 20)) & ~0
    got = orc.dequant_rows(gp.GGML_Q5_0, wb, 1, 32)[0]
    assert np.array_equal(got, vals[0])
    want = np.zeros(32, np.float32)
    want[3], want[20], want[31] = 5, -15, 15
    assert np.array_equal(got, want)


def test_q5_0_row_dot_is_scale_times_the_block_sum():
    # Q5_0FloatTensor.dot: sum += (q0 - 16) * x[j]; sum += (q1 - 16) * x[j + 16] for j < 16,
    # then result += scale * sum, block by block
    rng = np.random.default_rng(7)
    wb, vals = gp.random_weights(gp.GGML_Q5_0, 1, 64, rng)
    x = rng.standard_normal(64).astype(F32)
    blk = wb[0].reshape(2, 22)
    res = F32(0)
    for b_ in range(2):
        d = np.frombuffer(bytes(blk[b_, 0:2]), np.float16)[0].astype(F32)
        qh = int.from_bytes(bytes(blk[b_, 2:6]), "little")
        s_ = F32(0)
        for j in range(16):
            q0 = (blk[b_, 6 + j] & 15) | (((qh >> j) & 1) << 4)
            q1 = (blk[b_, 6 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4)
            s_ = F32(s_ + F32(F32(int(q0) - 16) * x[32 * b_ + j]))
            s_ = F32(s_ + F32(F32(int(q1) - 16) * x[32 * b_ + j + 16]))
        res = F32(res + F32(d * s_))
    assert orc.matmul(gp.GGML_Q5_0, wb, 1, 64, x)[0] == res


def test_q3_k_sub_blocks_of_16_take_their_own_scales():
    # 16 distinct scales, including top bits; code 5 = value +1, so each value is d*(sc-32)
    sc = np.array([[[0, 1, 17, 30, 33, 40, 47, 48, 15, 16, 31, 32, 49, 55, 62, 63]]])
    q = np.full((1, 256), 5, np.int64)
    wb, vals = gp.pack_q3_k(np.array([[0x3C00]], np.uint16), sc, q)
    got = orc.dequant_rows(gp.GGML_Q3_K, wb, 1, 256)[0]
    assert np.array_equal(got, vals[0])
    for j in range(256):
        h, r = divmod(j, 128)
        p_, r = divmod(r, 32)
        w, _ = divmod(r, 16)
        assert got[j] == sc[0, 0, 8 * h + 2 * p_ + w] - 32, j


def test_q3_k_codes_place_their_bits():
    # code c at element j: low bits at qs[32h + 16w + l] >> 2p, third bit at hmask[16w + l]
    # bit 4h + p; value (c - 4) with scale 33 (d = 1)
    sc = np.full((1, 1, 16), 33)
    rng = np.random.default_rng(3)
    q = rng.integers(0, 8, (1, 256))
    wb, _ = gp.pack_q3_k(np.array([[0x3C00]], np.uint16), sc, q)
    got = orc.dequant_rows(gp.GGML_Q3_K, wb, 1, 256)[0]
    assert np.array_equal(got, (q[0] - 4).astype(F32))


def test_q5_k_fifth_bits_and_scales():
    sc = np.array([[[1, 2, 3, 4, 49, 50, 61, 63]]])
    mn = np.zeros((1, 1, 8), np.int64)
    rng = np.random.default_rng(4)
    q = rng.integers(0, 32, (1, 256))
    wb, vals = gp.pack_q5_k(np.array([[0x3C00]], np.uint16), np.array([[0x3800]], np.uint16), sc, mn, q)
    got = orc.dequant_rows(gp.GGML_Q5_K, wb, 1, 256)[0]
    assert np.array_equal(got, vals[0])
    assert np.array_equal(got, (np.repeat(sc[0, 0], 32) * q[0]).astype(F32))


def test_iq4_nl_codebook_and_split_nibbles():
    idx = np.arange(32).reshape(1, 32) % 16
    wb, vals = gp.pack_iq4_nl(np.array([[0x3C00]], np.uint16), idx)
    got = orc.dequant_rows(gp.GGML_IQ4_NL, wb, 1, 32)[0]
    assert np.array_equal(got, vals[0])
    book = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    assert list(got[:16]) == book and list(got[16:]) == book
    assert wb[0, 2] == (0 | (0 << 4)) and wb[0, 3] == (1 | (1 << 4))


def test_iq4_xs_sub_block_scales_and_split_nibbles():
    ls = np.array([[[0, 31, 32, 33, 47, 48, 62, 63]]])
    idx = np.full((1, 256), 8)                   # codebook value +1
    idx[0, 16] = 15                              # sub-block 0, high nibble of byte 0: +113
    wb, vals = gp.pack_iq4_xs(np.array([[0x3C00]], np.uint16), ls, idx)
    got = orc.dequant_rows(gp.GGML_IQ4_XS, wb, 1, 256)[0]
    assert np.array_equal(got, vals[0])
    for ib in range(8):
        seg = got[32 * ib:32 * ib + 32]
        want = np.full(32, ls[0, 0, ib] - 32, F32)
        if ib == 0:
            want[16] = (ls[0, 0, 0] - 32) * 113
        assert np.array_equal(seg, want), ib
    assert wb[0, 8] == (8 | (15 << 4))


def test_q5_1_split_nibbles_fifth_bit_and_min():
    # element i < 16: low nibble of byte i; 16 + i: its high nibble; bit 4 from qh bit i;
    # value q * d + m (Q5_1FloatTensor.getFloat), here d = 1, m = 0.5
    q = np.zeros((1, 32), np.int64)
    q[0, 3], q[0, 20], q[0, 31], q[0, 16] = 5, 17, 31, 16
    wb, vals = gp.pack_q5_1(np.array([[0x3C00]], np.uint16), np.array([[0x3800]], np.uint16), q)
    assert wb[0, 8 + 3] == 5 and wb[0, 8 + 4] == (1 << 4) and wb[0, 8 + 0] == 0
    qh = int.from_bytes(bytes(wb[0, 4:8]), "little")
    assert qh == (1 << 20) | (1 << 31) | (1 << 16)
    got = orc.dequant_rows(gp.GGML_Q5_1, wb, 1, 32)[0]
    want = q[0].astype(F32) + F32(0.5)
    assert np.array_equal(got, want) and np.array_equal(got, vals[0])


def test_q5_1_row_dot_restates_the_java_loop():
    # Q5_1FloatTensor.dot: blockSum += q0*x[j]; blockSum += q1*x[j+16]; otherSum += x[j] +
    # x[j+16] for j < 16, then result += scale*blockSum + min*otherSum, block by block
    rng = np.random.default_rng(17)
    wb, _ = gp.random_weights(gp.GGML_Q5_1, 1, 96, rng)
    x = rng.standard_normal(96).astype(F32)
    blk = wb[0].reshape(3, 24)
    res = F32(0)
    for b_ in range(3):
        d = np.frombuffer(bytes(blk[b_, 0:2]), np.float16)[0].astype(F32)
        m = np.frombuffer(bytes(blk[b_, 2:4]), np.float16)[0].astype(F32)
        qh = int.from_bytes(bytes(blk[b_, 4:8]), "little")
        bs = os_ = F32(0)
        for j in range(16):
            q0 = (blk[b_, 8 + j] & 15) | (((qh >> j) & 1) << 4)
            q1 = (blk[b_, 8 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4)
            bs = F32(bs + F32(F32(int(q0)) * x[32 * b_ + j]))
            bs = F32(bs + F32(F32(int(q1)) * x[32 * b_ + j + 16]))
            os_ = F32(os_ + F32(x[32 * b_ + j] + x[32 * b_ + j + 16]))
        res = F32(res + F32(F32(d * bs) + F32(m * os_)))
    assert orc.matmul(gp.GGML_Q5_1, wb, 1, 96, x)[0] == res


def test_q2_k_reference_element_order_and_sub_block_scales():
    # the reference's order (Q2_KFloatTensor.getFloat): element j at bits 2(j%4) of quant byte
    # j/4 (not ggml's interleave of 32-element runs); scale byte j/16: low nibble sc, high m;
    # value d*sc*q - dmin*m, here d = dmin = 1
    rng = np.random.default_rng(21)
    q = rng.integers(0, 4, (1, 256))
    sc = rng.integers(0, 16, (1, 1, 16))
    mn = rng.integers(0, 16, (1, 1, 16))
    one = np.array([[0x3C00]], np.uint16)
    wb, vals = gp.pack_q2_k(one, one, sc, mn, q)
    for j in (0, 1, 5, 22, 255):
        assert (wb[0, 16 + j // 4] >> (2 * (j % 4))) & 3 == q[0, j]
    assert wb[0, 7] == sc[0, 0, 7] | (mn[0, 0, 7] << 4)
    got = orc.dequant_rows(gp.GGML_Q2_K, wb, 1, 256)[0]
    want = (np.repeat(sc[0, 0], 16) * q[0] - np.repeat(mn[0, 0], 16)).astype(F32)
    assert np.array_equal(got, want) and np.array_equal(got, vals[0])


def test_q2_k_row_dot_restates_dotq2kf32():
    # per sub-block of 16: sumQ += q*f, sumF += f; result += d*sc*sumQ - dmin*m*sumF
    rng = np.random.default_rng(22)
    wb, _ = gp.random_weights(gp.GGML_Q2_K, 1, 256, rng)
    x = rng.standard_normal(256).astype(F32)
    blk = wb[0]
    d = np.frombuffer(bytes(blk[80:82]), np.float16)[0].astype(F32)
    dmin = np.frombuffer(bytes(blk[82:84]), np.float16)[0].astype(F32)
    res = F32(0)
    for sb in range(16):
        sc, m = int(blk[sb] & 15), int(blk[sb] >> 4)
        sq = sf = F32(0)
        for i in range(16):
            j = 16 * sb + i
            q = (int(blk[16 + j // 4]) >> (2 * (j % 4))) & 3
            sq = F32(sq + F32(F32(q) * x[j]))
            sf = F32(sf + x[j])
        res = F32(res + F32(F32(F32(d * F32(sc)) * sq) - F32(F32(dmin * F32(m)) * sf)))
    assert orc.matmul(gp.GGML_Q2_K, wb, 1, 256, x)[0] == res


def _grid_levels(t):
    # entries, bytes per entry and the lattice levels a byte may take: IQ3_XXS 8 levels
    # (4, 12, .., 52 and 62: ggml's iq3xxs grid tops out at 62, not 60), IQ3_S the odd
    # numbers 1..15, IQ2_S the three levels 8, 25, 43
    return {gp.GGML_IQ3_XXS: (256, 4, [4, 12, 20, 28, 36, 44, 52, 62]),
            gp.GGML_IQ3_S: (512, 4, list(range(1, 16, 2))),
            gp.GGML_IQ2_S: (1024, 8, [8, 25, 43])}[t]


@pytest.mark.parametrize("t", IQ_TYPES, ids=[NAMES[t] for t in IQ_TYPES])
def test_iq_codebooks_are_ordered_lattice_tables(t):
    # The codebooks are format constants (ggml's iq3xxs/iq3s/iq2s grids).  Each lists distinct
    # lattice points in increasing order, every byte one of the format's levels, the first
    # entry all at the lowest level: a mistyped or swapped entry breaks one of these.  The
    # kernels' copy (llmplayer_amd/csrc/iq_grids.h) must hold the same values.
    import pathlib
    import re
    n, width, levels = _grid_levels(t)
    g = orc.iq_grid(t)
    assert len(g) == n and np.all(g[1:] > g[:-1])
    b = np.stack([(g >> np.uint64(8 * j)) & np.uint64(0xFF) for j in range(width)], -1).astype(np.int64)
    assert set(np.unique(b)) == set(levels)
    assert np.all(b[0] == levels[0])
    # each byte level occurs in every position: no byte column was dropped or duplicated
    for j in range(width):
        assert set(np.unique(b[:, j])) == set(levels), j
    src = (pathlib.Path(__file__).resolve().parents[1] / "llmplayer_amd" / "csrc" / "iq_grids.h").read_text()
    name = {gp.GGML_IQ3_XXS: "kIq3xxsGrid", gp.GGML_IQ3_S: "kIq3sGrid", gp.GGML_IQ2_S: "kIq2sGrid"}[t]
    body = re.search(name + r"\[\d+\][^=]*= \{(.*?)\};", src, re.S).group(1)
    dev = np.array([int(v, 16) for v in re.findall(r"0x([0-9a-f]+)", body)], np.uint64)
    assert np.array_equal(dev, g)


def test_iq3_xxs_sign_patterns_have_even_parity():
    # KSIGNS_IQ2XS: entry i keeps the 7-bit index and sets bit 7 so that the byte has an even
    # number of set bits (the eighth sign is implied); spot values from the reference table
    got = [orc.ksigns(i) for i in range(128)]
    assert all(v & 0x7F == i and bin(v).count("1") % 2 == 0 for i, v in enumerate(got))
    assert (got[0], got[1], got[2], got[3], got[64], got[127]) == (0, 129, 130, 3, 192, 255)


def test_iq3_xxs_word_fields_and_closed_form():
    # one super-block, every index 0 (entry 0 = four 4s): weight 32 ib32 + 8l + j is
    # (d * (0.5 + sc) * 0.5) * 4, negated by bit j of pattern ksigns(idx) of its 8-group
    d = np.array([[0x3C00]], np.uint16)   # 1.0
    rng = np.random.default_rng(31)
    si = rng.integers(0, 128, (1, 1, 8, 4))
    sc = rng.integers(0, 16, (1, 1, 8))
    grid = orc.iq_grid(gp.GGML_IQ3_XXS)
    wb, vals = gp.pack_iq3_xxs(d, np.zeros((1, 1, 64), np.int64), si, sc, grid)
    aux = int.from_bytes(bytes(wb[0, 66 + 4 * 5:66 + 4 * 6]), "little")
    assert aux >> 28 == sc[0, 0, 5] and (aux >> 14) & 0x7F == si[0, 0, 5, 2]
    got = orc.dequant_rows(gp.GGML_IQ3_XXS, wb, 1, 256)[0]
    for ib in range(8):
        for l in range(4):
            pat = orc.ksigns(int(si[0, 0, ib, l]))
            mag = F32(F32(F32(1.0) * F32(0.5 + sc[0, 0, ib])) * F32(0.5)) * F32(4)
            want = np.array([-mag if (pat >> j) & 1 else mag for j in range(8)], F32)
            assert np.array_equal(got[32 * ib + 8 * l:32 * ib + 8 * l + 8], want), (ib, l)
    assert np.array_equal(got, vals[0])


def test_iq3_s_ninth_bits_follow_the_reference_not_ggml():
    # The ninth index bit of 32-group g comes from qh[g/4 + g%2] (IQ3_SFloatTensor's
    # OFF_QH + ib32/4, +1 for a pair's second group; its CUDA kernel reads the same bytes).
    # With only qh[1] set, groups 1, 3, 4 and 6 take entries 256 + qs; ggml (qh[g]) would
    # give that to group 1 alone.
    d = np.array([[0x3C00]], np.uint16)
    rng = np.random.default_rng(32)
    qs = rng.integers(0, 256, (1, 1, 64))
    qh = np.zeros((1, 1, 8), np.int64)
    qh[0, 0, 1] = 0xFF
    grid = orc.iq_grid(gp.GGML_IQ3_S)
    sc = np.zeros((1, 1, 8), np.int64)        # db = d * 1
    signs = np.zeros((1, 1, 32), np.int64)
    wb, vals = gp.pack_iq3_s(d, qs, qh, signs, sc, grid)
    got = orc.dequant_rows(gp.GGML_IQ3_S, wb, 1, 256)[0]
    for g in range(8):
        high = 256 if g in (1, 3, 4, 6) else 0
        for k in range(8):   # the group's 8 indices, 4 weights each
            e = int(grid[int(qs[0, 0, 8 * g + k]) + high])
            want = np.array([(e >> (8 * j)) & 0xFF for j in range(4)], F32)
            assert np.array_equal(got[32 * g + 4 * k:32 * g + 4 * k + 4], want), (g, k)
    assert np.array_equal(got, vals[0])
    # the scale nibbles: d * (1 + 2 sc), group g from byte g/2, low nibble first
    sc = np.arange(8).reshape(1, 1, 8) * 2
    wb, _ = gp.pack_iq3_s(d, qs, qh, signs, sc, grid)
    got2 = orc.dequant_rows(gp.GGML_IQ3_S, wb, 1, 256)[0]
    assert np.array_equal(got2, got * np.repeat(1 + 2 * sc[0, 0], 32).astype(F32))


def test_iq2_s_high_bits_scale_halves_and_signs():
    # index l of 32-group ib32: qs[4 ib32 + l] | bits 2l..2l+1 of qh[ib32] << 8; the low scale
    # nibble covers l = 0, 1 and the high one l = 2, 3; sign bit j of byte 4 ib32 + l
    d = np.array([[0x3C00]], np.uint16)
    rng = np.random.default_rng(33)
    qs = rng.integers(0, 256, (1, 1, 32))
    qh = rng.integers(0, 256, (1, 1, 8))
    signs = rng.integers(0, 256, (1, 1, 32))
    sc = rng.integers(0, 16, (1, 1, 16))
    grid = orc.iq_grid(gp.GGML_IQ2_S)
    wb, vals = gp.pack_iq2_s(d, qs, qh, signs, sc, grid)
    assert wb[0, 74 + 3] == sc[0, 0, 6] | (sc[0, 0, 7] << 4)
    got = orc.dequant_rows(gp.GGML_IQ2_S, wb, 1, 256)[0]
    for ib in range(8):
        for l in range(4):
            idx = int(qs[0, 0, 4 * ib + l]) | (((int(qh[0, 0, ib]) >> (2 * l)) & 3) << 8)
            e = int(grid[idx])
            dl = F32(F32(F32(1.0) * F32(0.5 + sc[0, 0, 2 * ib + l // 2])) * F32(0.25))
            s = int(signs[0, 0, 4 * ib + l])
            want = np.array([(-1 if (s >> j) & 1 else 1) * F32(dl * F32((e >> (8 * j)) & 0xFF))
                             for j in range(8)], F32)
            assert np.array_equal(got[32 * ib + 8 * l:32 * ib + 8 * l + 8], want), (ib, l)
    assert np.array_equal(got, vals[0])


def test_mxfp4_scale_exponent_and_special_bytes():
    idx = np.tile(np.arange(16), 2).reshape(1, 32)
    for e, scale in ((127, 1.0), (130, 8.0), (120, 2.0 ** -7), (0, 0.0), (255, 0.0), (1, 2.0 ** -126)):
        wb, vals = gp.pack_mxfp4(np.array([[e]]), idx)
        got = orc.dequant_rows(gp.GGML_MXFP4, wb, 1, 32)[0]
        assert np.array_equal(got.view(np.uint32), vals[0].view(np.uint32)), e
        mags = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
        assert np.array_equal(np.abs(got[:8]), np.array(mags, F32) * F32(scale)), e
        assert np.all(got[9:16] == -got[1:8]) and np.array_equal(got[16:], got[:16]), e


@pytest.mark.parametrize("t", TYPES, ids=[NAMES[t] for t in TYPES])
def test_matmul_matches_float64_and_accumulates(t):
    rng = np.random.default_rng(90 + t)
    rows, cols = 24, 768
    wb, vals = gp.random_weights(t, rows, cols, rng)
    x = rng.standard_normal(cols).astype(F32)
    base = rng.standard_normal(rows).astype(F32)
    got = orc.matmul(t, wb, rows, cols, x, out=base)
    want = base.astype(np.float64) + vals.astype(np.float64) @ x.astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("t", [gp.GGML_F16, gp.GGML_BF16], ids=["f16", "bf16"])
def test_half_precision_rows_sum_sequentially_unfused(t):
    # FloatTensor.dot: sum += getFloat(i) * other[i], one float at a time
    rng = np.random.default_rng(95)
    wb, vals = gp.random_weights(t, 1, 64, rng, scale=1.0)
    x = rng.standard_normal(64).astype(F32)
    s = F32(0.0)
    for w, xv in zip(vals[0], x):
        s = F32(s + F32(w * xv))
    assert orc.matmul(t, wb, 1, 64, x)[0] == s


def test_rmsnorm_matches_float64_and_closed_form():
    rng = np.random.default_rng(96)
    x = rng.standard_normal(3072).astype(F32) * F32(5)
    w = rng.uniform(0.5, 1.5, 3072).astype(F32)
    got = orc.rmsnorm(x, w, 1e-5)
    np.testing.assert_allclose(got, rm.rms_norm_heads(x, w, 1, 3072, 1e-5), rtol=2e-6, atol=1e-7)
    c = np.full(256, 3.0, F32)                     # ss = 2304 exactly: r = 1/(float)sqrt(9 + eps)
    r = F32(1.0) / F32(np.sqrt(np.float64(F32(F32(2304.0) / F32(256)) + F32(1e-6))))
    assert np.array_equal(orc.rmsnorm(c, np.ones(256, F32), 1e-6), np.full(256, F32(3.0) * r))


def _block_setup(seed, t, merged=False, post=False, bias=False, rscale=0.0):
    Hq, Hkv, D, dim, S = 4, 2, 64, 256, 40
    qd, kvd = Hq * D, Hkv * D
    rng = np.random.default_rng(seed)
    cfg = orc.OracleConfig(Hq, Hkv, D, S, rope_type=0, norm_eps=1e-5)
    wq, vq = gp.random_weights(t, qd, dim, rng)
    wk, vk = gp.random_weights(t, kvd, dim, rng)
    wv, vv = gp.random_weights(t, kvd, dim, rng)
    wo, vo = gp.random_weights(t, dim, qd, rng)
    bw = orc.BlockWeights(dim, wo=wo, wo_type=t, residual_scale=rscale,
                          attn_norm=rng.uniform(0.5, 1.5, dim).astype(F32))
    if merged:
        bw.wqkv, bw.wqkv_type = np.concatenate([wq, wk, wv]), t
    else:
        bw.wq, bw.wk, bw.wv = wq, wk, wv
        bw.wq_type = bw.wk_type = bw.wv_type = t
    if post:
        bw.post_attn_norm = rng.uniform(0.5, 1.5, dim).astype(F32)
    if bias:
        bw.q_bias = rng.standard_normal(qd).astype(F32) * F32(0.1)
        bw.k_bias = rng.standard_normal(kvd).astype(F32) * F32(0.1)
        bw.v_bias = rng.standard_normal(kvd).astype(F32) * F32(0.1)
        bw.o_bias = rng.standard_normal(dim).astype(F32) * F32(0.1)
    kc = np.zeros((S, kvd), F32); vc = np.zeros((S, kvd), F32)
    pos = 30
    kc[:pos] = rng.standard_normal((pos, kvd)).astype(F32)
    vc[:pos] = rng.standard_normal((pos, kvd)).astype(F32)
    x = rng.standard_normal(dim).astype(F32) * F32(2)
    cs, sn = orc.rope_tables(D, S, 5e5)
    return cfg, bw, (vq, vk, vv, vo), kc, vc, x, pos, cs, sn


@pytest.mark.parametrize("t", [gp.GGML_F32, gp.GGML_Q8_0, gp.GGML_Q4_K, gp.GGML_Q6_K],
                         ids=["f32", "q8_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("post,bias,rscale", [(False, False, 0.0), (True, True, 0.25)],
                         ids=["prenorm", "postnorm-bias-granite"])
def test_attn_block_matches_float64_chain(t, post, bias, rscale):
    cfg, bw, (vq, vk, vv, vo), kc, vc, x, pos, cs, sn = _block_setup(100 + t, t, post=post,
                                                                    bias=bias, rscale=rscale)
    kc0, vc0 = kc.copy(), vc.copy()
    got = orc.attn_block(cfg, bw, kc, vc, x, 0, pos, rope_cos=cs, rope_sin=sn)
    Hq, Hkv, D = 4, 2, 64
    x64 = x.astype(np.float64)
    xb = rm.rms_norm_heads(x, bw.attn_norm, 1, 256, 1e-5)
    q = vq.astype(np.float64) @ xb
    k = vk.astype(np.float64) @ xb
    v = vv.astype(np.float64) @ xb
    if bias:
        q += bw.q_bias; k += bw.k_bias; v += bw.v_bias
    c, s = cs[pos].astype(np.float64), sn[pos].astype(np.float64)

    def rope(z, nh):
        z = z.reshape(nh, D).copy()
        a, b = z[:, 0::2].copy(), z[:, 1::2].copy()
        z[:, 0::2], z[:, 1::2] = a * c - b * s, a * s + b * c
        return z.reshape(-1)
    K, V = kc0.astype(np.float64), vc0.astype(np.float64)
    K[pos], V[pos] = rope(k, Hkv), v
    att = rm.attention(rope(q, Hq), K, V, Hq, Hkv, D, 0, pos, 1 / np.sqrt(D))
    o = vo.astype(np.float64) @ att
    if bias:
        o += bw.o_bias
    if post:
        o = rm.rms_norm_heads(o, bw.post_attn_norm, 1, 256, 1e-5)
    if rscale > 0:
        o *= rscale
    np.testing.assert_allclose(got, x64 + o, rtol=1e-4, atol=2e-5)
    np.testing.assert_allclose(kc[pos], K[pos], rtol=1e-4, atol=1e-5)


def test_attn_block_zero_output_projection_leaves_the_residual():
    cfg, bw, _, kc, vc, x, pos, cs, sn = _block_setup(120, gp.GGML_F32)
    bw.wo = np.zeros_like(bw.wo)
    assert np.array_equal(orc.attn_block(cfg, bw, kc, vc, x, 0, pos, rope_cos=cs, rope_sin=sn), x)
    b = np.linspace(-1, 1, 256).astype(F32)
    bw.o_bias = b
    assert np.array_equal(orc.attn_block(cfg, bw, kc, vc, x, 0, pos + 1, rope_cos=cs, rope_sin=sn),
                          x + b)


def test_attn_block_merged_qkv_equals_separate_projections():
    for t in (gp.GGML_Q4_K, gp.GGML_BF16):
        cfg, bw, _, kc, vc, x, pos, cs, sn = _block_setup(130 + t, t)
        cfg2, bw2, _, kc2, vc2, _, _, _, _ = _block_setup(130 + t, t, merged=True)
        a = orc.attn_block(cfg, bw, kc, vc, x, 0, pos, rope_cos=cs, rope_sin=sn)
        b = orc.attn_block(cfg2, bw2, kc2, vc2, x, 0, pos, rope_cos=cs, rope_sin=sn)
        assert np.array_equal(a, b) and np.array_equal(kc, kc2)


# ---- the reference GPU's Q8_1-input matvecs ---------------------------------------------------

def test_q8_1_quantiser_closed_forms():
    """d = max|x|/127, quants rint(x*127/max) with ties to even and +-127 at the extremes, a
    zero block all zero, the block sum exact on small integers."""
    x = np.zeros(96, F32)
    x[:32] = np.arange(-16, 16, dtype=F32)            # max 16: quants rint(x*127/16)
    x[32:64] = 0.0                                     # zero block
    x[64:96] = np.array([127, 2.5, 3.5, -2.5, -127] + [0.5] * 27, F32)   # max 127: inv = 1
    q, d, s = orc.quantize_q8_1(x)
    assert d[0] == F32(16) / F32(127) and d[1] == 0 and d[2] == 1
    want0 = np.clip(np.rint(x[:32] * (F32(127) / F32(16))), -127, 127)
    assert np.array_equal(q[:32], want0.astype(np.int8)) and q[0] == -127
    assert not q[32:64].any() and s[1] == 0
    assert list(q[64:69]) == [127, 2, 4, -2, -127] and (q[69:] == 0).all()   # 0.5 -> 0 (even)
    assert s[0] == -16 and s[2] == F32(127 + 2.5 + 3.5 - 2.5 - 127 + 27 * 0.5)


def test_q8_1_quantiser_against_numpy_and_its_error_bound():
    rng = np.random.default_rng(41)
    x = (rng.standard_normal(4096) * rng.uniform(0.1, 10, 4096)).astype(F32)
    q, d, s = orc.quantize_q8_1(x)
    xb = x.reshape(-1, 32)
    m = np.abs(xb).max(axis=1)
    assert np.array_equal(d, (m / F32(127)).astype(F32))
    want = np.clip(np.rint(xb * (F32(127) / m)[:, None]), -127, 127).astype(np.int8).reshape(-1)
    assert np.array_equal(q, want)
    # reconstruction within half a step; sums within float32 rounding of the float64 sum
    assert (np.abs(q.reshape(-1, 32) * d[:, None] - xb) <= 0.5 * d[:, None] * (1 + 1e-6)).all()
    np.testing.assert_allclose(s, xb.astype(np.float64).sum(axis=1), rtol=1e-5, atol=1e-4)


def test_staged_rmsnorm_matches_float64_and_the_plain_one():
    rng = np.random.default_rng(42)
    for n in (256, 3072, 8192):
        x = (rng.standard_normal(n) * 2).astype(F32)
        w = rng.uniform(0.5, 1.5, n).astype(F32)
        got = orc.rmsnorm_staged(x, w, 1e-5)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt((x64 ** 2).mean() + 1e-5) * w
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-7)
        np.testing.assert_allclose(got, orc.rmsnorm(x, w, 1e-5), rtol=1e-6, atol=1e-7)
    c = np.full(512, 3.0, F32)   # a constant vector: exact sums, r = 1/sqrt(9 + eps)
    got = orc.rmsnorm_staged(c, np.ones(512, F32), 0.0)
    assert np.array_equal(got, c * F32(1.0 / np.sqrt(9.0)))


Q8_1_TYPES = [gp.GGML_Q8_0, gp.GGML_Q4_K, gp.GGML_Q5_0, gp.GGML_Q3_K, gp.GGML_Q5_K, gp.GGML_IQ4_NL,
              gp.GGML_IQ4_XS]


@pytest.mark.parametrize("t", Q8_1_TYPES, ids=[NAMES[t] for t in Q8_1_TYPES])
def test_q8_1_matmul_equals_the_float_matmul_on_an_exactly_quantised_input(t):
    """On an input that Q8_1 represents exactly (x = d*q, with the block sum exact), the int8
    matvec is the float matvec of the dequantised weights (the independent packer's values):
    the Q4_K / Q5_K min term enters through the block sum, the scales through d.  A wrong
    nibble, bit or sign in a format's integer decode, or a scale on the wrong 16 or 32
    values, moves it far off."""
    rng = np.random.default_rng(43 + t)
    rows, cols = 24, 1024
    wb, vals = gp.random_weights(t, rows, cols, rng)
    qx = rng.integers(-127, 128, cols).astype(np.int8)
    qx[::32] = 127                                    # each block's max is 127: d exact
    d = (2.0 ** rng.integers(-6, 2, cols // 32)).astype(F32)
    x = (qx.reshape(-1, 32) * d[:, None]).astype(F32).reshape(-1)
    q, dd, s = orc.quantize_q8_1(x)
    assert np.array_equal(q, qx) and np.array_equal(dd, d)   # powers of two: exact
    got = orc.matmul_q8_1(t, wb, rows, cols, q, dd, s)
    want = vals.astype(np.float64) @ x.astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-4 * np.abs(want).max())


def test_q8_1_matmul_integer_closed_form_and_min_term():
    """Q8_0: a row of all-ones quants with d = 1 gives (d_x)*(sum of the input's quants) per
    block.  Q4_K: the min term is -(dmin*m)*s per sub-block, linear in the block sums."""
    cols = 64
    wb, _ = gp.pack_q8_0(gp._f16_bits(np.ones((1, 2))), np.ones((1, cols), np.int8))
    q = np.arange(-32, 32).astype(np.int8)
    d = np.array([0.5, 2.0], F32)
    got = orc.matmul_q8_1(gp.GGML_Q8_0, wb, 1, cols, q, d, np.zeros(2, F32))
    assert got[0] == F32(0.5 * q[:32].astype(int).sum() + 2.0 * q[32:].astype(int).sum())
    rng = np.random.default_rng(44)
    wb, _ = gp.random_weights(gp.GGML_Q4_K, 3, 256, rng)
    q = rng.integers(-127, 128, 256).astype(np.int8)
    d = np.full(8, 0.01, F32)
    a = orc.matmul_q8_1(gp.GGML_Q4_K, wb, 3, 256, q, d, np.zeros(8, F32))
    e = np.zeros(8, F32)
    e[3] = 1.0
    b = orc.matmul_q8_1(gp.GGML_Q4_K, wb, 3, 256, q, d, e)
    dmin = np.array([gp._f16_val(wb[r, 2:4].view(np.uint16))[0] for r in range(3)], np.float64)
    head = wb[:, 4:16]
    m3 = head[:, 7] & 63                               # sub-block 3's min: byte 3 + 4 of the scales
    np.testing.assert_allclose(a.astype(np.float64) - b, dmin * m3, rtol=1e-6, atol=1e-9)


def test_q8_1_routed_types_are_the_reference_gpus():
    """The int8 kernels CudaForwardPass picks by default (dp4aType, CudaForwardPass.java:216-226;
    Q6_K's is opt-in, :2029-2038)."""
    routed = {t for t in NAMES if orc.q8_1_routed(t)}
    assert routed == set(Q8_1_TYPES)


def test_attn_block_q8_1_mode_routes_the_reference_gpus_int8_types():
    """Non-dp4a types (F16, Q6_K, Q4_0, MXFP4) take the fp32 path in the Q8_1 mode: the block
    then differs from the fp32 mode only by the norm's summation order.  The int8 types' blocks
    move by the input quantisation (half a step of 1/127 of each block's maximum, times weights
    whose integer values reach 31 with Q5_K's unsigned codes and their min term): a loose
    bound that only shows the int8 path was taken; the exact-input test above pins it."""
    cases = [(t, 2e-5) for t in (gp.GGML_F16, gp.GGML_Q6_K, gp.GGML_Q4_0, gp.GGML_MXFP4)]
    cases += [(t, 6e-2) for t in Q8_1_TYPES]
    for t, tol in cases:
        cfg, bw, _, kc, vc, x, pos, cs, sn = _block_setup(150 + t, t)
        kc2, vc2 = kc.copy(), vc.copy()
        a = orc.attn_block(cfg, bw, kc, vc, x, 0, pos, rope_cos=cs, rope_sin=sn)
        bw.q8_1_input = True
        b = orc.attn_block(cfg, bw, kc2, vc2, x, 0, pos, rope_cos=cs, rope_sin=sn)
        err = np.abs(a - b).max() / np.abs(a - x).max()
        assert err <= tol, (t, err)
        if tol > 1e-3:
            assert err > 1e-6, "the int8 path was not taken"
