"""Packers for the GGUF weight formats of the reference's tensor classes, written from each
format's layout (the inverse direction of the dequantisers in oracle/block_oracle.c and of
the library's repacking), plus the exact float32 values each packed weight stands for.

Every packer takes the format's fields (scales, mins, quants) and returns (bytes [rows,
row_bytes] uint8, dequantised values [rows, cols] float32), the values computed in float32
in the reference's operation order (the dot() of Q8_0FloatTensor, Q4_0FloatTensor,
Q4_KFloatTensor, Q6_KFloatTensor, Q3_KFloatTensor, Q5_KFloatTensor, IQ4_NLFloatTensor,
IQ4_XSFloatTensor and MXFP4FloatTensor; Q5_0FloatTensor.getFloat; the IQ3_XXS, IQ3_S and IQ2_S
classes' getFloat, element by element).  Random fields give test weights whose dequantised
values are known without running the code under test.  The IQ packers take their format's
codebook as an argument (the tests pass the oracle's, which the table checks pin)."""
import numpy as np

F32 = np.float32
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K, GGML_BF16 = 0, 1, 2, 8, 12, 14, 30
GGML_Q5_0, GGML_Q3_K, GGML_Q5_K, GGML_IQ4_NL, GGML_IQ4_XS, GGML_MXFP4 = 6, 11, 13, 20, 23, 39
GGML_Q5_1, GGML_Q2_K = 7, 10
GGML_IQ3_XXS, GGML_IQ3_S, GGML_IQ2_S = 18, 21, 22

# the non-linear 4-bit codebook of IQ4_NL and IQ4_XS (GGUF's kvalues_iq4nl)
IQ4NL_VALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], F32)
# FP4 E2M1 by code: sign bit 3, exponent bits 2-1, mantissa bit 0 (OCP microscaling formats)
FP4_VALUES = np.array([s * m for s in (1.0, -1.0) for m in (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)], F32)


def _f16_bits(x):
    return np.asarray(x, np.float16).view(np.uint16)


def _f16_val(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(F32)


def pack_f32(w):
    w = np.ascontiguousarray(w, F32)
    return w.view(np.uint8).reshape(w.shape[0], -1).copy(), w.copy()


def pack_f16(w):
    h = np.asarray(w, np.float16)
    return h.view(np.uint8).reshape(h.shape[0], -1).copy(), h.astype(F32)


def pack_bf16(w):
    bits = (np.ascontiguousarray(w, F32).view(np.uint32) >> 16).astype(np.uint16)
    vals = (bits.astype(np.uint32) << 16).view(F32)
    return bits.view(np.uint8).reshape(bits.shape[0], -1).copy(), vals


def pack_q8_0(d_bits, q):
    """d_bits [rows, nb] fp16 scale bits, q [rows, nb*32] int8.  Block: d (2 B) + 32 int8."""
    rows, nb = d_bits.shape
    out = np.zeros((rows, nb, 34), np.uint8)
    out[:, :, 0:2] = np.asarray(d_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = np.asarray(q, np.int8).reshape(rows, nb, 32).view(np.uint8)
    vals = (_f16_val(d_bits)[..., None] * q.reshape(rows, nb, 32).astype(F32)).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def pack_q4_0(d_bits, q):
    """q [rows, nb*32] in 0..15; byte i of a block holds element 2i (low nibble) and 2i+1
    (high nibble), as Q4_0FloatTensor reads it."""
    rows, nb = d_bits.shape
    qb = np.asarray(q, np.uint8).reshape(rows, nb, 16, 2)
    out = np.zeros((rows, nb, 18), np.uint8)
    out[:, :, 0:2] = np.asarray(d_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = qb[..., 0] | (qb[..., 1] << 4)
    vals = ((q.reshape(rows, nb, 32).astype(np.int32) - 8).astype(F32) *
            _f16_val(d_bits)[..., None]).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def pack_q4_k(d_bits, dmin_bits, sc, mn, q):
    """Super-blocks of 256: d, dmin fp16; 8 six-bit scales and mins packed in 12 bytes
    (j < 4: bytes j and j+4 hold scale/min j in their low 6 bits and the top 2 bits of
    scale/min j+4; byte j+8 holds the low 4 bits of scale j+4 and of min j+4); 128 bytes of
    nibbles: byte 32g+l = element 64g+l (low) | element 64g+32+l (high).
    sc, mn [rows, ns, 8] in 0..63; q [rows, ns*256] in 0..15."""
    rows, ns = d_bits.shape
    out = np.zeros((rows, ns, 144), np.uint8)
    out[:, :, 0:2] = np.asarray(d_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, ns, 2)
    out[:, :, 2:4] = np.asarray(dmin_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, ns, 2)
    sc = np.asarray(sc, np.uint8)
    mn = np.asarray(mn, np.uint8)
    for j in range(4):
        out[:, :, 4 + j] = (sc[..., j] & 63) | ((sc[..., j + 4] >> 4) << 6)
        out[:, :, 8 + j] = (mn[..., j] & 63) | ((mn[..., j + 4] >> 4) << 6)
        out[:, :, 12 + j] = (sc[..., j + 4] & 15) | ((mn[..., j + 4] & 15) << 4)
    qq = np.asarray(q, np.uint8).reshape(rows, ns, 4, 2, 32)   # [group][half][l]
    out[:, :, 16:] = (qq[:, :, :, 0, :] | (qq[:, :, :, 1, :] << 4)).reshape(rows, ns, 128)
    d = _f16_val(d_bits)[..., None, None, None]
    dmin = _f16_val(dmin_bits)[..., None, None, None]
    scf = sc.reshape(rows, ns, 4, 2).astype(F32)[..., None]      # sub-block 2g+half
    mnf = mn.reshape(rows, ns, 4, 2).astype(F32)[..., None]
    ds = (d * scf).astype(F32)
    dm = (dmin * mnf).astype(F32)
    vals = ((ds * qq.astype(F32)).astype(F32) - dm).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def pack_q6_k(d_bits, sc, q):
    """Super-blocks of 256 (210 bytes): ql[128] low nibbles, qh[64] high 2-bit pairs, 16 int8
    scales, d fp16 at byte 208.  Element 128h + 32c + l (c = 0..3) takes its low nibble from
    ql[64h + l] (c = 0: low, c = 2: high nibble) or ql[64h + 32 + l] (c = 1: low, c = 3:
    high), its high two bits from bits 2c..2c+1 of qh[32h + l], and scale sc[8h + l/16 + 2c].
    sc [rows, ns, 16] int8; q [rows, ns*256] in 0..63."""
    rows, ns = d_bits.shape
    qq = np.asarray(q, np.uint8).reshape(rows, ns, 2, 4, 32)    # [half][c][l]
    out = np.zeros((rows, ns, 210), np.uint8)
    lo = qq & 15
    hi = qq >> 4
    ql = np.zeros((rows, ns, 2, 64), np.uint8)
    ql[..., 0:32] = lo[:, :, :, 0, :] | (lo[:, :, :, 2, :] << 4)
    ql[..., 32:64] = lo[:, :, :, 1, :] | (lo[:, :, :, 3, :] << 4)
    qh = hi[:, :, :, 0, :] | (hi[:, :, :, 1, :] << 2) | (hi[:, :, :, 2, :] << 4) | (hi[:, :, :, 3, :] << 6)
    out[:, :, 0:128] = ql.reshape(rows, ns, 128)
    out[:, :, 128:192] = qh.reshape(rows, ns, 64)
    out[:, :, 192:208] = np.asarray(sc, np.int8).view(np.uint8)
    out[:, :, 208:210] = np.asarray(d_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, ns, 2)
    d = _f16_val(d_bits)
    scv = np.asarray(sc, np.int8).astype(F32)                    # [rows, ns, 16]
    l = np.arange(32)
    vals = np.zeros((rows, ns, 2, 4, 32), F32)
    for h in range(2):
        for c in range(4):
            si = 8 * h + l // 16 + 2 * c
            ds = (d[..., None] * scv[:, :, si]).astype(F32)
            vals[:, :, h, c, :] = (ds * (qq[:, :, h, c, :].astype(F32) - 32)).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def _split_nibbles(idx):
    """[..., 32] codes -> [..., 16] bytes: code i in the low nibble of byte i, code 16+i in its
    high nibble (the split order of Q5_0, IQ4_NL, IQ4_XS sub-blocks and MXFP4)."""
    idx = np.asarray(idx, np.uint8)
    return (idx[..., :16] & 15) | ((idx[..., 16:] & 15) << 4)


def pack_q5_0(d_bits, q):
    """Blocks of 32 (22 bytes): d fp16, qh (uint32: bit i = bit 4 of element i), 16 bytes of
    split nibbles.  q [rows, nb*32] in 0..31; value (q - 16) * d."""
    rows, nb = d_bits.shape
    qq = np.asarray(q, np.int64).reshape(rows, nb, 32)
    out = np.zeros((rows, nb, 22), np.uint8)
    out[:, :, 0:2] = np.asarray(d_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, nb, 2)
    qh = ((qq >> 4) & 1) << np.arange(32)
    out[:, :, 2:6] = qh.sum(-1).astype(np.uint32)[..., None].view(np.uint8).reshape(rows, nb, 4)
    out[:, :, 6:] = _split_nibbles(qq & 15)
    vals = ((qq - 16).astype(F32) * _f16_val(d_bits)[..., None]).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def pack_q5_1(d_bits, m_bits, q):
    """Blocks of 32 (24 bytes): d fp16, m fp16, qh (uint32: bit i = bit 4 of element i), 16 bytes
    of split nibbles.  q [rows, nb*32] in 0..31; value q * d + m (two float roundings)."""
    rows, nb = d_bits.shape
    qq = np.asarray(q, np.int64).reshape(rows, nb, 32)
    out = np.zeros((rows, nb, 24), np.uint8)
    out[:, :, 0:2] = np.asarray(d_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:4] = np.asarray(m_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, nb, 2)
    qh = ((qq >> 4) & 1) << np.arange(32)
    out[:, :, 4:8] = qh.sum(-1).astype(np.uint32)[..., None].view(np.uint8).reshape(rows, nb, 4)
    out[:, :, 8:] = _split_nibbles(qq & 15)
    prod = (qq.astype(F32) * _f16_val(d_bits)[..., None]).astype(F32)
    vals = (prod + _f16_val(m_bits)[..., None]).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def pack_q2_k(d_bits, dmin_bits, sc, mn, q):
    """Super-blocks of 256 (84 bytes) in the reference's element order: 16 scale bytes (sub-block
    s of 16: low nibble sc, high nibble m), 64 quant bytes (element j at bits 2(j%4)..+1 of byte
    j/4), d fp16, dmin fp16.  sc, mn [rows, ns, 16] in 0..15, q [rows, ns*256] in 0..3; value
    ((d*sc)*q) - (dmin*m)."""
    rows, ns = d_bits.shape
    qq = np.asarray(q, np.int64).reshape(rows, ns, 64, 4)
    out = np.zeros((rows, ns, 84), np.uint8)
    out[:, :, 0:16] = (np.asarray(sc, np.int64) | (np.asarray(mn, np.int64) << 4)).astype(np.uint8)
    out[:, :, 16:80] = sum(qq[..., t] << (2 * t) for t in range(4)).astype(np.uint8)
    out[:, :, 80:82] = np.asarray(d_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, ns, 2)
    out[:, :, 82:84] = np.asarray(dmin_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, ns, 2)
    d = _f16_val(d_bits)[..., None]
    dmin = _f16_val(dmin_bits)[..., None]
    dsc = (d * np.asarray(sc, np.int64).astype(F32)).astype(F32)            # [rows, ns, 16]
    dm = (dmin * np.asarray(mn, np.int64).astype(F32)).astype(F32)
    qv = np.asarray(q, np.int64).reshape(rows, ns, 16, 16).astype(F32)
    vals = ((dsc[..., None] * qv).astype(F32) - dm[..., None]).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def pack_q3_k(d_bits, sc, q):
    """Super-blocks of 256 (110 bytes): hmask[32], qs[64], 12 bytes of 6-bit scales, d fp16.
    Element 128h + 32p + 16w + l (h < 2, p < 4, w < 2, l < 16) has its low two bits at bits
    2p..2p+1 of qs[32h + 16w + l] and its third bit at bit 4h + p of hmask[16w + l]; its
    sub-block is 8h + 2p + w.  Scale k: low four bits in byte k%8 (k < 8: low nibble, else
    high), top two bits at bits 2(k/4)..+1 of byte 8 + k%4.  sc [rows, ns, 16] in 0..63, q
    [rows, ns*256] in 0..7; value (d * (sc - 32)) * (q - 4)."""
    rows, ns = d_bits.shape
    qq = np.asarray(q, np.int64).reshape(rows, ns, 2, 4, 2, 16)     # [h][p][w][l]
    out = np.zeros((rows, ns, 110), np.int64)
    for h in range(2):
        for p in range(4):
            for w in range(2):
                out[:, :, 32 + 32 * h + 16 * w:32 + 32 * h + 16 * w + 16] |= (qq[:, :, h, p, w] & 3) << (2 * p)
                out[:, :, 16 * w:16 * w + 16] |= ((qq[:, :, h, p, w] >> 2) & 1) << (4 * h + p)
    scv = np.asarray(sc, np.int64)
    for k in range(16):
        out[:, :, 96 + k % 8] |= (scv[:, :, k] & 15) << (0 if k < 8 else 4)
        out[:, :, 104 + k % 4] |= ((scv[:, :, k] >> 4) & 3) << (2 * (k // 4))
    out = out.astype(np.uint8)
    out[:, :, 108:110] = np.asarray(d_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, ns, 2)
    d = _f16_val(d_bits)
    vals = np.zeros((rows, ns, 2, 4, 2, 16), F32)
    for h in range(2):
        for p in range(4):
            for w in range(2):
                dl = (d * (scv[:, :, 8 * h + 2 * p + w] - 32).astype(F32)).astype(F32)
                vals[:, :, h, p, w] = (dl[..., None] * (qq[:, :, h, p, w] - 4).astype(F32)).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def pack_q5_k(d_bits, dmin_bits, sc, mn, q):
    """Super-blocks of 256 (176 bytes): d, dmin fp16, the 12 scale/min bytes of Q4_K, qh[32]
    (bit 2g + s of byte l = bit 4 of element 64g + 32s + l), qs[128] (byte 32g + l: element
    64g + l low, 64g + 32 + l high).  q [rows, ns*256] in 0..31; value d*sc*q - dmin*m."""
    rows, ns = d_bits.shape
    q5 = np.asarray(q, np.int64)
    b4, _ = pack_q4_k(d_bits, dmin_bits, sc, mn, q5 & 15)
    b4 = b4.reshape(rows, ns, 144)
    out = np.zeros((rows, ns, 176), np.uint8)
    out[:, :, 0:16] = b4[:, :, 0:16]
    out[:, :, 48:176] = b4[:, :, 16:144]
    qq = q5.reshape(rows, ns, 4, 2, 32)                              # [g][s][l]
    qh = np.zeros((rows, ns, 32), np.int64)
    for g in range(4):
        for s_ in range(2):
            qh |= ((qq[:, :, g, s_] >> 4) & 1) << (2 * g + s_)
    out[:, :, 16:48] = qh.astype(np.uint8)
    d = _f16_val(d_bits)[..., None, None, None]
    dmin = _f16_val(dmin_bits)[..., None, None, None]
    ds = (d * np.asarray(sc, np.int64).reshape(rows, ns, 4, 2).astype(F32)[..., None]).astype(F32)
    dm = (dmin * np.asarray(mn, np.int64).reshape(rows, ns, 4, 2).astype(F32)[..., None]).astype(F32)
    vals = ((ds * qq.astype(F32)).astype(F32) - dm).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def pack_iq4_nl(d_bits, idx):
    """Blocks of 32 (18 bytes): d fp16, 16 bytes of split nibble codes; value d * codebook."""
    rows, nb = d_bits.shape
    ii = np.asarray(idx, np.int64).reshape(rows, nb, 32)
    out = np.zeros((rows, nb, 18), np.uint8)
    out[:, :, 0:2] = np.asarray(d_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = _split_nibbles(ii)
    vals = (_f16_val(d_bits)[..., None] * IQ4NL_VALUES[ii]).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def pack_iq4_xs(d_bits, ls, idx):
    """Super-blocks of 256 (136 bytes): d fp16, scales_h (uint16: bits 2ib..2ib+1 = top bits of
    sub-block ib's 6-bit scale), scales_l (4 bytes: low nibble of byte ib/2 for even ib, high
    for odd), qs[128] (sub-block ib of 32: bytes 16ib .. 16ib+15, split nibbles).  ls [rows,
    ns, 8] in 0..63; value (d * (ls - 32)) * codebook."""
    rows, ns = d_bits.shape
    lsv = np.asarray(ls, np.int64)
    ii = np.asarray(idx, np.int64).reshape(rows, ns, 8, 32)
    out = np.zeros((rows, ns, 136), np.uint8)
    out[:, :, 0:2] = np.asarray(d_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, ns, 2)
    sh = (((lsv >> 4) & 3) << (2 * np.arange(8))).sum(-1).astype(np.uint16)
    out[:, :, 2:4] = sh[..., None].view(np.uint8).reshape(rows, ns, 2)
    sl = (lsv[..., 0::2] & 15) | ((lsv[..., 1::2] & 15) << 4)
    out[:, :, 4:8] = sl.astype(np.uint8)
    out[:, :, 8:] = _split_nibbles(ii).reshape(rows, ns, 128)
    dl = (_f16_val(d_bits)[..., None] * (lsv - 32).astype(F32)).astype(F32)     # [rows, ns, 8]
    vals = (dl[..., None] * IQ4NL_VALUES[ii]).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def pack_mxfp4(e, idx):
    """Blocks of 32 (17 bytes): the E8M0 exponent byte e (scale 2^(e-127); 0 for e = 0 and
    e = 255), 16 bytes of split FP4 codes; value FP4 * scale."""
    rows, nb = e.shape
    ii = np.asarray(idx, np.int64).reshape(rows, nb, 32)
    ev = np.asarray(e, np.int64)
    out = np.zeros((rows, nb, 17), np.uint8)
    out[:, :, 0] = ev.astype(np.uint8)
    out[:, :, 1:] = _split_nibbles(ii)
    scale = np.where((ev == 0) | (ev == 255), 0.0, np.exp2((ev - 127).astype(np.float64))).astype(F32)
    vals = (FP4_VALUES[ii] * scale[..., None]).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def _parity_signs(i):
    """KSIGNS_IQ2XS[i]: the 7-bit index with an eighth bit making the count of set bits even."""
    i = np.asarray(i, np.int64)
    par = np.zeros_like(i)
    for k in range(7):
        par ^= (i >> k) & 1
    return i | (par << 7)


def _grid_bytes(grid, idx, width):
    """Byte j (j < width) of codebook entry idx: [..., width] as int64."""
    g = np.asarray(grid, np.uint64)[np.asarray(idx, np.int64)]
    return np.stack([((g >> np.uint64(8 * j)) & np.uint64(0xFF)).astype(np.int64) for j in range(width)], -1)


def pack_iq3_xxs(d_bits, qs, sign_idx, sc, grid):
    """Super-blocks of 256 (98 bytes): d fp16, 64 codebook indices (index 2l + h of 32-group
    ib32 at byte 8 ib32 + 2l + h, h = the 4-weight half of 8-weight group l), then per
    32-group a little-endian word: the 7-bit sign-pattern indices of its four 8-weight
    groups at bits 7l.. and the scale in bits 28-31.  qs [rows, ns, 64] in 0..255, sign_idx
    [rows, ns, 8, 4] in 0..127, sc [rows, ns, 8] in 0..15.  Element 32 ib32 + 8l + 4h + j is
    (d * (0.5 + sc) * 0.5) * grid[qs].byte(j), negated where bit 4h + j of the pattern is set
    (IQ3_XXSFloatTensor.getFloat)."""
    rows, ns = d_bits.shape
    qs = np.asarray(qs, np.int64)
    si = np.asarray(sign_idx, np.int64)
    sc = np.asarray(sc, np.int64)
    out = np.zeros((rows, ns, 98), np.uint8)
    out[:, :, 0:2] = np.asarray(d_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, ns, 2)
    out[:, :, 2:66] = qs.astype(np.uint8)
    aux = sum(si[..., l] << (7 * l) for l in range(4)) | (sc << 28)            # [rows, ns, 8]
    out[:, :, 66:98] = aux.astype(np.uint32)[..., None].view(np.uint8).reshape(rows, ns, 32)
    j = np.arange(256)
    ib32, l, h, jj = j // 32, (j % 32) // 8, (j % 8) // 4, j % 4
    d = _f16_val(d_bits)[..., None]
    db = ((d * (F32(0.5) + sc[:, :, ib32].astype(F32))).astype(F32) * F32(0.5)).astype(F32)
    gv = np.take_along_axis(_grid_bytes(grid, qs[:, :, ib32 * 8 + 2 * l + h], 4), jj[None, None, :, None], -1)[..., 0]
    neg = (_parity_signs(si[:, :, ib32, l]) >> (4 * h + jj)) & 1
    vals = (db * gv.astype(F32)).astype(F32)
    vals = np.where(neg == 1, -vals, vals).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def pack_iq3_s(d_bits, qs, qh, signs, sc, grid):
    """Super-blocks of 256 (110 bytes): d fp16, qs[64] (low 8 bits of index 2l + h of 32-group
    g at byte 8g + 2l + h), qh[8], signs[32] (one bit per weight: bit 4h + j of byte 4g + l),
    scales[4] (32-group g: nibble g%2 of byte g/2).  The ninth index bit is bit 2l + h of
    qh[g/4 + g%2]: IQ3_SFloatTensor.getFloat's OFF_QH + ib32/4 (+1 for the second group of a
    pair), as its dot and its CUDA kernel read it.  qs [rows, ns, 64], qh [rows, ns, 8],
    signs [rows, ns, 32] in 0..255, sc [rows, ns, 8] in 0..15.  Element 32g + 8l + 4h + j is
    (d * (1 + 2 sc)) * grid[index].byte(j), negated where its sign bit is set."""
    rows, ns = d_bits.shape
    qs, qh, signs, sc = (np.asarray(a, np.int64) for a in (qs, qh, signs, sc))
    out = np.zeros((rows, ns, 110), np.uint8)
    out[:, :, 0:2] = np.asarray(d_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, ns, 2)
    out[:, :, 2:66] = qs.astype(np.uint8)
    out[:, :, 66:74] = qh.astype(np.uint8)
    out[:, :, 74:106] = signs.astype(np.uint8)
    out[:, :, 106:110] = (sc[:, :, 0::2] | (sc[:, :, 1::2] << 4)).astype(np.uint8)
    j = np.arange(256)
    g, l, h, jj = j // 32, (j % 32) // 8, (j % 8) // 4, j % 4
    hi = (qh[:, :, g // 4 + g % 2] >> (2 * l + h)) & 1
    idx = qs[:, :, 8 * g + 2 * l + h] | (hi << 8)
    d = _f16_val(d_bits)[..., None]
    db = (d * (1 + 2 * sc[:, :, g]).astype(F32)).astype(F32)
    gv = np.take_along_axis(_grid_bytes(grid, idx, 4), jj[None, None, :, None], -1)[..., 0]
    neg = (signs[:, :, 4 * g + l] >> (4 * h + jj)) & 1
    vals = (db * gv.astype(F32)).astype(F32)
    vals = np.where(neg == 1, -vals, vals).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def pack_iq2_s(d_bits, qs, qh, signs, sc, grid):
    """Super-blocks of 256 (82 bytes): d fp16, qs[32] (low 8 bits of index l of 32-group ib32 at
    byte 4 ib32 + l), signs[32] (bit j of byte 4 ib32 + l), qh[8] (index bits 8-9 at bits
    2l..2l+1 of byte ib32), scales[8] (low nibble for the 32-group's first 16 weights, high
    for the last 16).  qs, signs [rows, ns, 32], qh [rows, ns, 8] in 0..255, sc [rows, ns, 16]
    in 0..15 (sc[2 ib32 + l/2]).  Element 32 ib32 + 8l + j is (d * (0.5 + sc) * 0.25) *
    grid[index].byte(j), negated where its sign bit is set (IQ2_SFloatTensor.getFloat)."""
    rows, ns = d_bits.shape
    qs, qh, signs, sc = (np.asarray(a, np.int64) for a in (qs, qh, signs, sc))
    out = np.zeros((rows, ns, 82), np.uint8)
    out[:, :, 0:2] = np.asarray(d_bits, np.uint16)[..., None].view(np.uint8).reshape(rows, ns, 2)
    out[:, :, 2:34] = qs.astype(np.uint8)
    out[:, :, 34:66] = signs.astype(np.uint8)
    out[:, :, 66:74] = qh.astype(np.uint8)
    out[:, :, 74:82] = (sc[:, :, 0::2] | (sc[:, :, 1::2] << 4)).astype(np.uint8)
    j = np.arange(256)
    ib32, l, jj = j // 32, (j % 32) // 8, j % 8
    idx = qs[:, :, 4 * ib32 + l] | (((qh[:, :, ib32] >> (2 * l)) & 3) << 8)
    d = _f16_val(d_bits)[..., None]
    dl = ((d * (F32(0.5) + sc[:, :, 2 * ib32 + l // 2].astype(F32))).astype(F32) * F32(0.25)).astype(F32)
    gv = np.take_along_axis(_grid_bytes(grid, idx, 8), jj[None, None, :, None], -1)[..., 0]
    neg = (signs[:, :, 4 * ib32 + l] >> jj) & 1
    vals = (dl * gv.astype(F32)).astype(F32)
    vals = np.where(neg == 1, -vals, vals).astype(F32)
    return out.reshape(rows, -1), vals.reshape(rows, -1)


def random_weights(t, rows, cols, rng, scale=0.05):
    """Random weights of GGML type t with magnitudes around `scale`: (bytes, float32 values)."""
    if t == GGML_F32:
        return pack_f32(rng.standard_normal((rows, cols)).astype(F32) * F32(scale))
    if t == GGML_F16:
        return pack_f16(rng.standard_normal((rows, cols)).astype(F32) * F32(scale))
    if t == GGML_BF16:
        return pack_bf16(rng.standard_normal((rows, cols)).astype(F32) * F32(scale))
    if t == GGML_Q8_0:
        nb = cols // 32
        d = _f16_bits(rng.uniform(0.5, 1.5, (rows, nb)) * scale / 64)
        return pack_q8_0(d, rng.integers(-128, 128, (rows, cols)).astype(np.int8))
    if t == GGML_Q4_0:
        nb = cols // 32
        d = _f16_bits(rng.uniform(0.5, 1.5, (rows, nb)) * scale / 4)
        return pack_q4_0(d, rng.integers(0, 16, (rows, cols)))
    if t == GGML_Q4_K:
        ns = cols // 256
        d = _f16_bits(rng.uniform(0.5, 1.5, (rows, ns)) * scale / 256)
        dmin = _f16_bits(rng.uniform(0.5, 1.5, (rows, ns)) * scale / 64)
        return pack_q4_k(d, dmin, rng.integers(0, 64, (rows, ns, 8)), rng.integers(0, 64, (rows, ns, 8)),
                         rng.integers(0, 16, (rows, cols)))
    if t == GGML_Q6_K:
        ns = cols // 256
        d = _f16_bits(rng.uniform(0.5, 1.5, (rows, ns)) * scale / 1024)
        return pack_q6_k(d, rng.integers(-128, 128, (rows, ns, 16)), rng.integers(0, 64, (rows, cols)))
    if t == GGML_Q5_0:
        nb = cols // 32
        d = _f16_bits(rng.uniform(0.5, 1.5, (rows, nb)) * scale / 8)
        return pack_q5_0(d, rng.integers(0, 32, (rows, cols)))
    if t == GGML_Q3_K:
        ns = cols // 256
        d = _f16_bits(rng.uniform(0.5, 1.5, (rows, ns)) * scale / 64)
        return pack_q3_k(d, rng.integers(0, 64, (rows, ns, 16)), rng.integers(0, 8, (rows, cols)))
    if t == GGML_Q5_K:
        ns = cols // 256
        d = _f16_bits(rng.uniform(0.5, 1.5, (rows, ns)) * scale / 512)
        dmin = _f16_bits(rng.uniform(0.5, 1.5, (rows, ns)) * scale / 64)
        return pack_q5_k(d, dmin, rng.integers(0, 64, (rows, ns, 8)), rng.integers(0, 64, (rows, ns, 8)),
                         rng.integers(0, 32, (rows, cols)))
    if t == GGML_IQ4_NL:
        nb = cols // 32
        d = _f16_bits(rng.uniform(0.5, 1.5, (rows, nb)) * scale / 64)
        return pack_iq4_nl(d, rng.integers(0, 16, (rows, cols)))
    if t == GGML_IQ4_XS:
        ns = cols // 256
        d = _f16_bits(rng.uniform(0.5, 1.5, (rows, ns)) * scale / 2048)
        return pack_iq4_xs(d, rng.integers(0, 64, (rows, ns, 8)), rng.integers(0, 16, (rows, cols)))
    if t == GGML_MXFP4:
        nb = cols // 32
        return pack_mxfp4(rng.integers(119, 124, (rows, nb)), rng.integers(0, 16, (rows, cols)))
    if t == GGML_Q5_1:
        nb = cols // 32
        d = _f16_bits(rng.uniform(0.5, 1.5, (rows, nb)) * scale / 8)
        m = _f16_bits(-rng.uniform(0.5, 1.5, (rows, nb)) * scale * 2)   # centred: q*d + m around 0
        return pack_q5_1(d, m, rng.integers(0, 32, (rows, cols)))
    if t == GGML_Q2_K:
        # centred, as a quantiser's are: dmin = d and m about 1.5 sc, the codes' mean
        ns = cols // 256
        d = _f16_bits(rng.uniform(0.5, 1.5, (rows, ns)) * scale / 8)
        sc = rng.integers(0, 11, (rows, ns, 16))
        mn = np.clip(np.rint(1.5 * sc) + rng.integers(-1, 2, sc.shape), 0, 15).astype(np.int64)
        return pack_q2_k(d, d, sc, mn, rng.integers(0, 4, (rows, cols)))
    if t in (GGML_IQ3_XXS, GGML_IQ3_S, GGML_IQ2_S):
        from oracle import oracle as orc   # the codebook
        ns = cols // 256
        grid = orc.iq_grid(t)
        u8 = lambda *shape: rng.integers(0, 256, (rows, ns) + shape)
        if t == GGML_IQ3_XXS:
            d = _f16_bits(rng.uniform(0.5, 1.5, (rows, ns)) * scale / 128)
            return pack_iq3_xxs(d, u8(64), rng.integers(0, 128, (rows, ns, 8, 4)),
                                rng.integers(0, 16, (rows, ns, 8)), grid)
        if t == GGML_IQ3_S:
            d = _f16_bits(rng.uniform(0.5, 1.5, (rows, ns)) * scale / 128)
            return pack_iq3_s(d, u8(64), u8(8), u8(32), rng.integers(0, 16, (rows, ns, 8)), grid)
        d = _f16_bits(rng.uniform(0.5, 1.5, (rows, ns)) * scale / 50)
        return pack_iq2_s(d, u8(32), u8(8), u8(32), rng.integers(0, 16, (rows, ns, 16)), grid)
    raise ValueError(t)
