/*
 * block_oracle.c -- TEST INFRASTRUCTURE ONLY (the same status as attn_oracle.c: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; nothing in the product
 * links or calls it).
 *
 * CPU restatement of the attention half of a transformer layer around the attention core:
 * TransformerBlock.forward's pre-attention RMSNorm, residual scale and residual add
 * (TransformerBlock.java, attention half), and Attention.forward's Q/K/V projections, biases
 * and output projection (Attention.java:76-110, 232-238), over projection weights in the GGUF
 * block formats of the reference's tensor classes (the tensor package's FloatTensor classes):
 *   F32 (0), F16 (1), Q4_0 (2), Q5_0 (6), Q5_1 (7), Q8_0 (8), Q2_K (10), Q3_K (11), Q4_K (12),
 *   Q5_K (13), Q6_K (14), IQ3_XXS (18), IQ4_NL (20), IQ3_S (21), IQ2_S (22), IQ4_XS (23),
 *   BF16 (30), MXFP4 (39)  (GGMLType ids).
 *
 * Dequantised weights are bit-identical to what each class's dot() stages (or getFloat()
 * returns); a row's dot follows the scalar classes of the java/ tree: F32 one
 * SimdVectorOps.dot over the row (orc_dot's 8-lane order), F16 and BF16 FloatTensor.dot's
 * sequential unfused sum, the block formats one orc_dot per block added in block order.  The
 * java21 Simd*FloatTensor classes, which the JVM prefers when the Vector API is present,
 * produce the same weights in another summation order; GPU parity on projections is to a
 * tolerance, so that choice only moves the last bits.
 *
 * Pinning: tests/test_block_oracle.py (dequantisation against an independent packer written
 * from each format's definition, Float16 against numpy, matmul and RMSNorm against float64,
 * the block against a float64 chain, residual identities).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "iq_grids.h"
#include "orc.h"

#define ORC_GGML_F32 0
#define ORC_GGML_F16 1
#define ORC_GGML_Q4_0 2
#define ORC_GGML_Q5_0 6
#define ORC_GGML_Q5_1 7
#define ORC_GGML_Q2_K 10
#define ORC_GGML_Q8_0 8
#define ORC_GGML_Q3_K 11
#define ORC_GGML_Q4_K 12
#define ORC_GGML_Q5_K 13
#define ORC_GGML_Q6_K 14
#define ORC_GGML_IQ4_NL 20
#define ORC_GGML_IQ3_XXS 18
#define ORC_GGML_IQ3_S 21
#define ORC_GGML_IQ2_S 22
#define ORC_GGML_IQ4_XS 23
#define ORC_GGML_BF16 30
#define ORC_GGML_MXFP4 39

/* IQ4_NLFloatTensor.KVALUES_IQ4NL (IQ4_NLFloatTensor.java:25-28), shared by IQ4_XS. */
static const float kvalues_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                        1,    13,   25,  38,  53,  69,  89,  113};
/* MXFP4FloatTensor.FP4_TABLE (MXFP4FloatTensor.java:39-42): E2M1 values by nibble. */
static const float fp4_e2m1[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                   -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

/* MXFP4FloatTensor.e8m0ToFloat (MXFP4FloatTensor.java:104-110): 2^(e - 127), 0 for e = 0
 * and e = 255. */
static float e8m0_to_f32(int e)
{
    if (e == 0 || e == 255) return 0.0f;
    uint32_t bits = (uint32_t)e << 23;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Float16.toFloat (Float16.java:11-34): sign, exponent and significand moved into float32,
 * subnormals normalised, infinities and NaNs kept. */
float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15);
    int exponent = (h >> 10) & 0x1F;
    uint32_t significand = h & 0x03FF;
    uint32_t bits;
    if (exponent == 0) {
        if (significand == 0) {
            bits = sign << 31;
            float f;
            memcpy(&f, &bits, 4);
            return f;
        }
        while ((significand & 0x0400) == 0) {
            significand <<= 1;
            exponent--;
        }
        significand &= 0x03FF;
        exponent++;
    } else if (exponent == 0x1F) {
        bits = (sign << 31) | 0x7F800000u | (significand << 13);
        float f;
        memcpy(&f, &bits, 4);
        return f;
    }
    bits = (sign << 31) | ((uint32_t)(exponent + (127 - 15)) << 23) | (significand << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float bf16_to_f32(uint16_t b)  /* BF16FloatTensor.getFloat: bits << 16 */
{
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Weights per block and bytes per block of a type (GGMLType.java:4-35); 0 if unsupported. */
int orc_ggml_block(int type, int *bytes)
{
    switch (type) {
    case ORC_GGML_F32: *bytes = 4; return 1;
    case ORC_GGML_F16: *bytes = 2; return 1;
    case ORC_GGML_BF16: *bytes = 2; return 1;
    case ORC_GGML_Q4_0: *bytes = 18; return 32;
    case ORC_GGML_Q5_0: *bytes = 22; return 32;
    case ORC_GGML_Q5_1: *bytes = 24; return 32;
    case ORC_GGML_Q2_K: *bytes = 84; return 256;
    case ORC_GGML_Q8_0: *bytes = 34; return 32;
    case ORC_GGML_Q3_K: *bytes = 110; return 256;
    case ORC_GGML_Q4_K: *bytes = 144; return 256;
    case ORC_GGML_Q5_K: *bytes = 176; return 256;
    case ORC_GGML_Q6_K: *bytes = 210; return 256;
    case ORC_GGML_IQ4_NL: *bytes = 18; return 32;
    case ORC_GGML_IQ4_XS: *bytes = 136; return 256;
    case ORC_GGML_MXFP4: *bytes = 17; return 32;
    case ORC_GGML_IQ3_XXS: *bytes = 98; return 256;
    case ORC_GGML_IQ3_S: *bytes = 110; return 256;
    case ORC_GGML_IQ2_S: *bytes = 82; return 256;
    default: *bytes = 0; return 0;
    }
}

/* IQ3_XXS sign patterns (IQGridTables.KSIGNS_IQ2XS): the 7-bit index with an eighth bit that
 * makes the count of set bits even (the pattern's eighth sign is implied by parity). */
static int orc_ksigns(int i)
{
    int p = 0;
    for (int k = 0; k < 7; k++) p ^= (i >> k) & 1;
    return i | (p << 7);
}
int orc_ksigns_entry(int i) { return orc_ksigns(i & 0x7F); }

/* Codebook entry `i` of an IQ format's table (for the table checks of the tests); 0 past the end. */
uint64_t orc_iq_grid(int type, int i)
{
    if (type == ORC_GGML_IQ3_XXS) return i >= 0 && i < 256 ? orc_iq3xxs_grid[i] : 0;
    if (type == ORC_GGML_IQ3_S) return i >= 0 && i < 512 ? orc_iq3s_grid[i] : 0;
    if (type == ORC_GGML_IQ2_S) return i >= 0 && i < 1024 ? orc_iq2s_grid[i] : 0;
    return 0;
}

/* Dequantised values of one block (`n` weights) exactly as the class's dot() stages them. */
static void dequant_block(int type, const uint8_t *b, float *out)
{
    switch (type) {
    case ORC_GGML_Q8_0: {   /* Q8_0FloatTensor.dot: scale * quant */
        float scale = orc_f16_to_f32(le16(b));
        for (int i = 0; i < 32; i++) out[i] = scale * (float)(int8_t)b[2 + i];
        break;
    }
    case ORC_GGML_Q4_0: {   /* Q4_0FloatTensor.dot: element 2i = low nibble of byte i */
        float scale = orc_f16_to_f32(le16(b));
        for (int i = 0; i < 16; i++) {
            int lo = b[2 + i] & 0x0F, hi = (b[2 + i] >> 4) & 0x0F;
            out[2 * i] = (float)(lo - 8) * scale;
            out[2 * i + 1] = (float)(hi - 8) * scale;
        }
        break;
    }
    case ORC_GGML_Q4_K: {   /* Q4_KFloatTensor.dot */
        float d = orc_f16_to_f32(le16(b)), dmin = orc_f16_to_f32(le16(b + 2));
        const uint8_t *sb = b + 4, *qs = b + 16;
        int sc[8], mn[8];
        for (int s = 0; s < 8; s++) {
            if (s < 4) {
                sc[s] = sb[s] & 0x3F;
                mn[s] = sb[s + 4] & 0x3F;
            } else {
                sc[s] = (sb[s + 4] & 0x0F) | ((sb[s - 4] >> 6) << 4);
                mn[s] = ((sb[s + 4] >> 4) & 0x0F) | ((sb[s] >> 6) << 4);
            }
        }
        for (int g = 0; g < 4; g++) {
            float ds0 = d * (float)sc[2 * g], dm0 = dmin * (float)mn[2 * g];
            float ds1 = d * (float)sc[2 * g + 1], dm1 = dmin * (float)mn[2 * g + 1];
            for (int l = 0; l < 32; l++) {
                int q = qs[g * 32 + l];
                out[g * 64 + l] = ds0 * (float)(q & 0x0F) - dm0;
                out[g * 64 + 32 + l] = ds1 * (float)((q >> 4) & 0x0F) - dm1;
            }
        }
        break;
    }
    case ORC_GGML_Q6_K: {   /* Q6_KFloatTensor.dot */
        const uint8_t *ql = b, *qh = b + 128;
        const int8_t *sc = (const int8_t *)(b + 192);
        float d = orc_f16_to_f32(le16(b + 208));
        for (int half = 0; half < 2; half++) {
            for (int l = 0; l < 32; l++) {
                int ql0 = ql[half * 64 + l], ql1 = ql[half * 64 + 32 + l], h = qh[half * 32 + l];
                int q0 = (ql0 & 0x0F) | (((h >> 0) & 3) << 4);
                int q1 = (ql1 & 0x0F) | (((h >> 2) & 3) << 4);
                int q2 = ((ql0 >> 4) & 0x0F) | (((h >> 4) & 3) << 4);
                int q3 = ((ql1 >> 4) & 0x0F) | (((h >> 6) & 3) << 4);
                int si = half * 8 + l / 16;
                float ds0 = d * (float)sc[si], ds1 = d * (float)sc[si + 2];
                float ds2 = d * (float)sc[si + 4], ds3 = d * (float)sc[si + 6];
                out[half * 128 + l] = ds0 * (float)(q0 - 32);
                out[half * 128 + 32 + l] = ds1 * (float)(q1 - 32);
                out[half * 128 + 64 + l] = ds2 * (float)(q2 - 32);
                out[half * 128 + 96 + l] = ds3 * (float)(q3 - 32);
            }
        }
        break;
    }
    case ORC_GGML_Q5_0: {   /* Q5_0FloatTensor.getFloat: (quant - 16) * scale, split nibbles */
        float scale = orc_f16_to_f32(le16(b));
        uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
        for (int i = 0; i < 32; i++) {
            int nib = i < 16 ? (b[6 + i] & 0x0F) : ((b[6 + i - 16] >> 4) & 0x0F);
            int q = nib | (int)(((qh >> i) & 1u) << 4);
            out[i] = (float)(q - 16) * scale;
        }
        break;
    }
    case ORC_GGML_Q5_1: {   /* Q5_1FloatTensor.getFloat: quant * scale + min, split nibbles */
        float scale = orc_f16_to_f32(le16(b)), mn = orc_f16_to_f32(le16(b + 2));
        uint32_t qh = (uint32_t)b[4] | ((uint32_t)b[5] << 8) | ((uint32_t)b[6] << 16) | ((uint32_t)b[7] << 24);
        for (int i = 0; i < 32; i++) {
            int nib = i < 16 ? (b[8 + i] & 0x0F) : ((b[8 + i - 16] >> 4) & 0x0F);
            int q = nib | (int)(((qh >> i) & 1u) << 4);
            out[i] = (float)q * scale + mn;
        }
        break;
    }
    case ORC_GGML_Q2_K: {   /* Q2_KFloatTensor.getFloat: d * sc * q - dmin * m, element j at
                               bits 2(j%4) of qs byte j/4, scale byte j/16 */
        float d = orc_f16_to_f32(le16(b + 80)), dmin = orc_f16_to_f32(le16(b + 82));
        for (int j = 0; j < 256; j++) {
            int sc = b[j / 16] & 0x0F, m = b[j / 16] >> 4;
            int q = (b[16 + j / 4] >> (2 * (j % 4))) & 3;
            out[j] = d * (float)sc * (float)q - dmin * (float)m;
        }
        break;
    }
    case ORC_GGML_Q3_K: {   /* Q3_KFloatTensor.dot: dl = d * (sc - 32), value dl * q */
        const uint8_t *hm = b, *qs = b + 32, *raw = b + 96;
        float d = orc_f16_to_f32(le16(b + 108));
        int sc[16];
        for (int i = 0; i < 8; i++) {
            sc[i] = raw[i] & 0x0F;
            sc[i + 8] = raw[i] >> 4;
        }
        for (int i = 0; i < 4; i++) {
            int v = raw[8 + i];
            sc[i] |= (v & 3) << 4;
            sc[i + 4] |= ((v >> 2) & 3) << 4;
            sc[i + 8] |= ((v >> 4) & 3) << 4;
            sc[i + 12] |= ((v >> 6) & 3) << 4;
        }
        for (int half = 0; half < 2; half++)
            for (int pair = 0; pair < 4; pair++)
                for (int w16 = 0; w16 < 2; w16++) {
                    float dl = d * (float)(sc[half * 8 + pair * 2 + w16] - 32);
                    for (int l = 0; l < 16; l++) {
                        int low = (qs[half * 32 + w16 * 16 + l] >> (2 * pair)) & 3;
                        int hb = (hm[w16 * 16 + l] >> (half * 4 + pair)) & 1;
                        out[half * 128 + pair * 32 + w16 * 16 + l] = dl * (float)((low | (hb << 2)) - 4);
                    }
                }
        break;
    }
    case ORC_GGML_Q5_K: {   /* Q5_KFloatTensor.dot: ds * q - dm, q = nibble | qh bit << 4 */
        float d = orc_f16_to_f32(le16(b)), dmin = orc_f16_to_f32(le16(b + 2));
        const uint8_t *sb = b + 4, *qh = b + 16, *qs = b + 48;
        int sc[8], mn[8];
        for (int s = 0; s < 8; s++) {
            if (s < 4) {
                sc[s] = sb[s] & 0x3F;
                mn[s] = sb[s + 4] & 0x3F;
            } else {
                sc[s] = (sb[s + 4] & 0x0F) | ((sb[s - 4] >> 6) << 4);
                mn[s] = ((sb[s + 4] >> 4) & 0x0F) | ((sb[s] >> 6) << 4);
            }
        }
        for (int g = 0; g < 4; g++) {
            float ds0 = d * (float)sc[2 * g], dm0 = dmin * (float)mn[2 * g];
            float ds1 = d * (float)sc[2 * g + 1], dm1 = dmin * (float)mn[2 * g + 1];
            for (int l = 0; l < 32; l++) {
                int q0 = (qs[g * 32 + l] & 0x0F) | (((qh[l] >> (2 * g)) & 1) << 4);
                int q1 = ((qs[g * 32 + l] >> 4) & 0x0F) | (((qh[l] >> (2 * g + 1)) & 1) << 4);
                out[g * 64 + l] = ds0 * (float)q0 - dm0;
                out[g * 64 + 32 + l] = ds1 * (float)q1 - dm1;
            }
        }
        break;
    }
    case ORC_GGML_IQ4_NL: {   /* IQ4_NLFloatTensor.dot: scale * KVALUES[nibble], split nibbles */
        float scale = orc_f16_to_f32(le16(b));
        for (int i = 0; i < 16; i++) {
            out[i] = scale * kvalues_iq4nl[b[2 + i] & 0x0F];
            out[i + 16] = scale * kvalues_iq4nl[(b[2 + i] >> 4) & 0x0F];
        }
        break;
    }
    case ORC_GGML_IQ4_XS: {   /* IQ4_XSFloatTensor.dot: dl = d * (ls - 32), split nibbles per 32 */
        float d = orc_f16_to_f32(le16(b));
        int scales_h = le16(b + 2);
        for (int ib = 0; ib < 8; ib++) {
            int sl = b[4 + ib / 2];
            int low4 = (ib & 1) ? ((sl >> 4) & 0x0F) : (sl & 0x0F);
            int ls = low4 | (((scales_h >> (2 * ib)) & 3) << 4);
            float dl = d * (float)(ls - 32);
            for (int i = 0; i < 16; i++) {
                int p = b[8 + ib * 16 + i];
                out[ib * 32 + i] = dl * kvalues_iq4nl[p & 0x0F];
                out[ib * 32 + 16 + i] = dl * kvalues_iq4nl[(p >> 4) & 0x0F];
            }
        }
        break;
    }
    case ORC_GGML_MXFP4: {   /* MXFP4FloatTensor.dot: FP4_TABLE[nibble] * 2^(e - 127), split */
        float scale = e8m0_to_f32(b[0]);
        for (int i = 0; i < 16; i++) {
            out[i] = fp4_e2m1[b[1 + i] & 0x0F] * scale;
            out[i + 16] = fp4_e2m1[(b[1 + i] >> 4) & 0x0F] * scale;
        }
        break;
    }
    case ORC_GGML_IQ3_XXS: {   /* IQ3_XXSFloatTensor.dot (IQ3_XXSFloatTensor.java:77-113) */
        /* 64 codebook indices at 2, then per 32 weights a little-endian word at 66 + 4*ib32:
         * four 7-bit sign-pattern indices (bits 7l..7l+6) and the scale in bits 28..31 */
        float d = orc_f16_to_f32(le16(b));
        const uint8_t *qs = b + 2, *sas = b + 66;
        for (int ib32 = 0; ib32 < 8; ib32++) {
            uint32_t aux = (uint32_t)sas[4 * ib32] | ((uint32_t)sas[4 * ib32 + 1] << 8) |
                           ((uint32_t)sas[4 * ib32 + 2] << 16) | ((uint32_t)sas[4 * ib32 + 3] << 24);
            float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
            for (int l = 0; l < 4; l++) {
                int signs = orc_ksigns((int)((aux >> (7 * l)) & 0x7F));
                uint32_t g1 = orc_iq3xxs_grid[qs[ib32 * 8 + 2 * l]];
                uint32_t g2 = orc_iq3xxs_grid[qs[ib32 * 8 + 2 * l + 1]];
                for (int j = 0; j < 4; j++) {
                    out[ib32 * 32 + l * 8 + j] = db * (float)((g1 >> (8 * j)) & 0xFF) * ((signs >> j) & 1 ? -1.0f : 1.0f);
                    out[ib32 * 32 + l * 8 + 4 + j] =
                        db * (float)((g2 >> (8 * j)) & 0xFF) * ((signs >> (j + 4)) & 1 ? -1.0f : 1.0f);
                }
            }
        }
        break;
    }
    case ORC_GGML_IQ3_S: {   /* IQ3_SFloatTensor.dot (IQ3_SFloatTensor.java:110-170) */
        /* qs (low 8 index bits) at 2, qh (9th bits) at 66, sign bits at 74, 4-bit scales at 106.
         * The 9th bits of 32-group g come from qh[(g >> 2) + (g & 1)]: the reference's
         * OFF_QH + ib32/4 (+1 for the pair's second group), which its CUDA kernel
         * (matmul_iq3_s.cu:129, 158) shares; ggml's dequantiser reads qh[g]. */
        float d = orc_f16_to_f32(le16(b));
        const uint8_t *qs = b + 2, *qh = b + 66, *sg = b + 74, *scl = b + 106;
        for (int g = 0; g < 8; g++) {
            int sb = scl[g / 2];
            float db = d * (float)(1 + 2 * ((g & 1) ? (sb >> 4) & 0x0F : sb & 0x0F));
            int h = qh[(g >> 2) + (g & 1)];
            for (int l = 0; l < 4; l++) {
                uint32_t g1 = orc_iq3s_grid[qs[g * 8 + 2 * l] | ((h << (8 - 2 * l)) & 256)];
                uint32_t g2 = orc_iq3s_grid[qs[g * 8 + 2 * l + 1] | ((h << (7 - 2 * l)) & 256)];
                int signs = sg[g * 4 + l];
                for (int j = 0; j < 4; j++) {
                    out[g * 32 + l * 8 + j] = db * (float)((g1 >> (8 * j)) & 0xFF) * ((signs >> j) & 1 ? -1.0f : 1.0f);
                    out[g * 32 + l * 8 + 4 + j] =
                        db * (float)((g2 >> (8 * j)) & 0xFF) * ((signs >> (j + 4)) & 1 ? -1.0f : 1.0f);
                }
            }
        }
        break;
    }
    case ORC_GGML_IQ2_S: {   /* IQ2_SFloatTensor.dot (IQ2_SFloatTensor.java:84-113) */
        /* qs (low 8 index bits) at 2, sign bits at 34, qh (bits 8-9 of the 4 indices of a
         * 32-group, two bits each) at 66, two 4-bit scales per 32-group at 74 */
        float d = orc_f16_to_f32(le16(b));
        const uint8_t *qs = b + 2, *sg = b + 34, *qh = b + 66, *scl = b + 74;
        for (int ib32 = 0; ib32 < 8; ib32++) {
            float db0 = d * (0.5f + (float)(scl[ib32] & 0x0F)) * 0.25f;
            float db1 = d * (0.5f + (float)((scl[ib32] >> 4) & 0x0F)) * 0.25f;
            for (int l = 0; l < 4; l++) {
                float dl = l < 2 ? db0 : db1;
                uint64_t gr = orc_iq2s_grid[qs[ib32 * 4 + l] | ((qh[ib32] << (8 - 2 * l)) & 0x300)];
                int signs = sg[ib32 * 4 + l];
                for (int j = 0; j < 8; j++)
                    out[ib32 * 32 + l * 8 + j] = dl * (float)((gr >> (8 * j)) & 0xFF) * ((signs >> j) & 1 ? -1.0f : 1.0f);
            }
        }
        break;
    }
    default: break;
    }
}

/* Dequantised row of `cols` weights (cols a multiple of the block size). */
int orc_dequant_row(int type, const uint8_t *row, int cols, float *out)
{
    int bytes, n = orc_ggml_block(type, &bytes);
    if (n == 0 || cols % n) return -1;
    if (type == ORC_GGML_F32) {
        memcpy(out, row, sizeof(float) * (size_t)cols);
    } else if (type == ORC_GGML_F16) {
        for (int i = 0; i < cols; i++) out[i] = orc_f16_to_f32(le16(row + 2 * i));
    } else if (type == ORC_GGML_BF16) {
        for (int i = 0; i < cols; i++) out[i] = bf16_to_f32(le16(row + 2 * i));
    } else {
        for (int b = 0; b < cols / n; b++) dequant_block(type, row + (size_t)b * bytes, out + b * n);
    }
    return 0;
}

/* One output row: FloatTensor.dot of the row with x, in the order the scalar class uses. */
static float row_dot(int type, const uint8_t *row, int cols, const float *x, float *tmp)
{
    int bytes, n = orc_ggml_block(type, &bytes);
    if (type == ORC_GGML_F32) {               /* F32FloatTensor.dot: one SimdVectorOps.dot */
        memcpy(tmp, row, sizeof(float) * (size_t)cols);
        return orc_dot(tmp, x, cols);
    }
    if (type == ORC_GGML_F16 || type == ORC_GGML_BF16) {   /* FloatTensor.dot */
        float sum = 0.0f;
        for (int i = 0; i < cols; i++) {
            float w = type == ORC_GGML_F16 ? orc_f16_to_f32(le16(row + 2 * i))
                                           : bf16_to_f32(le16(row + 2 * i));
            sum += w * x[i];
        }
        return sum;
    }
    float result = 0.0f;                       /* block formats: result += dot(block) */
    if (type == ORC_GGML_Q5_0) {              /* Q5_0FloatTensor.dot: scale * sequential sum */
        for (int b = 0; b < cols / n; b++) {
            const uint8_t *blk = row + (size_t)b * bytes;
            float scale = orc_f16_to_f32(le16(blk));
            uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                          ((uint32_t)blk[5] << 24);
            float sum = 0.0f;
            for (int j = 0; j < 16; j++) {
                int q0 = (blk[6 + j] & 0x0F) | (int)(((qh >> j) & 1u) << 4);
                int q1 = ((blk[6 + j] >> 4) & 0x0F) | (int)(((qh >> (j + 16)) & 1u) << 4);
                sum += (float)(q0 - 16) * x[b * 32 + j];
                sum += (float)(q1 - 16) * x[b * 32 + j + 16];
            }
            result += scale * sum;
        }
        return result;
    }
    if (type == ORC_GGML_Q5_1) {   /* Q5_1FloatTensor.dot: scale * blockSum + min * otherSum */
        for (int b = 0; b < cols / n; b++) {
            const uint8_t *blk = row + (size_t)b * bytes;
            float scale = orc_f16_to_f32(le16(blk)), mn = orc_f16_to_f32(le16(blk + 2));
            uint32_t qh = (uint32_t)blk[4] | ((uint32_t)blk[5] << 8) | ((uint32_t)blk[6] << 16) |
                          ((uint32_t)blk[7] << 24);
            float bsum = 0.0f, osum = 0.0f;
            for (int j = 0; j < 16; j++) {
                int q0 = (blk[8 + j] & 0x0F) | (int)(((qh >> j) & 1u) << 4);
                int q1 = ((blk[8 + j] >> 4) & 0x0F) | (int)(((qh >> (j + 16)) & 1u) << 4);
                bsum += (float)q0 * x[b * 32 + j];
                bsum += (float)q1 * x[b * 32 + j + 16];
                osum += x[b * 32 + j] + x[b * 32 + j + 16];
            }
            result += scale * bsum + mn * osum;
        }
        return result;
    }
    if (type == ORC_GGML_Q2_K) {   /* Q2_KFloatTensor.dotQ2KF32: per sub-block of 16 */
        for (int b = 0; b < cols / n; b++) {
            const uint8_t *blk = row + (size_t)b * bytes;
            float d = orc_f16_to_f32(le16(blk + 80)), dmin = orc_f16_to_f32(le16(blk + 82));
            for (int sb = 0; sb < 16; sb++) {
                int sc = blk[sb] & 0x0F, m = blk[sb] >> 4;
                float sum_q = 0.0f, sum_f = 0.0f;
                for (int i = 0; i < 16; i++) {
                    int j = sb * 16 + i;
                    int q = (blk[16 + j / 4] >> (2 * (j % 4))) & 3;
                    float f = x[b * 256 + j];
                    sum_q += (float)q * f;
                    sum_f += f;
                }
                result += d * (float)sc * sum_q - dmin * (float)m * sum_f;
            }
        }
        return result;
    }
    for (int b = 0; b < cols / n; b++) {
        dequant_block(type, row + (size_t)b * bytes, tmp);
        result += orc_dot(tmp, x + b * n, n);
    }
    return result;
}

/* FloatTensor.matmulParallel (FloatTensor.java:61-67): out[row] += dot(row, x) for each of
 * `rows` rows of `cols` weights stored row after row. */
int orc_matmul(int type, const uint8_t *w, int rows, int cols, const float *x, float *out)
{
    int bytes, n = orc_ggml_block(type, &bytes);
    if (n == 0 || cols % n) return -1;
    size_t row_bytes = (size_t)(cols / n) * bytes;
    float *tmp = (float *)malloc(sizeof(float) * (size_t)cols);
    for (int r = 0; r < rows; r++) out[r] += row_dot(type, w + (size_t)r * row_bytes, cols, x, tmp);
    free(tmp);
    return 0;
}

/* SimdVectorOps.rmsnorm (SimdVectorOps.java:50-74): ss in orc_dot's 8-lane order,
 * r = 1/(float)sqrt(ss/size + eps), out = (x*r)*w.  out may alias x. */
void orc_rmsnorm(float *out, const float *x, const float *w, int size, float eps)
{
    float ss = orc_dot(x, x, size);
    ss = 1.0f / (float)sqrt((double)(ss / (float)size + eps));
    for (int i = 0; i < size; i++) out[i] = x[i] * ss * w[i];
}

/* ---- the reference GPU's Q8_1 input (its default "dp4a" matvecs) ----------------------------
 * CudaForwardPass (CudaForwardPass.java:783-790: cuda.dp4a defaults to true; :1998-2090: Q4_K,
 * Q8_0, Q5_0, Q3_K, Q5_K, IQ4_NL and IQ4_XS take the int8 kernels, Q6_K stays on the fp32 one
 * unless cuda.dp4a.q6 is set) normalises x, quantises it to Q8_1 blocks (rmsnorm_quantize.cu,
 * quantize_q8.cu) and runs matmul_<type>_dp4a*.cu: exact int8 dot products per 32 values,
 * scaled in float.  The
 * restatement fixes two reduction orders the reference leaves to its launch geometry (and to
 * CUDA's rsqrtf): the norm's sum of squares and each block's sum, both in the library's
 * staging order, so that the quantised bytes are the GPU's exactly. */

/* The library's staged RMSNorm: 256 threads, thread t sums the squares of the 4-value chunks
 * c = t, t+256, ... with FMAs (values in order); each 64-thread wave reduces by a butterfly
 * (xor 1, 2, 4, 8, 16, 32); the four wave totals are added in order; r = 1/(float)sqrt((double)
 * (ss/size + eps)); out = (x*r)*w (size a multiple of 4). */
void orc_rmsnorm_staged(float *out, const float *x, const float *w, int size, float eps)
{
    float part[256], red[4];
    const int n4 = size / 4;
    for (int t = 0; t < 256; t++) {
        float s = 0.0f;
        for (int c = t; c < n4; c += 256)
            for (int e = 0; e < 4; e++) s = fmaf(x[4 * c + e], x[4 * c + e], s);
        part[t] = s;
    }
    for (int wv = 0; wv < 4; wv++) {
        float v[64], nv[64];
        memcpy(v, part + 64 * wv, sizeof(v));
        for (int off = 1; off < 64; off <<= 1) {
            for (int i = 0; i < 64; i++) nv[i] = v[i] + v[i ^ off];
            memcpy(v, nv, sizeof(v));
        }
        red[wv] = v[0];
    }
    float tot = red[0];
    for (int wv = 1; wv < 4; wv++) tot = tot + red[wv];
    float v = tot / (float)size;
    v = v + eps;
    const float r = 1.0f / (float)sqrt((double)v);
    for (int i = 0; i < size; i++) out[i] = (x[i] * r) * w[i];
}

/* Q8_1 blocks of 32 values (quantize_q8.cu, rmsnorm_quantize.cu): d = max|x|/127, quants
 * rint(x * (127/max|x|)) clamped to +-127 (all 0 when max|x| = 0), s = the block's sum, here
 * ((x0 + x1) + (x2 + x3)) per 4 values, then a butterfly over the block's 8 groups (xor 4, 2,
 * 1).  n a multiple of 32. */
void orc_quantize_q8_1(const float *x, int n, int8_t *q, float *d, float *s)
{
    for (int b = 0; b < n / 32; b++) {
        const float *xb = x + 32 * b;
        float m = 0.0f;
        for (int i = 0; i < 32; i++) m = fmaxf(m, fabsf(xb[i]));
        const float inv = m > 0.0f ? 127.0f / m : 0.0f;
        for (int i = 0; i < 32; i++) {
            float r = rintf(xb[i] * inv);
            r = r > 127.0f ? 127.0f : (r < -127.0f ? -127.0f : r);
            q[32 * b + i] = (int8_t)r;
        }
        d[b] = m / 127.0f;
        float g[8], ng[8];
        for (int t = 0; t < 8; t++) g[t] = (xb[4 * t] + xb[4 * t + 1]) + (xb[4 * t + 2] + xb[4 * t + 3]);
        for (int off = 4; off > 0; off >>= 1) {
            for (int t = 0; t < 8; t++) ng[t] = g[t] + g[t ^ off];
            memcpy(g, ng, sizeof(g));
        }
        s[b] = g[0];
    }
}

/* get_scale_min_k4 of the Q4_K head's 12 scale bytes (q = head + 4): sub-block j's 6-bit
 * scale and min. */
static void q4k_scale_min(const uint8_t *q, int j, int *sc, int *m)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* The int8 matvecs on a Q8_1 input (q [cols], d and s [cols/32]); out[row] += the row's dot:
 *   Q4_K (matmul_q4_k_dp4a.cu): per sub-block j of 32, ((d*sc_j)*d_x)*dp_j - (dmin*m_j)*s_x
 *   Q5_K (matmul_q5_k_dp4a.cu:123-124): the same, q = nibble | fifth bit << 4
 *   Q8_0 (matmul_q8_0_dp4a.cu): per block, (d*d_x)*dp
 *   Q5_0 (matmul_q5_0_dp4a_smem.cu:111): per block, (d*d_x)*dp, q = (nibble | bit << 4) - 16
 *   IQ4_NL (matmul_iq4_nl_dp4a.cu:100): per block, (d*d_x)*dp, q = KVALUES[nibble]
 *   IQ4_XS (matmul_iq4_xs_dp4a_mw.cu:115): per sub-block ib, (dl*d_x)*dp, dl = d*(ls - 32)
 *   Q3_K (matmul_q3_k_dp4a.cu:142): per block of 32 (halves w = 0, 1 of 16 with scales dl_w =
 *        d*(sc - 32)), (dl_0*d_x)*dp_0 + (dl_1*d_x)*dp_1, q = (2 bits | high bit << 2) - 4
 * with dp the exact integer dot of the block's weights with the input's quants, added over
 * the row's blocks in order (the reference adds per lane, then a warp tree).  -1 for other
 * types. */
int orc_matmul_q8_1(int type, const uint8_t *w, int rows, int cols, const int8_t *q,
                    const float *d, const float *s, float *out)
{
    if (type == ORC_GGML_Q4_K) {
        if (cols % 256) return -1;
        const int ns = cols / 256;
        for (int r = 0; r < rows; r++) {
            float acc = 0.0f;
            for (int b = 0; b < ns; b++) {
                const uint8_t *blk = w + ((size_t)r * ns + b) * 144;
                const float dd = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
                const float dmin = orc_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
                for (int g = 0; g < 4; g++)
                    for (int h = 0; h < 2; h++) {   /* sub-block 2g + h: nibble h of bytes 32g .. 32g+31 */
                        const int j = 2 * g + h, xb = b * 8 + j;
                        int dp = 0;
                        for (int l = 0; l < 32; l++) {
                            const int nib = (blk[16 + 32 * g + l] >> (4 * h)) & 15;
                            dp += nib * q[32 * xb + l];
                        }
                        int sc, mn;
                        q4k_scale_min(blk + 4, j, &sc, &mn);
                        acc += ((dd * (float)sc) * d[xb]) * (float)dp - (dmin * (float)mn) * s[xb];
                    }
            }
            out[r] += acc;
        }
        return 0;
    }
    if (type == ORC_GGML_Q5_K) {
        if (cols % 256) return -1;
        const int ns = cols / 256;
        for (int r = 0; r < rows; r++) {
            float acc = 0.0f;
            for (int b = 0; b < ns; b++) {
                const uint8_t *blk = w + ((size_t)r * ns + b) * 176, *qh = blk + 16, *qs = blk + 48;
                const float dd = orc_f16_to_f32(le16(blk)), dmin = orc_f16_to_f32(le16(blk + 2));
                for (int g = 0; g < 4; g++)
                    for (int h = 0; h < 2; h++) {   /* sub-block 2g + h: nibble h, qh bit 2g + h */
                        const int j = 2 * g + h, xb = b * 8 + j;
                        int dp = 0;
                        for (int l = 0; l < 32; l++) {
                            const int q5 = ((qs[32 * g + l] >> (4 * h)) & 15) | (((qh[l] >> j) & 1) << 4);
                            dp += q5 * q[32 * xb + l];
                        }
                        int sc, mn;
                        q4k_scale_min(blk + 4, j, &sc, &mn);
                        acc += ((dd * (float)sc) * d[xb]) * (float)dp - (dmin * (float)mn) * s[xb];
                    }
            }
            out[r] += acc;
        }
        return 0;
    }
    if (type == ORC_GGML_Q3_K) {
        if (cols % 256) return -1;
        const int ns = cols / 256;
        for (int r = 0; r < rows; r++) {
            float acc = 0.0f;
            for (int b = 0; b < ns; b++) {
                const uint8_t *blk = w + ((size_t)r * ns + b) * 110, *hm = blk, *qs = blk + 32, *raw = blk + 96;
                const float dd = orc_f16_to_f32(le16(blk + 108));
                for (int hf = 0; hf < 2; hf++)
                    for (int pair = 0; pair < 4; pair++) {   /* Q8_1 block 8b + 4hf + pair */
                        const int xb = b * 8 + hf * 4 + pair;
                        float dl[2];
                        int dp[2] = {0, 0};
                        for (int w16 = 0; w16 < 2; w16++) {
                            const int si = hf * 8 + pair * 2 + w16;   /* decodeQ3KScale */
                            const int lo = si < 8 ? (raw[si & 7] & 15) : (raw[si & 7] >> 4);
                            const int hi = (raw[8 + (si & 3)] >> ((si >> 2) * 2)) & 3;
                            dl[w16] = dd * (float)((lo | (hi << 4)) - 32);
                            for (int l = 0; l < 16; l++) {
                                const int low = (qs[hf * 32 + w16 * 16 + l] >> (2 * pair)) & 3;
                                const int hb = (hm[w16 * 16 + l] >> (hf * 4 + pair)) & 1;
                                dp[w16] += ((low | (hb << 2)) - 4) * q[32 * xb + 16 * w16 + l];
                            }
                        }
                        acc += (dl[0] * d[xb]) * (float)dp[0] + (dl[1] * d[xb]) * (float)dp[1];
                    }
            }
            out[r] += acc;
        }
        return 0;
    }
    if (type == ORC_GGML_Q5_0 || type == ORC_GGML_IQ4_NL) {
        if (cols % 32) return -1;
        const int nb = cols / 32, bs = type == ORC_GGML_Q5_0 ? 22 : 18;
        for (int r = 0; r < rows; r++) {
            float acc = 0.0f;
            for (int b = 0; b < nb; b++) {
                const uint8_t *blk = w + ((size_t)r * nb + b) * bs;
                const float dd = orc_f16_to_f32(le16(blk));
                int dp = 0;
                if (type == ORC_GGML_Q5_0) {
                    const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) |
                                        ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
                    for (int l = 0; l < 16; l++) {
                        const int q0 = ((blk[6 + l] & 15) | (int)(((qh >> l) & 1u) << 4)) - 16;
                        const int q1 = ((blk[6 + l] >> 4) | (int)(((qh >> (l + 16)) & 1u) << 4)) - 16;
                        dp += q0 * q[32 * b + l] + q1 * q[32 * b + 16 + l];
                    }
                } else {
                    for (int l = 0; l < 16; l++)
                        dp += (int)kvalues_iq4nl[blk[2 + l] & 15] * q[32 * b + l] +
                              (int)kvalues_iq4nl[blk[2 + l] >> 4] * q[32 * b + 16 + l];
                }
                acc += (dd * d[b]) * (float)dp;
            }
            out[r] += acc;
        }
        return 0;
    }
    if (type == ORC_GGML_IQ4_XS) {
        if (cols % 256) return -1;
        const int ns = cols / 256;
        for (int r = 0; r < rows; r++) {
            float acc = 0.0f;
            for (int b = 0; b < ns; b++) {
                const uint8_t *blk = w + ((size_t)r * ns + b) * 136;
                const float dd = orc_f16_to_f32(le16(blk));
                const uint32_t sh = le16(blk + 2);
                const uint32_t sl = (uint32_t)blk[4] | ((uint32_t)blk[5] << 8) | ((uint32_t)blk[6] << 16) |
                                    ((uint32_t)blk[7] << 24);
                for (int ib = 0; ib < 8; ib++) {
                    const int ls = (int)((sl >> (4 * ib)) & 15) | (int)(((sh >> (2 * ib)) & 3) << 4);
                    const float dl = dd * (float)(ls - 32);
                    const int xb = b * 8 + ib;
                    int dp = 0;
                    for (int l = 0; l < 16; l++)
                        dp += (int)kvalues_iq4nl[blk[8 + 16 * ib + l] & 15] * q[32 * xb + l] +
                              (int)kvalues_iq4nl[blk[8 + 16 * ib + l] >> 4] * q[32 * xb + 16 + l];
                    acc += (dl * d[xb]) * (float)dp;
                }
            }
            out[r] += acc;
        }
        return 0;
    }
    if (type == ORC_GGML_Q8_0) {
        if (cols % 32) return -1;
        const int nb = cols / 32;
        for (int r = 0; r < rows; r++) {
            float acc = 0.0f;
            for (int b = 0; b < nb; b++) {
                const uint8_t *blk = w + ((size_t)r * nb + b) * 34;
                const float dd = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
                int dp = 0;
                for (int l = 0; l < 32; l++) dp += (int)(int8_t)blk[2 + l] * q[32 * b + l];
                acc += (dd * d[b]) * (float)dp;
            }
            out[r] += acc;
        }
        return 0;
    }
    return -1;
}

/* The types the reference GPU runs on its Q8_1 input (CudaForwardPass.java:216-226 with
 * :2029-2038: Q6_K's int8 kernel is opt-in). */
int orc_q8_1_routed(int type)
{
    return type == ORC_GGML_Q4_K || type == ORC_GGML_Q8_0 || type == ORC_GGML_Q5_0 ||
           type == ORC_GGML_Q3_K || type == ORC_GGML_Q5_K || type == ORC_GGML_IQ4_NL ||
           type == ORC_GGML_IQ4_XS;
}

/* One projection in the Q8_1 mode: the int8 matvec for the routed types, else the fp32 one. */
static int matmul_mode(int q8, int type, const uint8_t *w, int rows, int cols, const float *x,
                       const int8_t *xq, const float *xd, const float *xs, float *out)
{
    if (q8 && orc_q8_1_routed(type))
        return orc_matmul_q8_1(type, w, rows, cols, xq, xd, xs, out);
    return orc_matmul(type, w, rows, cols, x, out);
}

typedef struct {
    int dim;                     /* embeddingLength */
    float residual_scale;        /* Granite residualScale, 0 = off */
    const float *attn_norm;      /* [dim] RMSNorm weights, NULL = copy (OLMo2) */
    const float *post_attn_norm; /* [dim] or NULL */
    const uint8_t *wq, *wk, *wv; /* [q_dim][dim], [kv_dim][dim] x2 */
    const uint8_t *wqkv;         /* merged [q_dim + 2 kv_dim][dim] (used when non-NULL) */
    const uint8_t *wo;           /* [dim][q_dim] */
    int wq_type, wk_type, wv_type, wqkv_type, wo_type;
    const float *q_bias, *k_bias, *v_bias, *o_bias;
    int q8_1_input;              /* 1: the reference GPU's Q8_1-input matvecs (see above) */
} orc_block_w;

/* The attention half of one layer (TransformerBlock.forward up to the residual add, with
 * Attention.forward inside it) over an fp32 cache: x [dim] is updated in place,
 * x += residual_scale? * postnorm?(Wo . attention(Wq/k/v . rmsnorm(x))).  Layer semantics
 * (QK-norm, RoPE, window, append) are orc_forward_from_projections'.  attn_out (or NULL)
 * receives the attention output [q_dim], the output projection's input. */
int orc_attn_block(const orc_cfg *c, const orc_block_w *bw, float *kcache, float *vcache,
                   const float *qnorm_w, const float *knorm_w, const float *rope_cos,
                   const float *rope_sin, float *x, int layer, int pos, int n_threads,
                   float *attn_out)
{
    const int dim = bw->dim, qd = c->n_heads * c->head_size, kvd = c->n_kv_heads * c->head_size;
    float *xb = (float *)calloc((size_t)dim, sizeof(float));
    float *qkv = (float *)calloc((size_t)(qd + 2 * kvd), sizeof(float));
    float *xb2 = (float *)calloc((size_t)qd, sizeof(float));
    float *att = (float *)calloc((size_t)c->n_heads * (size_t)(pos + 1), sizeof(float));
    float *q = qkv, *k = qkv + qd, *v = qkv + qd + kvd;
    const int q8 = bw->q8_1_input, xn = dim > qd ? dim : qd;
    int8_t *xq = (int8_t *)calloc((size_t)xn, 1);
    float *xd = (float *)calloc((size_t)xn / 32 + 1, sizeof(float));
    float *xs = (float *)calloc((size_t)xn / 32 + 1, sizeof(float));
    int rc = 0;
    if (bw->attn_norm) {
        if (q8) orc_rmsnorm_staged(xb, x, bw->attn_norm, dim, c->norm_eps);
        else orc_rmsnorm(xb, x, bw->attn_norm, dim, c->norm_eps);
    } else {
        memcpy(xb, x, sizeof(float) * (size_t)dim);
    }
    if (q8) orc_quantize_q8_1(xb, dim, xq, xd, xs);
    if (bw->wqkv) {
        rc |= matmul_mode(q8, bw->wqkv_type, bw->wqkv, qd + 2 * kvd, dim, xb, xq, xd, xs, qkv);
    } else {
        rc |= matmul_mode(q8, bw->wq_type, bw->wq, qd, dim, xb, xq, xd, xs, q);
        rc |= matmul_mode(q8, bw->wk_type, bw->wk, kvd, dim, xb, xq, xd, xs, k);
        rc |= matmul_mode(q8, bw->wv_type, bw->wv, kvd, dim, xb, xq, xd, xs, v);
    }
    if (bw->q_bias) for (int i = 0; i < qd; i++) q[i] += bw->q_bias[i];
    if (bw->k_bias) for (int i = 0; i < kvd; i++) k[i] += bw->k_bias[i];
    if (bw->v_bias) for (int i = 0; i < kvd; i++) v[i] += bw->v_bias[i];
    orc_forward_from_projections(c, kcache, vcache, qnorm_w, knorm_w, rope_cos, rope_sin, q, k, v,
                                 layer, pos, xb2, att, 0, n_threads);
    if (attn_out) memcpy(attn_out, xb2, sizeof(float) * (size_t)qd);
    memset(xb, 0, sizeof(float) * (size_t)dim);
    if (q8) orc_quantize_q8_1(xb2, qd, xq, xd, xs);   /* quantizeXb2: the attention output */
    rc |= matmul_mode(q8, bw->wo_type, bw->wo, dim, qd, xb2, xq, xd, xs, xb);
    if (bw->o_bias) for (int i = 0; i < dim; i++) xb[i] += bw->o_bias[i];
    if (bw->post_attn_norm) orc_rmsnorm(xb, xb, bw->post_attn_norm, dim, c->norm_eps);
    if (bw->residual_scale > 0.0f)
        for (int i = 0; i < dim; i++) xb[i] *= bw->residual_scale;
    for (int i = 0; i < dim; i++) x[i] += xb[i];
    free(xb);
    free(qkv);
    free(xb2);
    free(att);
    free(xq);
    free(xd);
    free(xs);
    return rc;
}
