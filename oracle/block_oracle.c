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
 *   F32 (0), F16 (1), Q4_0 (2), Q8_0 (8), Q4_K (12), Q6_K (14), BF16 (30)  (GGMLType ids).
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

#include "orc.h"

#define ORC_GGML_F32 0
#define ORC_GGML_F16 1
#define ORC_GGML_Q4_0 2
#define ORC_GGML_Q8_0 8
#define ORC_GGML_Q4_K 12
#define ORC_GGML_Q6_K 14
#define ORC_GGML_BF16 30

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
    case ORC_GGML_Q8_0: *bytes = 34; return 32;
    case ORC_GGML_Q4_K: *bytes = 144; return 256;
    case ORC_GGML_Q6_K: *bytes = 210; return 256;
    default: *bytes = 0; return 0;
    }
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
} orc_block_w;

/* The attention half of one layer (TransformerBlock.forward up to the residual add, with
 * Attention.forward inside it) over an fp32 cache: x [dim] is updated in place,
 * x += residual_scale? * postnorm?(Wo . attention(Wq/k/v . rmsnorm(x))).  Layer semantics
 * (QK-norm, RoPE, window, append) are orc_forward_from_projections'. */
int orc_attn_block(const orc_cfg *c, const orc_block_w *bw, float *kcache, float *vcache,
                   const float *qnorm_w, const float *knorm_w, const float *rope_cos,
                   const float *rope_sin, float *x, int layer, int pos, int n_threads)
{
    const int dim = bw->dim, qd = c->n_heads * c->head_size, kvd = c->n_kv_heads * c->head_size;
    float *xb = (float *)calloc((size_t)dim, sizeof(float));
    float *qkv = (float *)calloc((size_t)(qd + 2 * kvd), sizeof(float));
    float *xb2 = (float *)calloc((size_t)qd, sizeof(float));
    float *att = (float *)calloc((size_t)c->n_heads * (size_t)(pos + 1), sizeof(float));
    float *q = qkv, *k = qkv + qd, *v = qkv + qd + kvd;
    int rc = 0;
    if (bw->attn_norm)
        orc_rmsnorm(xb, x, bw->attn_norm, dim, c->norm_eps);
    else
        memcpy(xb, x, sizeof(float) * (size_t)dim);
    if (bw->wqkv) {
        rc |= orc_matmul(bw->wqkv_type, bw->wqkv, qd + 2 * kvd, dim, xb, qkv);
    } else {
        rc |= orc_matmul(bw->wq_type, bw->wq, qd, dim, xb, q);
        rc |= orc_matmul(bw->wk_type, bw->wk, kvd, dim, xb, k);
        rc |= orc_matmul(bw->wv_type, bw->wv, kvd, dim, xb, v);
    }
    if (bw->q_bias) for (int i = 0; i < qd; i++) q[i] += bw->q_bias[i];
    if (bw->k_bias) for (int i = 0; i < kvd; i++) k[i] += bw->k_bias[i];
    if (bw->v_bias) for (int i = 0; i < kvd; i++) v[i] += bw->v_bias[i];
    orc_forward_from_projections(c, kcache, vcache, qnorm_w, knorm_w, rope_cos, rope_sin, q, k, v,
                                 layer, pos, xb2, att, 0, n_threads);
    memset(xb, 0, sizeof(float) * (size_t)dim);
    rc |= orc_matmul(bw->wo_type, bw->wo, dim, qd, xb2, xb);
    if (bw->o_bias) for (int i = 0; i < dim; i++) xb[i] += bw->o_bias[i];
    if (bw->post_attn_norm) orc_rmsnorm(xb, xb, bw->post_attn_norm, dim, c->norm_eps);
    if (bw->residual_scale > 0.0f)
        for (int i = 0; i < dim; i++) xb[i] *= bw->residual_scale;
    for (int i = 0; i < dim; i++) x[i] += xb[i];
    free(xb);
    free(qkv);
    free(xb2);
    free(att);
    return rc;
}
