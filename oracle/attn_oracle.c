/*
 * attn_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of LLMPlayer's Java decode attention, used as the parity checker for the
 * HIP path (tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg).  Nothing in
 * the product (llmplayer_amd/, include/) may link, load or call this file.
 *
 * It follows the Java float semantics of the reference:
 *   - Java never contracts a*b+c into an FMA; only Vector.fma is fused
 *     (SimdVectorOps.java:24, :41).  Build with -ffp-contract=off; fmaf() is used exactly
 *     where the reference calls Vector.fma.
 *   - Math.exp / Math.sqrt / Math.cos / Math.sin / Math.pow run in double and are cast to
 *     float (ScalarOps.java:45, SimdVectorOps.java:84, Attention.java:140, :390,
 *     RoPE.java:83, :102-103).  libm double functions are used the same way.
 *   - SimdVectorOps.dot accumulates SPECIES_PREFERRED lanes with FMA and then calls
 *     reduceLanes(ADD) (SimdVectorOps.java:17-31).  The lane count (8 on AVX2, 16 on
 *     AVX-512) and the reduction order are JVM-defined.  This restatement fixes ONE
 *     documented order: 8 lanes, lane l accumulates elements i = l (mod 8) in increasing i
 *     with fmaf, then the lanes are summed left to right (((l0+l1)+l2)+...+l7), which is the
 *     Vector API's scalar fallback order; the scalar tail (len % 8) uses a separate multiply
 *     and add.  The HIP kernels reproduce this order wherever a bit-exact result is required
 *     (the QK-norm sum of squares that feeds the appended K row).
 *
 * Parity pinning: the Java reference cannot run here (no JVM; the gguf package is missing
 * from the published tree), and the reference holds no tests or golden vectors.  Each
 * function below is pinned in tests/test_oracle.py by closed forms and invariants
 * (identity rotation at p=0, pair-norm preservation, NORMAL/NEOX pairing, out=V0 at n=1,
 * uniform scores give the mean of V, GQA head mapping, fp64 brute force on tiny shapes,
 * window boundaries, QK-norm scale invariance, flash == two-pass).  The last-ulp behaviour of
 * HotSpot's Math intrinsics and of reduceLanes is NOT pinned (parity unpinned at ulp level).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_LANES 8

/* SimdVectorOps.dot (SimdVectorOps.java:17-31), 8-lane restatement described above. */
float orc_dot(const float *a, const float *b, int len)
{
    float lane[ORC_LANES] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    int upper = len - (len % ORC_LANES);
    for (; i < upper; i += ORC_LANES)
        for (int l = 0; l < ORC_LANES; l++)
            lane[l] = fmaf(a[i + l], b[i + l], lane[l]);
    float sum = lane[0];
    for (int l = 1; l < ORC_LANES; l++)
        sum = sum + lane[l];
    for (; i < len; i++) {
        float p = a[i] * b[i];
        sum = sum + p;
    }
    return sum;
}

/* SimdVectorOps.saxpy (SimdVectorOps.java:34-47): y = fma(x, a, y) on full lanes, then a
 * separate multiply and add on the tail. */
void orc_saxpy(float a, const float *x, float *y, int len)
{
    int i = 0;
    int upper = len - (len % ORC_LANES);
    for (; i < upper; i++)
        y[i] = fmaf(x[i], a, y[i]);
    for (; i < len; i++) {
        float p = a * x[i];
        y[i] = y[i] + p;
    }
}

/* SimdVectorOps.softmax (SimdVectorOps.java:77-98) == ScalarOps.softmax (ScalarOps.java:38-52):
 * scalar max, e = (float)exp(x - max) with a sequential fp32 sum, then x *= 1/sum. */
void orc_softmax(float *x, int n)
{
    float maxv = -INFINITY;
    for (int i = 0; i < n; i++)
        if (x[i] > maxv) maxv = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        float d = x[i] - maxv;
        x[i] = (float)exp((double)d);
        sum = sum + x[i];
    }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++)
        x[i] = x[i] * inv;
}

/* Qwen3MoEInferenceEngine.softmaxWithSink (Qwen3MoEInferenceEngine.java:562-575): the sink
 * logit joins the max and the denominator, and gets no weight of its own. */
void orc_softmax_with_sink(float *x, int n, float sink)
{
    float maxv = sink;
    for (int i = 0; i < n; i++)
        if (x[i] > maxv) maxv = x[i];
    float sum = (float)exp((double)(sink - maxv));
    for (int i = 0; i < n; i++) {
        float d = x[i] - maxv;
        x[i] = (float)exp((double)d);
        sum = sum + x[i];
    }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++)
        x[i] = x[i] * inv;
}

/* Qwen3.5 attention output gate (Qwen35InferenceEngine.java:580-583, sigmoid at :628-630):
 * out[i] *= 1/(1 + (float)exp(-gate[i])). */
void orc_sigmoid_gate(float *out, const float *gate, int n)
{
    for (int i = 0; i < n; i++) {
        float e = (float)exp((double)(-gate[i]));
        float sg = 1.0f / (1.0f + e);
        out[i] = out[i] * sg;
    }
}

/* Attention.applyPerHeadNorm (Attention.java:384-394) with SimdVectorOps.scaleWeighted
 * (SimdVectorOps.java:150-162): ss = dot(x,x); r = 1/(float)sqrt(ss/D + eps); x = (x*r)*w. */
void orc_per_head_norm(float *vec, const float *w, int n_heads, int head_size, float eps)
{
    for (int h = 0; h < n_heads; h++) {
        float *x = vec + (size_t)h * head_size;
        float ss = orc_dot(x, x, head_size);
        float t = ss / (float)head_size;
        t = t + eps;
        float r = 1.0f / (float)sqrt((double)t);
        for (int i = 0; i < head_size; i++) {
            float xs = x[i] * r;
            x[i] = xs * w[i];
        }
    }
}

/* RoPE tables (RoPE.java:45-106, non-YaRN branch):
 *   baseFreq = (float)(1.0 / pow(theta, 2.0*i/R)); baseFreq /= freqFactors[i] (if given);
 *   freq = baseFreq * freqScale  (freqScale = 1/linearFreqScale when linearFreqScale > 1);
 *   angle = (float)pos * freq;  cos = (float)cos(angle);  sin = (float)sin(angle).
 * Tables are [max_seq][R/2]. */
void orc_rope_tables(int rope_dim, int max_seq, float theta, float linear_freq_scale,
                     const float *freq_factors, int n_freq_factors, float *cos_t, float *sin_t)
{
    int half = rope_dim / 2;
    float freq_scale = 1.0f;
    if (linear_freq_scale > 1.0f)
        freq_scale = 1.0f / linear_freq_scale;
    float *freq = (float *)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
    for (int i = 0; i < half; i++) {
        double ex = 2.0 * (double)i / (double)rope_dim;
        float base = (float)(1.0 / pow((double)theta, ex));
        if (freq_factors && i < n_freq_factors)
            base = base / freq_factors[i];
        freq[i] = base * freq_scale;
    }
    for (int pos = 0; pos < max_seq; pos++) {
        for (int i = 0; i < half; i++) {
            float angle = (float)pos * freq[i];
            cos_t[(size_t)pos * half + i] = (float)cos((double)angle);
            sin_t[(size_t)pos * half + i] = (float)sin((double)angle);
        }
    }
    free(freq);
}

/* RoPE tables, YaRN branch (RoPE.java:45-106 with YarnParams, :107-117; used by the MoE and
 * MLA engines, Qwen3MoEInferenceEngine.java:60-66, DeepSeek2InferenceEngine.java:48), in Java's
 * float/double steps:
 *   freqScale = 1/s;
 *   corrDim(beta) = R * (float)log(L / (beta*2*pi)) / (2 * (float)log(theta))  (RoPE.yarnCorrDim);
 *   low = max(0, (float)floor(corrDim(betaFast))), high = min(R/2 - 1, (float)ceil(corrDim(betaSlow)));
 *   attnFactor = logMul > 0 ? 0.1*logMul*(float)log(s) + 1 : 1;
 *   mscale = attnFactor * (1 + 0.1*(float)log(1/freqScale));
 *   ramp(i) = 1 - min(1, max(0, (i - low) / max(0.001, high - low)))  (RoPE.yarnRamp);
 *   freq = (freqScale*base) * (1 - ramp) + base * ramp, base as in the plain branch;
 *   angle = (float)pos * freq; cos/sin as in the plain branch.
 * With s <= 1 the plain branch runs (no linear scale: the MoE engines pass none).  *mscale gets
 * the attention-magnitude factor (1 without YaRN); the engines scale scores by
 * mscale^2/sqrt(headSize) (Qwen3MoEInferenceEngine.java:277-279). */
void orc_rope_tables_yarn(int rope_dim, int max_seq, float theta, const float *freq_factors,
                          int n_freq_factors, float scaling_factor, int orig_ctx, float beta_fast,
                          float beta_slow, float yarn_log_mul, float *cos_t, float *sin_t,
                          float *mscale)
{
    if (!(scaling_factor > 1.0f)) {
        orc_rope_tables(rope_dim, max_seq, theta, 1.0f, freq_factors, n_freq_factors, cos_t, sin_t);
        if (mscale)
            *mscale = 1.0f;
        return;
    }
    int half = rope_dim / 2;
    float freq_scale = 1.0f / scaling_factor;
    const double pi = 3.141592653589793;   /* Math.PI */
    float corr_low = (float)rope_dim * (float)log((double)orig_ctx / ((double)beta_fast * 2.0 * pi)) /
                     (2.0f * (float)log((double)theta));
    float corr_high = (float)rope_dim * (float)log((double)orig_ctx / ((double)beta_slow * 2.0 * pi)) /
                      (2.0f * (float)log((double)theta));
    float fl = (float)floor((double)corr_low);
    corr_low = fl > 0.0f ? fl : 0.0f;
    float ce = (float)ceil((double)corr_high);
    float lim = (float)rope_dim / 2.0f - 1.0f;
    corr_high = lim < ce ? lim : ce;
    float attn_factor = 1.0f;
    if (yarn_log_mul > 0.0f)
        attn_factor = 0.1f * yarn_log_mul * (float)log((double)scaling_factor) + 1.0f;
    float ms = attn_factor * (1.0f + 0.1f * (float)log((double)(1.0f / freq_scale)));
    if (mscale)
        *mscale = ms;
    float *freq = (float *)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
    for (int i = 0; i < half; i++) {
        double ex = 2.0 * (double)i / (double)rope_dim;
        float base = (float)(1.0 / pow((double)theta, ex));
        if (freq_factors && i < n_freq_factors)
            base = base / freq_factors[i];
        float span = corr_high - corr_low;
        float y = ((float)i - corr_low) / (span > 0.001f ? span : 0.001f);
        float cl = y < 0.0f ? 0.0f : y;
        cl = cl < 1.0f ? cl : 1.0f;
        float ramp = 1.0f - cl;
        float interp = freq_scale * base;
        float a = interp * (1.0f - ramp);
        float b = base * ramp;
        freq[i] = a + b;
    }
    for (int pos = 0; pos < max_seq; pos++) {
        for (int i = 0; i < half; i++) {
            float angle = (float)pos * freq[i];
            cos_t[(size_t)pos * half + i] = (float)cos((double)angle);
            sin_t[(size_t)pos * half + i] = (float)sin((double)angle);
        }
    }
    free(freq);
}

/* RoPE.applyAllHeads (RoPE.java:176-193): NORMAL pairs (2i, 2i+1) via RoPE.apply
 * (RoPE.java:145-170); NEOX pairs (i, i+R/2) via ropeNeox (SimdVectorOps.java:165-186).
 * Both compute x0' = x0*c - x1*s, x1' = x0*s + x1*c with separately rounded products. */
void orc_rope_apply_all(float *vec, int n_heads, int head_size, int rope_dim, int rope_type,
                        const float *cos_t, const float *sin_t, int pos)
{
    int half = rope_dim / 2;
    const float *c = cos_t + (size_t)pos * half;
    const float *s = sin_t + (size_t)pos * half;
    for (int h = 0; h < n_heads; h++) {
        float *x = vec + (size_t)h * head_size;
        for (int i = 0; i < half; i++) {
            int i0 = (rope_type == 0) ? 2 * i : i;
            int i1 = (rope_type == 0) ? 2 * i + 1 : half + i;
            float v0 = x[i0], v1 = x[i1];
            float a = v0 * c[i], b = v1 * s[i];
            float e = v0 * s[i], f = v1 * c[i];
            x[i0] = a - b;
            x[i1] = e + f;
        }
    }
}

/* Architecture ids for Attention.isGlobalLayer (Attention.java:250-276). */
enum { ORC_ARCH_OTHER = 0, ORC_ARCH_GEMMA2 = 1, ORC_ARCH_GEMMA3 = 2, ORC_ARCH_GPT_OSS = 3,
       ORC_ARCH_COHERE2 = 4, ORC_ARCH_GPT_OSS_MOE = 5 };

int orc_is_global_layer(int arch, int layer)
{
    switch (arch) {
    case ORC_ARCH_GEMMA2: return layer % 2 == 1;
    case ORC_ARCH_GEMMA3: return layer % 6 == 5;
    case ORC_ARCH_GPT_OSS: return layer % 2 == 0;
    /* GPT-OSS with experts on the Qwen3MoE engine: even layers windowed
     * (Qwen3MoEInferenceEngine.java:280-286; engine choice LLMEngine.java:144). */
    case ORC_ARCH_GPT_OSS_MOE: return layer % 2 == 1;
    case ORC_ARCH_COHERE2: return layer % 4 == 3;
    default: return 1;
    }
}

/* Layer-independent attention hyper-parameters (the subset of ModelConfig read by
 * Attention.java:284-367). */
#include "orc.h"

/* KVCache.storeK / storeV (KVCache.java:164-179), FLOAT32 mode: cache[layer][pos*kvDim + j]. */
void orc_kv_store(float *cache_layer, int pos, const float *x, int kv_dim)
{
    memcpy(cache_layer + (size_t)pos * kv_dim, x, sizeof(float) * (size_t)kv_dim);
}

/* ---- KVCache Q8_0 mode (KVCache.java:11-28, 218-282) -----------------------------------
 * Blocks of 32 values with one fp32 scale each.  The JVM picks one of two contracts at class
 * load (KVCache.loadQ8Ops, KVCache.java:54-62): SimdQ8KvOps when the Vector API is present
 * and its preferred float species has exactly 8 lanes (AVX2 hosts, SimdQ8KvOps.java:27-33),
 * otherwise the scalar one (quantizeBlocksScalar / dotQ8BlockScalar / saxpyQ8BlockScalar).
 * ORC_Q8_SCALAR restates the scalar contract (round half up); ORC_Q8_SIMD8 restates the
 * 8-lane one (truncating quantize, FMA lanes in dot and saxpy, SimdQ8KvOps.java:37-117). */
#define ORC_Q8_BLOCK 32
#define ORC_Q8_SCALAR 1
#define ORC_Q8_SIMD8 2

/* Math.round(float): the closest int, ties toward positive infinity.  floor(y) and y - floor(y)
 * are exact for |y| < 2^22, which covers every quantized value (|y| <= 127.x). */
int orc_round_half_up(float y)
{
    float r = floorf(y);
    float frac = y - r;
    if (frac >= 0.5f) r = r + 1.0f;
    return (int)r;
}

/* quantizeBlocksScalar (KVCache.java:218-243). */
void orc_q8_quantize(const float *src, int n, int8_t *dst, float *scales)
{
    int blocks = n / ORC_Q8_BLOCK;
    for (int b = 0; b < blocks; b++) {
        const float *x = src + (size_t)b * ORC_Q8_BLOCK;
        float max_abs = 0.0f;
        for (int i = 0; i < ORC_Q8_BLOCK; i++) {
            float a = x[i] >= 0 ? x[i] : -x[i];
            if (a > max_abs) max_abs = a;
        }
        float scale = max_abs / 127.0f;
        float inv = scale != 0.0f ? 1.0f / scale : 0.0f;
        scales[b] = scale;
        for (int i = 0; i < ORC_Q8_BLOCK; i++) {
            float y = x[i] * inv;
            int q = orc_round_half_up(y);
            if (q > 127) q = 127;
            else if (q < -128) q = -128;
            dst[(size_t)b * ORC_Q8_BLOCK + i] = (int8_t)q;
        }
    }
}

/* dotQ8BlockScalar (KVCache.java:252-267): per block a sequential unfused sum, then * scale. */
float orc_q8_dot(const float *q, const int8_t *kq, const float *ks, int n)
{
    int blocks = n / ORC_Q8_BLOCK;
    float total = 0.0f;
    for (int b = 0; b < blocks; b++) {
        float acc = 0.0f;
        for (int i = 0; i < ORC_Q8_BLOCK; i++) {
            float p = q[b * ORC_Q8_BLOCK + i] * (float)kq[b * ORC_Q8_BLOCK + i];
            acc = acc + p;
        }
        float t = acc * ks[b];
        total = total + t;
    }
    return total;
}

/* saxpyQ8BlockScalar (KVCache.java:269-282): out += (weight*scale) * quant, unfused. */
void orc_q8_saxpy(float weight, const int8_t *vq, const float *vs, float *out, int n)
{
    int blocks = n / ORC_Q8_BLOCK;
    for (int b = 0; b < blocks; b++) {
        float w = weight * vs[b];
        for (int i = 0; i < ORC_Q8_BLOCK; i++) {
            float p = w * (float)vq[b * ORC_Q8_BLOCK + i];
            out[b * ORC_Q8_BLOCK + i] = out[b * ORC_Q8_BLOCK + i] + p;
        }
    }
}

/* SimdQ8KvOps.quantize (SimdQ8KvOps.java:86-117): block max of |x| (order-free), the same
 * scale and inverse as the scalar path, then F2I, i.e. truncation toward zero, and a clamp to
 * [-128, 127]. */
void orc_q8_quantize_simd8(const float *src, int n, int8_t *dst, float *scales)
{
    int blocks = n / ORC_Q8_BLOCK;
    for (int b = 0; b < blocks; b++) {
        const float *x = src + (size_t)b * ORC_Q8_BLOCK;
        float max_abs = 0.0f;
        for (int i = 0; i < ORC_Q8_BLOCK; i++) {
            float a = fabsf(x[i]);
            if (a > max_abs) max_abs = a;
        }
        float scale = max_abs / 127.0f;
        float inv = scale != 0.0f ? 1.0f / scale : 0.0f;
        scales[b] = scale;
        for (int i = 0; i < ORC_Q8_BLOCK; i++) {
            float y = x[i] * inv;
            int q = (int)y;                       /* |y| <= 127.x: in range, toward zero */
            if (q > 127) q = 127;
            else if (q < -128) q = -128;
            dst[(size_t)b * ORC_Q8_BLOCK + i] = (int8_t)q;
        }
    }
}

/* SimdQ8KvOps.dot (SimdQ8KvOps.java:37-63): per block, 8 lanes each FMA-accumulate the
 * elements i = l (mod 8) in chunk order; the lanes are summed (left to right, the order the
 * restatement fixes for reduceLanes(ADD)), multiplied by the scale and added to the total. */
float orc_q8_dot_simd8(const float *q, const int8_t *kq, const float *ks, int n)
{
    int blocks = n / ORC_Q8_BLOCK;
    float total = 0.0f;
    for (int b = 0; b < blocks; b++) {
        float lane[ORC_LANES] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int c = 0; c < ORC_Q8_BLOCK; c += ORC_LANES)
            for (int l = 0; l < ORC_LANES; l++) {
                int i = b * ORC_Q8_BLOCK + c + l;
                lane[l] = fmaf((float)kq[i], q[i], lane[l]);
            }
        float sum = lane[0];
        for (int l = 1; l < ORC_LANES; l++) sum = sum + lane[l];
        float t = sum * ks[b];
        total = total + t;
    }
    return total;
}

/* SimdQ8KvOps.saxpy (SimdQ8KvOps.java:66-84): out = fma(quant, weight*scale, out). */
void orc_q8_saxpy_simd8(float weight, const int8_t *vq, const float *vs, float *out, int n)
{
    int blocks = n / ORC_Q8_BLOCK;
    for (int b = 0; b < blocks; b++) {
        float w = weight * vs[b];
        for (int i = 0; i < ORC_Q8_BLOCK; i++) {
            int j = b * ORC_Q8_BLOCK + i;
            out[j] = fmaf((float)vq[j], w, out[j]);
        }
    }
}

/* First attended position (Attention.java:330-335). */
int orc_start_pos(const orc_cfg *c, int layer, int pos)
{
    if (c->sliding_window > 0 && !orc_is_global_layer(c->arch, layer)) {
        int s = pos - c->sliding_window + 1;
        return s > 0 ? s : 0;
    }
    return 0;
}

/* A layer's cache in either KVCache mode: FLOAT32 rows [max_seq][kvDim], or Q8_0 quants
 * [max_seq][kvDim] with scales [max_seq][kvDim/32] (KVCache.java:86-94). */
typedef struct {
    float *kf, *vf;          /* FLOAT32 mode */
    int8_t *kq, *vq;         /* Q8_0 mode    */
    float *ks, *vs;
} orc_layer_cache;

static float cache_dot(const orc_layer_cache *kv, int q8, int t, int kv_dim, int off,
                       const float *q, int D)
{
    if (!q8) return orc_dot(q, kv->kf + (size_t)t * kv_dim + off, D);
    size_t base = (size_t)t * kv_dim + off;
    if (q8 == ORC_Q8_SIMD8)
        return orc_q8_dot_simd8(q, kv->kq + base, kv->ks + base / ORC_Q8_BLOCK, D);
    return orc_q8_dot(q, kv->kq + base, kv->ks + base / ORC_Q8_BLOCK, D);
}

static void cache_saxpy(const orc_layer_cache *kv, int q8, int t, int kv_dim, int off, float a,
                        float *out, int D)
{
    if (!q8) {
        orc_saxpy(a, kv->vf + (size_t)t * kv_dim + off, out, D);
        return;
    }
    size_t base = (size_t)t * kv_dim + off;
    if (q8 == ORC_Q8_SIMD8)
        orc_q8_saxpy_simd8(a, kv->vq + base, kv->vs + base / ORC_Q8_BLOCK, out, D);
    else
        orc_q8_saxpy(a, kv->vq + base, kv->vs + base / ORC_Q8_BLOCK, out, D);
}

/* Attention.forwardFromProjections (Attention.java:284-367) over a cache in either mode
 * (KVCache.storeK/storeV/dotK/saxpyV, KVCache.java:164-210). */
static void forward_impl(const orc_cfg *c, const orc_layer_cache *kv, int q8,
                         const float *qnorm_w, const float *knorm_w, const float *rope_cos,
                         const float *rope_sin, float *q, float *k, const float *v, int layer,
                         int pos, float *out, float *att_scratch, int use_flash, int n_threads)
{
    const int Hq = c->n_heads, Hkv = c->n_kv_heads, D = c->head_size;
    const int kv_dim = Hkv * D;
    const int kv_mul = Hq / Hkv;

    if (qnorm_w && knorm_w) {
        orc_per_head_norm(q, qnorm_w, Hq, D, c->norm_eps);
        orc_per_head_norm(k, knorm_w, Hkv, D, c->norm_eps);
    }
    int irope_skip = c->no_rope_interval > 0 &&
                     (layer % c->no_rope_interval) == (c->no_rope_interval - 1);
    int cohere_skip = c->nope_on_global && orc_is_global_layer(c->arch, layer);
    if (!irope_skip && !cohere_skip && rope_cos && rope_sin) {
        orc_rope_apply_all(q, Hq, D, c->rope_dim, c->rope_type, rope_cos, rope_sin, pos);
        orc_rope_apply_all(k, Hkv, D, c->rope_dim, c->rope_type, rope_cos, rope_sin, pos);
    }
    if (!q8) {
        orc_kv_store(kv->kf, pos, k, kv_dim);
        orc_kv_store(kv->vf, pos, v, kv_dim);
    } else {
        size_t base = (size_t)pos * kv_dim;
        void (*quant)(const float *, int, int8_t *, float *) =
            q8 == ORC_Q8_SIMD8 ? orc_q8_quantize_simd8 : orc_q8_quantize;
        quant(k, kv_dim, kv->kq + base, kv->ks + base / ORC_Q8_BLOCK);
        quant(v, kv_dim, kv->vq + base, kv->vs + base / ORC_Q8_BLOCK);
    }

    float scale = c->attention_scale > 0.0f ? c->attention_scale
                                            : (float)(1.0 / sqrt((double)D));
    int start = orc_start_pos(c, layer, pos);
    int seq_len = pos + 1 - start;
    float softcap = c->softcap;
    memset(out, 0, sizeof(float) * (size_t)Hq * D);

    int nt = n_threads > 0 ? n_threads : 1;
    (void)nt;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
    for (int h = 0; h < Hq; h++) {
        int kv_off = (h / kv_mul) * D;
        const float *qh = q + (size_t)h * D;
        float *oh = out + (size_t)h * D;
        if (use_flash && !c->sinks) {
            float max_score = -INFINITY;
            float sum_exp = 0.0f;
            for (int t = start; t <= pos; t++) {
                float score = cache_dot(kv, q8, t, kv_dim, kv_off, qh, D);
                float s = score * scale;
                if (softcap > 0.0f) {
                    float r = s / softcap;
                    s = softcap * (float)tanh((double)r);
                }
                float new_max = s > max_score ? s : max_score;
                float scale_old = (max_score == -INFINITY)
                                      ? 0.0f
                                      : (float)exp((double)(max_score - new_max));
                float scale_new = (float)exp((double)(s - new_max));
                if (scale_old != 1.0f)
                    for (int i = 0; i < D; i++) oh[i] = oh[i] * scale_old;
                cache_saxpy(kv, q8, t, kv_dim, kv_off, scale_new, oh, D);
                float m = sum_exp * scale_old;
                sum_exp = m + scale_new;
                max_score = new_max;
            }
            if (sum_exp > 0.0f) {
                float inv = 1.0f / sum_exp;
                for (int i = 0; i < D; i++) oh[i] = oh[i] * inv;
            }
        } else {
            float *att = att_scratch + (size_t)h * seq_len;
            for (int t = start; t <= pos; t++) {
                float score = cache_dot(kv, q8, t, kv_dim, kv_off, qh, D);
                float s = score * scale;
                if (softcap > 0.0f) {
                    float r = s / softcap;
                    s = softcap * (float)tanh((double)r);
                }
                att[t - start] = s;
            }
            if (c->sinks)
                orc_softmax_with_sink(att, seq_len, c->sinks[h]);
            else
                orc_softmax(att, seq_len);
            for (int t = start; t <= pos; t++)
                cache_saxpy(kv, q8, t, kv_dim, kv_off, att[t - start], oh, D);
        }
    }
}

/* Attention.forwardFromProjections (Attention.java:284-367), optional bias omitted (absent
 * from every configuration this build covers).  q and k are modified in place exactly as
 * state.q / state.k are; the K/V rows are appended at `pos`; out = xb2[Hq*D].
 * use_flash != 0 selects the online-softmax loop of Attention.forward (Attention.java:161-207).
 * kcache/vcache are one layer's FLOAT32 [max_seq][kvDim] arrays.  rope_cos/rope_sin are the
 * table the layer selects (global or local, Attention.java:317); NULL skips RoPE (NoPE). */
void orc_forward_from_projections(const orc_cfg *c, float *kcache, float *vcache,
                                  const float *qnorm_w, const float *knorm_w,
                                  const float *rope_cos, const float *rope_sin,
                                  float *q, float *k, const float *v,
                                  int layer, int pos, float *out, float *att_scratch,
                                  int use_flash, int n_threads)
{
    orc_layer_cache kv = {kcache, vcache, NULL, NULL, NULL, NULL};
    forward_impl(c, &kv, 0, qnorm_w, knorm_w, rope_cos, rope_sin, q, k, v, layer, pos, out,
                 att_scratch, use_flash, n_threads);
}

/* The same layer-call over a Q8_0 cache (KVCache Mode.Q8_0): quants [max_seq][kvDim],
 * scales [max_seq][kvDim/32] for K and V. */
void orc_forward_from_projections_q8(const orc_cfg *c, int8_t *kq, float *ks, int8_t *vq,
                                     float *vs, const float *qnorm_w, const float *knorm_w,
                                     const float *rope_cos, const float *rope_sin, float *q,
                                     float *k, const float *v, int layer, int pos, float *out,
                                     float *att_scratch, int use_flash, int n_threads,
                                     int q8_mode)
{
    orc_layer_cache kv = {NULL, NULL, kq, vq, ks, vs};
    int mode = q8_mode == ORC_Q8_SIMD8 ? ORC_Q8_SIMD8 : ORC_Q8_SCALAR;
    forward_impl(c, &kv, mode, qnorm_w, knorm_w, rope_cos, rope_sin, q, k, v, layer, pos, out,
                 att_scratch, use_flash, n_threads);
}

/* The reference has no batched prefill: the prompt runs as P sequential single-token
 * forwards (LLMEngine.java:478-480, InferenceEngine.prefill at InferenceEngine.java:374-381).
 * This helper runs those P calls for one layer; q/k/v are [P][Hq*D] / [P][kvDim] inputs,
 * out is [P][Hq*D].  Inputs are copied, so q/k/v are not modified. */
void orc_prefill_sequential(const orc_cfg *c, float *kcache, float *vcache,
                            const float *qnorm_w, const float *knorm_w,
                            const float *rope_cos, const float *rope_sin,
                            const float *q, const float *k, const float *v,
                            int layer, int pos0, int n_tokens, float *out, int n_threads)
{
    const int qdim = c->n_heads * c->head_size;
    const int kv_dim = c->n_kv_heads * c->head_size;
    float *qb = (float *)malloc(sizeof(float) * (size_t)qdim);
    float *kb = (float *)malloc(sizeof(float) * (size_t)kv_dim);
    float *att = (float *)malloc(sizeof(float) * (size_t)c->n_heads * (size_t)(pos0 + n_tokens));
    for (int i = 0; i < n_tokens; i++) {
        memcpy(qb, q + (size_t)i * qdim, sizeof(float) * (size_t)qdim);
        memcpy(kb, k + (size_t)i * kv_dim, sizeof(float) * (size_t)kv_dim);
        orc_forward_from_projections(c, kcache, vcache, qnorm_w, knorm_w, rope_cos, rope_sin,
                                     qb, kb, v + (size_t)i * kv_dim, layer, pos0 + i,
                                     out + (size_t)i * qdim, att, 0, n_threads);
    }
    free(qb);
    free(kb);
    free(att);
}

/* The same P sequential single-token forwards over a Q8_0 cache (KVCache Mode.Q8_0): each
 * token's K/V rows are quantised as they are appended (KVCache.storeK/storeV) and later
 * tokens attend to the quantised rows.  q8_mode selects the JVM's contract. */
void orc_prefill_sequential_q8(const orc_cfg *c, int8_t *kq, float *ks, int8_t *vq, float *vs,
                               const float *qnorm_w, const float *knorm_w,
                               const float *rope_cos, const float *rope_sin,
                               const float *q, const float *k, const float *v,
                               int layer, int pos0, int n_tokens, float *out, int n_threads,
                               int q8_mode)
{
    const int qdim = c->n_heads * c->head_size;
    const int kv_dim = c->n_kv_heads * c->head_size;
    float *qb = (float *)malloc(sizeof(float) * (size_t)qdim);
    float *kb = (float *)malloc(sizeof(float) * (size_t)kv_dim);
    float *att = (float *)malloc(sizeof(float) * (size_t)c->n_heads * (size_t)(pos0 + n_tokens));
    for (int i = 0; i < n_tokens; i++) {
        memcpy(qb, q + (size_t)i * qdim, sizeof(float) * (size_t)qdim);
        memcpy(kb, k + (size_t)i * kv_dim, sizeof(float) * (size_t)kv_dim);
        orc_forward_from_projections_q8(c, kq, ks, vq, vs, qnorm_w, knorm_w, rope_cos, rope_sin,
                                        qb, kb, v + (size_t)i * kv_dim, layer, pos0 + i,
                                        out + (size_t)i * qdim, att, 0, n_threads, q8_mode);
    }
    free(qb);
    free(kb);
    free(att);
}

/* ---- Gemma 4 (Gemma4InferenceEngine.java:295-420) -----------------------------------------
 * RMSNorm.apply with offsets (RMSNorm.java:24-35): a sequential, unfused sum of squares,
 * r = 1/(float)sqrt(ss/size + eps), x = (x*r)*w.  w == NULL is RMSNorm.applyNoScale
 * (RMSNorm.java:40-50), x = x*r, the weightless V-norm of Gemma 4. */
void orc_rms_norm_seq(float *x, const float *w, int size, float eps)
{
    float ss = 0.0f;
    for (int i = 0; i < size; i++) {
        float v = x[i];
        ss += v * v;
    }
    ss = 1.0f / (float)sqrt((double)(ss / (float)size + eps));
    for (int i = 0; i < size; i++) x[i] = w ? x[i] * ss * w[i] : x[i] * ss;
}

/* The attention half of Gemma4InferenceEngine.forwardLayer (Gemma4InferenceEngine.java:
 * 300-420) for one layer: per-head QK-norm (RMSNorm.apply order) and RoPE on q; when the
 * layer has its own KV (k, v non-NULL): K-norm, weightless V-norm, RoPE on k, store at `pos`;
 * otherwise (shared-KV layer) the cache is the source layer's and is only read.  Scores are
 * sequential float dots with scale 1.0, softmax as written inline there (max, (float)exp,
 * sequential sum, multiply by 1/sum), out[i] = sum over t of att*v in increasing t.
 * c->head_size is the layer type's head size; window applies when is_swa.  q, k, v are
 * modified in place as qBuf/kBuf/vBuf are. */
void orc_forward_gemma4(const orc_cfg *c, float *kcache, float *vcache, const float *qnorm_w,
                        const float *knorm_w, const float *rope_cos, const float *rope_sin,
                        float *q, float *k, float *v, int is_swa, int pos, float *out,
                        float *att_scratch, int n_threads)
{
    const int Hq = c->n_heads, Hkv = c->n_kv_heads, D = c->head_size;
    const int kv_dim = Hkv * D;
    const int kv_mul = Hq / Hkv;
    if (qnorm_w)
        for (int h = 0; h < Hq; h++) orc_rms_norm_seq(q + (size_t)h * D, qnorm_w, D, c->norm_eps);
    if (rope_cos && rope_sin)
        orc_rope_apply_all(q, Hq, D, c->rope_dim, c->rope_type, rope_cos, rope_sin, pos);
    if (k && v) {
        if (knorm_w)
            for (int h = 0; h < Hkv; h++) orc_rms_norm_seq(k + (size_t)h * D, knorm_w, D, c->norm_eps);
        for (int h = 0; h < Hkv; h++) orc_rms_norm_seq(v + (size_t)h * D, NULL, D, c->norm_eps);
        if (rope_cos && rope_sin)
            orc_rope_apply_all(k, Hkv, D, c->rope_dim, c->rope_type, rope_cos, rope_sin, pos);
        orc_kv_store(kcache, pos, k, kv_dim);
        orc_kv_store(vcache, pos, v, kv_dim);
    }
    const int start = (is_swa && c->sliding_window > 0 && pos - c->sliding_window + 1 > 0)
                          ? pos - c->sliding_window + 1 : 0;
    const int n = pos + 1 - start;
    int nt = n_threads > 0 ? n_threads : 1;
    (void)nt;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
    for (int h = 0; h < Hq; h++) {
        const int kvh = h / kv_mul;
        const float *qh = q + (size_t)h * D;
        float *att = att_scratch + (size_t)h * n;
        for (int t = start; t <= pos; t++) {
            const float *kt = kcache + (size_t)t * kv_dim + (size_t)kvh * D;
            float score = 0.0f;
            for (int i = 0; i < D; i++) score += qh[i] * kt[i];
            att[t - start] = score * 1.0f;
        }
        float max_val = -INFINITY;
        for (int t = 0; t < n; t++)
            if (att[t] > max_val) max_val = att[t];
        float sum = 0.0f;
        for (int t = 0; t < n; t++) {
            float e = (float)exp((double)(att[t] - max_val));
            att[t] = e;
            sum += e;
        }
        float inv = 1.0f / sum;
        for (int t = 0; t < n; t++) att[t] *= inv;
        float *oh = out + (size_t)h * D;
        for (int i = 0; i < D; i++) {
            float val = 0.0f;
            for (int t = start; t <= pos; t++)
                val += att[t - start] * vcache[(size_t)t * kv_dim + (size_t)kvh * D + i];
            oh[i] = val;
        }
    }
}

int orc_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
