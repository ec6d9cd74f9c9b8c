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
       ORC_ARCH_COHERE2 = 4 };

int orc_is_global_layer(int arch, int layer)
{
    switch (arch) {
    case ORC_ARCH_GEMMA2: return layer % 2 == 1;
    case ORC_ARCH_GEMMA3: return layer % 6 == 5;
    case ORC_ARCH_GPT_OSS: return layer % 2 == 0;
    case ORC_ARCH_COHERE2: return layer % 4 == 3;
    default: return 1;
    }
}

/* Layer-independent attention hyper-parameters (the subset of ModelConfig read by
 * Attention.java:284-367). */
typedef struct {
    int n_heads;          /* headCount */
    int n_kv_heads;       /* headCountKV */
    int head_size;        /* headSize */
    int rope_dim;         /* ropeDimensionCount */
    int rope_type;        /* 0 = NORMAL, 2 = NEOX */
    int max_seq;          /* KV cache capacity */
    float norm_eps;       /* normEps (QK-norm) */
    int sliding_window;   /* 0 = none */
    float attention_scale;/* > 0 overrides 1/sqrt(headSize) */
    float softcap;        /* attnLogitSoftCap, 0 = off */
    int arch;             /* ORC_ARCH_* */
    int no_rope_interval; /* noRopeLayerInterval, 0 = off */
    int nope_on_global;   /* useNoPeOnGlobalLayers */
} orc_cfg;

/* KVCache.storeK / storeV (KVCache.java:164-179), FLOAT32 mode: cache[layer][pos*kvDim + j]. */
void orc_kv_store(float *cache_layer, int pos, const float *x, int kv_dim)
{
    memcpy(cache_layer + (size_t)pos * kv_dim, x, sizeof(float) * (size_t)kv_dim);
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

/* Attention.forwardFromProjections (Attention.java:284-367), optional bias omitted (absent
 * from every configuration this build covers).  q and k are modified in place exactly as
 * state.q / state.k are; the K/V rows are appended at `pos`; out = xb2[Hq*D].
 * use_flash != 0 selects the online-softmax loop of Attention.forward (Attention.java:161-207).
 * kcache/vcache are one layer's [max_seq][kvDim] arrays.  rope_cos/rope_sin are the table
 * the layer selects (global or local, Attention.java:317); NULL skips RoPE (NoPE layer). */
void orc_forward_from_projections(const orc_cfg *c, float *kcache, float *vcache,
                                  const float *qnorm_w, const float *knorm_w,
                                  const float *rope_cos, const float *rope_sin,
                                  float *q, float *k, const float *v,
                                  int layer, int pos, float *out, float *att_scratch,
                                  int use_flash, int n_threads)
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
    orc_kv_store(kcache, pos, k, kv_dim);
    orc_kv_store(vcache, pos, v, kv_dim);

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
        if (use_flash) {
            float max_score = -INFINITY;
            float sum_exp = 0.0f;
            for (int t = start; t <= pos; t++) {
                float score = orc_dot(qh, kcache + (size_t)t * kv_dim + kv_off, D);
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
                orc_saxpy(scale_new, vcache + (size_t)t * kv_dim + kv_off, oh, D);
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
                float score = orc_dot(qh, kcache + (size_t)t * kv_dim + kv_off, D);
                float s = score * scale;
                if (softcap > 0.0f) {
                    float r = s / softcap;
                    s = softcap * (float)tanh((double)r);
                }
                att[t - start] = s;
            }
            orc_softmax(att, seq_len);
            for (int t = start; t <= pos; t++)
                orc_saxpy(att[t - start], vcache + (size_t)t * kv_dim + kv_off, oh, D);
        }
    }
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

int orc_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
