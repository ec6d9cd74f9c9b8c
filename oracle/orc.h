/* orc.h -- TEST INFRASTRUCTURE ONLY: declarations shared by the oracle's C files. */
#ifndef ORC_H
#define ORC_H

/* Attention hyper-parameters read by Attention.forwardFromProjections. */
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
    const float *sinks;   /* per query head attention-sink logits (GPT-OSS), NULL = none */
} orc_cfg;

float orc_dot(const float *a, const float *b, int len);
void orc_forward_from_projections(const orc_cfg *c, float *kcache, float *vcache,
                                  const float *qnorm_w, const float *knorm_w,
                                  const float *rope_cos, const float *rope_sin,
                                  float *q, float *k, const float *v,
                                  int layer, int pos, float *out, float *att_scratch,
                                  int use_flash, int n_threads);

#endif
