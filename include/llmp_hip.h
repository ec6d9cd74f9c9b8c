/*
 * llmp_hip.h -- C ABI of libllmp_hip.so, the MI355X (gfx950) attention path for LLMPlayer.
 *
 * The library replaces, for the attention steps of the GPU forward pass, what the reference
 * reaches through CudaBindings / CudaContext (FFM downcalls into libcuda + NVRTC kernels):
 * steps 2b'-5 of CudaForwardPass.forwardAttentionPart (per-head QK-norm, RoPE, KV append,
 * scores / softmax / PV).  Paths cited below are relative to the reference tree
 * (src/main/java21/it/denzosoft/llmplayer/... unless stated otherwise).
 *
 * Conventions (shaped for a Panama FFM binding, as CudaBindings.java:23-95 binds libcuda):
 *  - every function returns an int status: LLMP_OK (0) on success, like CUDA_SUCCESS
 *    (CudaBindings.java:15); a non-zero status carries a message readable with
 *    llmp_last_error (per calling thread);
 *  - device pointers, streams, events and handles are uint64_t (bound as JAVA_LONG, the way
 *    CUdeviceptr is, CudaBindings.java:133-158); scalars are int32 / float;
 *  - host arrays are plain pointers (FFM MemorySegment addresses);
 *  - stream 0 means the library's own stream (created by llmp_init); launches on one stream
 *    run in order.  A handle is single-owner and not re-entrant: calls on one handle must not
 *    overlap (the reference keeps one GPU KV cache per forward pass, CudaForwardPass.java:407-416).
 *  - every entry point makes the library's device current on the calling thread first, so
 *    any Java thread may call it (HIP device selection is per thread).
 */
#ifndef LLMP_HIP_H
#define LLMP_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------------------------- */
#define LLMP_OK                 0
#define LLMP_ERR_INVALID_ARG    1  /* bad size, null pointer, unsupported shape            */
#define LLMP_ERR_OUT_OF_RANGE   2  /* layer / position outside the cache                    */
#define LLMP_ERR_NOT_INIT       3  /* llmp_init not called                                  */
#define LLMP_ERR_NO_DEVICE      4  /* no HIP device / wrong architecture                    */
#define LLMP_ERR_OUT_OF_MEMORY  5  /* allocation would not fit in free HBM                  */
#define LLMP_ERR_UNSUPPORTED    6  /* shape or mode this build has no kernel for            */
#define LLMP_ERR_HIP            7  /* a HIP runtime call failed (message has the HIP error) */
#define LLMP_ERR_BAD_HANDLE     8  /* unknown or destroyed handle                           */

/* ---- enums ----------------------------------------------------------------------------- */
#define LLMP_KV_F32             0  /* fp32 cache rows (KVCache.Mode.FLOAT32, KVCache.java:79) */
#define LLMP_KV_Q8_0            1  /* int8 quants + fp32 scale per 32 values (KVCache.Mode.Q8_0,
                                      KVCache.java:11-28, 79; 1.125 bytes per value); the
                                      appended row rounds half up like quantizeBlocksScalar
                                      (KVCache.java:218-243)                                  */
#define LLMP_KV_Q8_0_TRUNC      2  /* the same format, appended rows truncated toward zero like
                                      SimdQ8KvOps.quantize (SimdQ8KvOps.java:86-117), the
                                      contract the JVM runs on 8-lane (AVX2) hosts            */

#define LLMP_ROPE_NORMAL        0  /* pairs (2i, 2i+1)    RoPE.ROPE_TYPE_NORMAL, RoPE.java:18 */
#define LLMP_ROPE_NEOX          2  /* pairs (i, i + R/2)  RoPE.ROPE_TYPE_NEOX,   RoPE.java:19 */

#define LLMP_ROPE_SEL_NONE     -1  /* NoPE layer (Attention.java:311-320 skip)               */
#define LLMP_ROPE_SEL_GLOBAL    0  /* Attention.rope                                         */
#define LLMP_ROPE_SEL_LOCAL     1  /* Attention.ropeLocal (Gemma 3 local theta, Attention.java:317) */

/* ---- context (replaces CudaContext.create / close, CudaContext.java:102-160) ----------- */

/* Select HIP device `device`, check it is gfx950 and create the library stream. */
int llmp_init(int device);
/* Destroy every handle, the stream and the library's device allocations. */
int llmp_shutdown(void);
/* Device facts (DeviceInfo.java:1-22): compute units, total and free HBM bytes, and the
 * architecture name (NUL-terminated, truncated to name_len). Any out pointer may be NULL. */
int llmp_device_info(int *n_cu, int64_t *hbm_total, int64_t *hbm_free, char *name, int name_len);
/* Copy the calling thread's last error message (NUL-terminated) into buf. */
int llmp_last_error(char *buf, int len);

/* ---- memory and streams (CudaContext.allocBuffer / writeBuffer / readBuffer /
 *      fillBufferZero / finish, CudaContext.java:368-491, 578-628) ------------------------- */
int llmp_malloc(uint64_t *dptr, uint64_t bytes);
int llmp_free(uint64_t dptr);
int llmp_memcpy_htod(uint64_t dst, const void *src, uint64_t bytes, uint64_t stream);
int llmp_memcpy_dtoh(void *dst, uint64_t src, uint64_t bytes, uint64_t stream);
int llmp_memcpy_dtod(uint64_t dst, uint64_t src, uint64_t bytes, uint64_t stream);
/* Zero `bytes` of device memory (hipMemsetAsync: not for use inside a graph capture). */
int llmp_memset_zero(uint64_t dst, uint64_t bytes, uint64_t stream);
int llmp_stream_create(uint64_t *stream);
int llmp_stream_destroy(uint64_t stream);
int llmp_stream_sync(uint64_t stream);
int llmp_event_create(uint64_t *event);
int llmp_event_destroy(uint64_t event);
int llmp_event_record(uint64_t event, uint64_t stream);
int llmp_event_sync(uint64_t event);
int llmp_event_elapsed_ms(float *ms, uint64_t start, uint64_t end);

/* ---- device KV cache (CudaForwardPass.java:407-416 per-layer K/V buffers; sizing as
 *      LLMEngine.estimateKvCache, LLMEngine.java:917-928) --------------------------------- */

/* One zero-filled device pool for n_layers x {K,V}, laid out head-major.  LLMP_KV_F32:
 * [layer][K|V][kv_head][pos][head_dim] fp32.  LLMP_KV_Q8_0(_TRUNC): per layer the K quants
 * [kv_head][pos][head_dim] int8, K scales [kv_head][pos][head_dim/32] fp32, then the same for
 * V.  The pool also holds each layer's range exponents (below).  Fails with
 * LLMP_ERR_OUT_OF_MEMORY when the pool would not fit in free HBM.  head_dim must be 64, 128 or
 * 256 (any cache type), 96 (fp32 caches: Phi-3), 80 (fp32 caches, decode only: Phi-2) or 512
 * (fp32 caches and decode only, the full-attention layers of Gemma 4, whose two head sizes take
 * one handle each).  Kernels are instantiated for GQA groups 1-8 (1-4 at head_dim 96, 1-2 at 80);
 * a larger group (GLM-4's 16 or 24 query heads per KV head) runs as several groups of its
 * largest instantiated divisor per KV head, so every group is accepted.
 *
 * Range exponents: per layer and KV head, E = max(0, floor(log2 max|x|) - 14) over every K (and
 * V) value stored since the pool was created or cleared, raised by each append and by
 * llmp_kv_write(_q8).  The multi-token calls split rows into fp16 hi/lo parts, which hold
 * magnitudes below 65504, and scale them by 2^-E first.  Values written through the addresses of
 * llmp_kv_layer_ptrs are not tracked: keep them below 2^15 in magnitude, or write them with
 * llmp_kv_write. */
int llmp_kv_create(int n_layers, int max_seq, int n_kv_heads, int head_dim, int dtype,
                   uint64_t *handle);
int llmp_kv_destroy(uint64_t handle);
/* Read rows [pos0, pos0+n) of one layer into host arrays in the reference layout
 * [pos][kvDim] (KVCache.keyLayer / valueLayer, KVCache.java:149-161).  Either out may be NULL.
 * fp32 caches only (LLMP_ERR_UNSUPPORTED on a Q8_0 cache: use llmp_kv_read_q8). */
int llmp_kv_read(uint64_t handle, int layer, int pos0, int n, float *host_k, float *host_v);
/* Write rows [pos0, pos0+n) of one layer from host arrays in the reference layout
 * (the inverse of llmp_kv_read; restores a saved prefix, ConversationCache.java:36-56). */
int llmp_kv_write(uint64_t handle, int layer, int pos0, int n, const float *host_k,
                  const float *host_v);
/* Q8_0 caches: rows [pos0, pos0+n) of one layer in the reference's Q8_0 layout
 * (KVCache.keyQuants / keyScales, KVCache.java:91-94): quants [pos][kvDim] int8 and scales
 * [pos][kvDim/32] fp32, for K and V.  Any out may be NULL. */
int llmp_kv_read_q8(uint64_t handle, int layer, int pos0, int n, int8_t *k_quants,
                    float *k_scales, int8_t *v_quants, float *v_scales);
/* The inverse of llmp_kv_read_q8. */
int llmp_kv_write_q8(uint64_t handle, int layer, int pos0, int n, const int8_t *k_quants,
                     const float *k_scales, const int8_t *v_quants, const float *v_scales);
/* Device addresses of one layer's K and V planes ([kv_head][pos][head_dim] fp32, or the quant
 * planes of a Q8_0 cache).  Rows written through them do not raise the range exponents (see
 * llmp_kv_create). */
int llmp_kv_layer_ptrs(uint64_t handle, int layer, uint64_t *k_plane, uint64_t *v_plane);
/* Zero the whole pool and its range exponents (a new conversation; hipMemsetAsync: not for use
 * inside a graph capture). */
int llmp_kv_clear(uint64_t handle, uint64_t stream);

/* ---- RoPE tables (RoPE.java:45-106; upload as CudaForwardPass.java:398-402) ------------ */

/* Host helper: fill cos/sin tables [max_seq][rope_dim/2] exactly as the RoPE constructor
 * does (non-YaRN branch, RoPE.java:80-105): freq_i = (float)(1/pow(theta, 2i/R)) / ff[i]
 * * freqScale, angle = (float)pos * freq_i, cos = (float)cos(angle), sin = (float)sin(angle).
 * freq_factors may be NULL; linear_freq_scale <= 1 means no scaling. */
int llmp_rope_table(int rope_dim, int max_seq, float theta, float linear_freq_scale,
                    const float *freq_factors, int n_freq_factors, float *cos_out,
                    float *sin_out);
/* Host helper: the YaRN branch of the RoPE constructor (RoPE.java:45-117 with YarnParams, the
 * tables of the MoE and MLA engines, Qwen3MoEInferenceEngine.java:60-66): NTK-by-parts blend of
 * freq_i and freq_i/scaling_factor between the correction dims of beta_fast and beta_slow
 * (RoPE.yarnCorrDim, yarnRamp), angles and cos/sin as llmp_rope_table.  *mscale (may be NULL)
 * receives the attention-magnitude factor; the engines scale scores by mscale^2/sqrt(headSize)
 * (Qwen3MoEInferenceEngine.java:277-279), which llmp_layer_config takes as its custom scale.
 * scaling_factor <= 1 builds the plain table with mscale 1.  The reference's defaults are
 * beta_fast 32, beta_slow 1 (RoPE.YarnParams). */
int llmp_rope_table_yarn(int rope_dim, int max_seq, float theta, const float *freq_factors,
                         int n_freq_factors, float scaling_factor, int orig_ctx, float beta_fast,
                         float beta_slow, float yarn_log_mul, float *cos_out, float *sin_out,
                         float *mscale);
/* Upload a table ([max_seq][half_rope] each) as the global or local table of a handle.
 * `which` is LLMP_ROPE_SEL_GLOBAL or LLMP_ROPE_SEL_LOCAL.  The reference uploads only the
 * global table (CudaForwardPass.java:398-402); the local one serves Gemma 3 local layers
 * (InferenceEngine.java:58-78, Attention.java:317). */
int llmp_rope_upload(uint64_t handle, int which, const float *cos_t, const float *sin_t,
                     int max_seq, int half_rope);

/* ---- per-layer attention configuration (ModelConfig fields read by
 *      Attention.forwardFromProjections, Attention.java:284-367) ------------------------- */

/* n_heads / n_kv_heads / head_dim: headCount, headCountKV, headSize (n_kv_heads and head_dim
 * must equal the handle's).  rope_type: LLMP_ROPE_NORMAL / LLMP_ROPE_NEOX.  rope_sel:
 * LLMP_ROPE_SEL_*.  window: slidingWindow (0 = none); is_global: Attention.isGlobalLayer
 * (Attention.java:250-276) -- a global layer ignores the window.  scale: attentionScale, or
 * <= 0 for (float)(1/sqrt(headSize)) (Attention.java:326-328).  softcap: attnLogitSoftCap
 * (0 = off, Attention.java:352-354).  eps: normEps for QK-norm.  qnorm_w / knorm_w: host
 * arrays of head_dim floats (RMSNorm.cacheWeights, Attention.java:53-64) or NULL for no
 * QK-norm (both or neither).  Called once per layer at set-up; it may allocate. */
int llmp_layer_config(uint64_t handle, int layer, int n_heads, int n_kv_heads, int head_dim,
                      int rope_type, int rope_sel, int window, int is_global, float scale,
                      float softcap, float eps, const float *qnorm_w, const float *knorm_w);

/* Attention sinks of a layer (GPT-OSS, Qwen3MoEInferenceEngine.java:88-95, 295, 309-313):
 * sinks[n_heads] host fp32 logits in the units of the scaled scores.  Each one joins its
 * query head's softmax max and denominator and takes no value (softmaxWithSink,
 * Qwen3MoEInferenceEngine.java:562-575); decode and prefill apply them.  NULL removes them; a
 * later llmp_layer_config with another head count removes them too.  May allocate. */
int llmp_layer_sinks(uint64_t handle, int layer, const float *sinks);

/* Norm order of a layer (Gemma 4, Gemma4InferenceEngine.java:318-355).  Bits:
 *   LLMP_NORM_SEQUENTIAL  the K-norm sums squares one value at a time, unfused (RMSNorm.apply
 *                         with offsets, RMSNorm.java:24-35) instead of SimdVectorOps.dot's
 *                         8-lane FMA order; the appended K row follows it bit for bit.
 *   LLMP_NORM_V           the V row is RMS-normalised without weights before it is stored
 *                         (RMSNorm.applyNoScale, RMSNorm.java:40-50), in the sequential order.
 * 0 (the default) is the Attention.forwardFromProjections behaviour.  Decode and prefill apply
 * both; the query's norm (never stored) keeps the fast order, a difference far inside the
 * output tolerance. */
#define LLMP_NORM_SEQUENTIAL 1
#define LLMP_NORM_V          2
int llmp_layer_norm_mode(uint64_t handle, int layer, int mode);

/* ---- decode attention: one layer-call for one new token --------------------------------
 * Replaces CudaForwardPass.forwardAttentionPart steps 2b'-5 (CudaForwardPass.java:1529-1570):
 * rmsnorm_per_head (Q, K) -> rope_apply (Q, K) -> kv_cache_update -> attention_full, with the
 * CPU semantics of Attention.forwardFromProjections (Attention.java:284-367): sliding window,
 * local/global RoPE, soft-cap, custom scale.
 *   q:   device fp32 [n_heads*head_dim]   raw projection (read only: unlike the reference's
 *                                         in-place kernels, q and k are not rewritten)
 *   k,v: device fp32 [n_kv_heads*head_dim]
 *   out: device fp32 [n_heads*head_dim]   (gpuXb2)
 * The K row stored at `position` is QK-norm + RoPE of k, bit-identical to the CPU path's
 * KVCache.storeK; the V row is v.  splits: number of split-K partitions per KV head (1..1024),
 * or <= 0 to let the library choose.  Errors: LLMP_ERR_OUT_OF_RANGE for position outside
 * [0, max_seq) or a bad layer; LLMP_ERR_INVALID_ARG for a layer never configured. */
int llmp_attn_decode(uint64_t handle, int layer, int position, uint64_t q, uint64_t k,
                     uint64_t v, uint64_t out, int splits, uint64_t stream);

/* The same layer-call with the position read from device memory when the kernels run:
 * d_position points to an int32 holding the position (the reference's tokenParams[0],
 * CudaForwardPass.java:138-141, written per token by uploadXAndUpdateParams, :1283-1292).
 * The launch is planned for the longest step of the layer (position max_seq-1), so one
 * capture of this call (llmp_graph_*) replays correctly at every position: the kernels derive
 * the window, rows per split and the splits actually used from the device value.  A device
 * position outside [0, max_seq) makes the call a no-op (nothing is read or written). */
int llmp_attn_decode_devpos(uint64_t handle, int layer, uint64_t d_position, uint64_t q,
                            uint64_t k, uint64_t v, uint64_t out, int splits, uint64_t stream);

/* llmp_attn_decode (d_position == 0) or llmp_attn_decode_devpos (d_position != 0, `position`
 * unused) with an optional output gate: gate, when non-zero, is a device fp32 [n_heads *
 * head_dim] array and out = attention * sigmoid(gate), sigmoid(x) = 1/(1 + exp(-x)) (the
 * Qwen3.5 attention output gate, Qwen35InferenceEngine.java:580-583, 628-630; on the reference
 * GPU a separate sigmoid-multiply launch, Qwen35CudaForwardPass.java:1136-1137). */
int llmp_attn_decode_ex(uint64_t handle, int layer, int position, uint64_t d_position,
                        uint64_t q, uint64_t k, uint64_t v, uint64_t gate, uint64_t out,
                        int splits, uint64_t stream);

/* Decode for a shared-KV layer (Gemma 4: the last sharedKvLayers layers reuse the cache of an
 * earlier layer of the same type and compute no K/V, Gemma4InferenceEngine.java:171-180,
 * 336-366): `layer`'s configuration (heads, window, RoPE, q-norm, scale, sinks) over the rows
 * of `src_layer`'s cache in the same handle, which must already hold row `position`; nothing
 * is appended.  position / d_position and gate as in llmp_attn_decode_ex. */
int llmp_attn_decode_shared(uint64_t handle, int layer, int src_layer, int position,
                            uint64_t d_position, uint64_t q, uint64_t gate, uint64_t out,
                            int splits, uint64_t stream);

/* Launch plan llmp_attn_decode would use for this call: splits per KV head, waves per
 * workgroup (2, 4 or 8), rows per split and the first attended position.  Any out may be NULL. */
int llmp_decode_plan(uint64_t handle, int layer, int position, int splits, int *out_splits,
                     int *out_waves, int *out_rows_per_split, int *out_start);

/* ---- graph capture (CudaContext.beginCapture / endCapture / launchGraph,
 *      CudaContext.java:585-613): record a sequence of launches on a stream once, replay it
 *      with one call.  Arguments (positions included) are frozen at capture time. ---------- */
/* Start capturing the work enqueued on `stream` (0 = the library stream; capture mode
 * "thread local").  Profiling must be off while capturing.  A graph holds the device addresses
 * its launches had at capture time.  Decode's split workspace is allocated once by
 * llmp_kv_create and never moves, but set-up calls (llmp_layer_config, llmp_layer_sinks,
 * llmp_rope_upload, llmp_layer_weight) and a prefill call that grows the handle's prefill
 * workspace can free memory an earlier graph refers to: capture after set-up, and capture
 * again after any of them. */
int llmp_graph_begin(uint64_t stream);
/* Stop capturing and instantiate the graph; *graph receives an executable-graph handle. */
int llmp_graph_end(uint64_t stream, uint64_t *graph);
int llmp_graph_launch(uint64_t graph, uint64_t stream);
int llmp_graph_destroy(uint64_t graph);

/* ---- prefill attention: n_tokens prompt tokens in one call --------------------------------
 * The reference runs a prompt as n_tokens sequential single-token forwards
 * (InferenceEngine.prefill, InferenceEngine.java:374-381; LLMEngine.java:478-480); this call
 * computes the same attention outputs and cache rows for positions pos0 .. pos0+n_tokens-1:
 *   q:   device bf16 [n_tokens][n_heads*head_dim]
 *   k,v: device bf16 [n_tokens][n_kv_heads*head_dim]
 *   out: device fp32 [n_tokens][n_heads*head_dim] (16-byte aligned)
 * K/V rows are appended exactly as n_tokens llmp_attn_decode calls would write them (inputs
 * widened to fp32, QK-norm and RoPE in the CPU path's float order).  Token i attends causally
 * to rows [start(pos0+i), pos0+i] (start from the layer's sliding window), on MFMA with bf16
 * hi/lo split operands and fp32 accumulation.  Rows before pos0 must already be in the cache.
 * Over a Q8_0 cache each new row is quantised exactly as a decode append quantises it (under
 * the handle's contract) and attention reads every row dequantised (quant * block scale), as
 * the reference's sequential forwards over KVCache Mode.Q8_0 do.
 * Partial RoPE (rotated dims < head_dim, NORMAL or NEOX pairs) is applied as in decode.
 * The handle keeps a workspace for the key tiles a call attends (fp16 hi/lo images of K and
 * V: about 9 bytes per key, KV head and head_dim element); a call that needs more than any
 * earlier call grows it (hipFree + hipMalloc: such a call cannot be captured in a graph, and
 * graphs captured before it must not be replayed after it). */
int llmp_attn_prefill(uint64_t handle, int layer, int pos0, int n_tokens, uint64_t q,
                      uint64_t k, uint64_t v, uint64_t out, uint64_t stream);
/* llmp_attn_prefill with an optional output gate (device fp32 [n_tokens][n_heads*head_dim],
 * 0 = none): out = attention * sigmoid(gate), as llmp_attn_decode_ex applies it. */
int llmp_attn_prefill_ex(uint64_t handle, int layer, int pos0, int n_tokens, uint64_t q,
                         uint64_t k, uint64_t v, uint64_t gate, uint64_t out, uint64_t stream);
/* Prefill of a shared-KV layer (llmp_attn_decode_shared for n_tokens tokens): `layer`'s
 * configuration over src_layer's rows, which must already hold positions pos0 ..
 * pos0+n_tokens-1 (the source layer ran the same tokens first); nothing is appended. */
int llmp_attn_prefill_shared(uint64_t handle, int layer, int src_layer, int pos0, int n_tokens,
                             uint64_t q, uint64_t gate, uint64_t out, uint64_t stream);

/* Multi-token attention on fp32 projections: the contract of the reference's own prompt and
 * speculative-verification path, which runs the tokens as sequential fp32 forwards
 * (InferenceEngine.prefill, InferenceEngine.java:374-381; LLMEngine.forwardBatch,
 * LLMEngine.java:1019-1033) and stores the fp32 k/v rows (Attention.java:284-367,
 * KVCache.java:164-179).  As llmp_attn_prefill_ex, with
 *   q:   device fp32 [n_tokens][n_heads*head_dim]   (4-byte aligned)
 *   k,v: device fp32 [n_tokens][n_kv_heads*head_dim]
 * The appended rows are bit-identical to n_tokens llmp_attn_decode calls on the same fp32
 * inputs; attention runs on the same fp16 hi/lo MFMA path (K, Q, V and P each split into two
 * fp16 parts, ~2^-22 of each operand's magnitude).  Range: any finite input.  K and V rows are
 * scaled by their layer's range exponents (llmp_kv_create) and the queries of each 16-token block
 * by the exponent of their largest magnitude before the split, so values beyond fp16's 65504
 * keep that precision; scores of ~1e3 and more are then resolved to ~2^-21 of their magnitude
 * (fp32: 2^-24).  gate may be 0.  The bf16 entry points take the same path. */
int llmp_attn_prefill_f32(uint64_t handle, int layer, int pos0, int n_tokens, uint64_t q,
                          uint64_t k, uint64_t v, uint64_t gate, uint64_t out, uint64_t stream);
/* No counterpart in the reference.  For callers that cannot allocate device memory: code under
 * HIP graph capture, serving loops and harnesses that forbid hipMalloc.  llmp_attn_prefill_f32
 * with its workspace (the key-tile images, or the split-K partials of a short chunk after a
 * long prefix) in a static device array of LLMP_PREFILL_STATIC_BYTES that each GPU holds until
 * the process ends, instead of the handle's grown workspace: the call allocates and frees
 * nothing (and records no profiling events).  A call whose workspace would exceed the array
 * fails with LLMP_ERR_INVALID_ARG: images take Hkv * ceil(keys/TK) * tile bytes (2048 tokens at
 * head_dim 64 with 8 KV heads: 9.2 MB; at head_dim 128: 17.8 MB), partials ksplit * n_tokens *
 * n_heads * (head_dim + 2) * 4 bytes (16 tokens after a 32k prefix at 24/8/128: 12.8 MB).
 * Every call on a GPU shares its one array, which keeps the last call's contents (every byte a
 * call reads it first writes): calls that overlap in time on one GPU (other streams, other
 * threads) race. */
#define LLMP_PREFILL_STATIC_BYTES (32u << 20)
int llmp_attn_prefill_f32_static(uint64_t handle, int layer, int pos0, int n_tokens,
                                 uint64_t q, uint64_t k, uint64_t v, uint64_t gate, uint64_t out,
                                 uint64_t stream);
/* llmp_attn_prefill_shared with an fp32 q (device fp32 [n_tokens][n_heads*head_dim]). */
int llmp_attn_prefill_shared_f32(uint64_t handle, int layer, int src_layer, int pos0,
                                 int n_tokens, uint64_t q, uint64_t gate, uint64_t out,
                                 uint64_t stream);

/* ---- the attention half of a layer around the attention core ------------------------------
 * Replaces CudaForwardPass.forwardAttentionPart steps 1-2b and 6-6c (CudaForwardPass.java:
 * 1498-1527, 1572-1587) with the CPU path's semantics (TransformerBlock.forward's attention
 * half and Attention.forward's projections, Attention.java:76-110, 232-238): x (the residual
 * stream, gpuX) becomes x + rscale? * postnorm?(Wo . attention(W{q,k,v} . rmsnorm(x) + bias)
 * + o_bias).  Projection weights keep their GGUF type; the library repacks them at upload. */
/* GGMLType ids (GGMLType.java:4-35) with a projection kernel. */
#define LLMP_GGML_F32    0
#define LLMP_GGML_F16    1
#define LLMP_GGML_Q4_0   2   /* the reference's nibble order: element 2i low, 2i+1 high      */
#define LLMP_GGML_Q8_0   8
#define LLMP_GGML_Q4_K  12
#define LLMP_GGML_Q6_K  14
#define LLMP_GGML_BF16  30
#define LLMP_GGML_Q5_0   6   /* split nibbles: element i low nibble of byte i, 16+i high      */
#define LLMP_GGML_Q3_K  11
#define LLMP_GGML_Q5_K  13
#define LLMP_GGML_IQ4_NL 20  /* split nibbles, as Q5_0                                         */
#define LLMP_GGML_IQ4_XS 23  /* split nibbles within each sub-block of 32 (its dot() order)   */
#define LLMP_GGML_MXFP4 39   /* split nibbles; E8M0 exponent byte first                       */
#define LLMP_GGML_Q5_1   7   /* split nibbles, as Q5_0; value q*d + m                           */
#define LLMP_GGML_Q2_K  10   /* the reference's order: element j at bits 2(j%4) of qs byte j/4 */
#define LLMP_GGML_IQ3_XXS 18 /* codebook format (256 lattice words of 4 bytes)                 */
#define LLMP_GGML_IQ3_S 21   /* codebook format; ninth index bits read as the reference does  */
#define LLMP_GGML_IQ2_S 22   /* codebook format (1024 lattice words of 8 bytes)                */
/* Weight slots of a layer (TransformerLayerWeights): matrices are [rows][cols] in GGUF row
 * order; vectors are fp32. */
#define LLMP_W_ATTN_NORM      0  /* [dim] attnNorm RMSNorm weights; absent: x is copied (OLMo2) */
#define LLMP_W_Q              1  /* [n_heads*head_dim][dim]                                     */
#define LLMP_W_K              2  /* [n_kv_heads*head_dim][dim]                                  */
#define LLMP_W_V              3  /* [n_kv_heads*head_dim][dim]                                  */
#define LLMP_W_QKV            4  /* merged [q_dim + 2*kv_dim][dim] (Phi-3); replaces Q, K, V     */
#define LLMP_W_O              5  /* [dim][n_heads*head_dim]                                     */
#define LLMP_W_Q_BIAS         6  /* [q_dim]  (Qwen2)                                            */
#define LLMP_W_K_BIAS         7  /* [kv_dim]                                                    */
#define LLMP_W_V_BIAS         8  /* [kv_dim]                                                    */
#define LLMP_W_O_BIAS         9  /* [dim]    attn_output.bias                                   */
#define LLMP_W_POST_ATTN_NORM 10 /* [dim]    postAttnNorm (Gemma 2/3, GLM4, OLMo2)              */
#define LLMP_W_SLOTS          11
/* Model-wide block parameters: dim = embeddingLength (a multiple of 32, at most 16384);
 * residual_scale = Granite's residualScale (0 = off). */
int llmp_block_config(uint64_t handle, int dim, float residual_scale);
/* How the block's projections read their input.  LLMP_INPUT_F32 (the default): every type
 * takes the fp32 (normalised) input, the CPU engine's arithmetic (FloatTensor.matmul).
 * LLMP_INPUT_Q8_1: Q4_K, Q8_0, Q5_0, Q3_K, Q5_K, IQ4_NL and IQ4_XS weights take a Q8_1 copy
 * of the input (blocks of 32: scale max|x|/127, int8 quants, block sum) and exact int8 dot
 * products, the reference GPU's default matvecs (CudaForwardPass.java:783-790 cuda.dp4a,
 * :216-226 and :1998-2090; quantize_q8.cu, rmsnorm_quantize.cu, matmul_<type>_dp4a*.cu); the
 * other types (F32, F16, BF16, Q4_0, Q5_1, Q2_K, Q6_K, MXFP4, IQ3_XXS, IQ3_S, IQ2_S) keep the
 * fp32 input, as there. */
#define LLMP_INPUT_F32   0
#define LLMP_INPUT_Q8_1  1
int llmp_block_input_mode(uint64_t handle, int mode);
/* Upload one slot of a configured layer: data = host bytes in the GGUF layout of ggml_type
 * (rows * row_bytes; fp32 for the vectors), or NULL to clear the slot.  The weight is repacked
 * into per-row planes on the device.  Set-up only: it allocates and synchronises. */
int llmp_layer_weight(uint64_t handle, int layer, int slot, int ggml_type, int rows, int cols,
                      const void *data, uint64_t nbytes);
/* The attention half of one layer on the device residual x (fp32 [dim], updated in place):
 * pre-norm and Q/K/V projections, the attention core of llmp_attn_decode (its K/V append,
 * window, QK-norm, RoPE and sinks), output projection, post-norm, residual scale and add.
 * position / d_position as in llmp_attn_decode_ex; no allocation, so it can be captured. */
int llmp_attn_block(uint64_t handle, int layer, int position, uint64_t d_position, uint64_t x,
                    int splits, uint64_t stream);

/* The attention half of n_tokens consecutive tokens (positions pos0 .. pos0+n_tokens-1) on the
 * device residual rows x (fp32 [n_tokens][dim], 16-byte aligned, updated in place): what
 * n_tokens llmp_attn_block calls compute, with each projection weight read once per group of
 * up to 16 tokens (a group of one token runs the single-token call, which is faster for one
 * token).  Replaces LLMEngine.forwardBatch's per-token attention halves
 * (LLMEngine.java:1019-1033), batched as docs/optimization/speculative-decoding.md:120-140
 * plans for the verification of K draft tokens.  The projections run on the matrix cores with
 * each fp32 input split into two fp16 parts (fp32-accurate products, fp32 sums in another order
 * than the CPU path); any finite residual is taken: the inputs of a group are scaled by a power
 * of two that brings the largest below 2^15 (a small first kernel computes it with each token's
 * RMSNorm factor), the outputs by its inverse.  The attention is llmp_attn_prefill_f32's (the
 * appended rows bit-identical to single-token appends of the same projections).  In the
 * LLMP_INPUT_Q8_1 mode the routed types take each token's Q8_1 input as llmp_attn_block
 * forms it (the same staged norm and quantiser) and exact integer block dots on the matrix
 * cores, and Wo the quantised attention output.  At head_dim 80 (no prefill kernel) and for
 * layers whose fp32 or bf16 weights reach 65504, the tokens run one llmp_attn_block call each.  The call may grow the
 * handle's prefill workspace, as llmp_attn_prefill_f32 does (not for use under graph capture
 * then). */
int llmp_attn_block_batch(uint64_t handle, int layer, int pos0, int n_tokens, uint64_t x,
                          uint64_t stream);

/* ---- profiling (the reference's -Dcuda.profile section timers,
 *      CudaForwardPass.java:1646-1737, as HIP events around each kernel) ------------------ */
#define LLMP_PROF_DECODE_SPLIT   0  /* split-K decode kernel (QK-norm, RoPE, append, QK/softmax/PV;
                                        its last workgroup per KV head merges the splits where the
                                        launch plan allows: the 2- and 8-wave plans whose partials
                                        fit one batch of loads per thread)                      */
#define LLMP_PROF_DECODE_REDUCE  1  /* log-sum-exp combine of the splits (no launch, so no count,
                                        when one split or the split kernel merged them)          */
#define LLMP_PROF_PREFILL_APPEND 2  /* prefill: exact K/V append of the prompt tokens       */
#define LLMP_PROF_PREFILL_ATTN   3  /* prefill: key-tile images + MFMA causal attention      */
#define LLMP_PROF_KINDS          4
/* on != 0 records a HIP event pair around every launch of the handle's kernels. */
int llmp_profile_enable(uint64_t handle, int on);
/* Waits for recorded launches of `kind` and returns their count and summed duration (ms)
 * since the last reset. */
int llmp_profile_read(uint64_t handle, int kind, int *count, double *total_ms);
int llmp_profile_reset(uint64_t handle);

/* ---- utilities ---------------------------------------------------------------------------
 * A plain device-to-device copy kernel (one 16-byte load and store per thread); used to
 * calibrate HBM byte counters against a kernel of known traffic.  bytes % 16 == 0. */
int llmp_copy_kernel(uint64_t dst, uint64_t src, uint64_t bytes, uint64_t stream);

#ifdef __cplusplus
}
#endif
#endif /* LLMP_HIP_H */
