// Internal declarations shared by the runtime (llmp_runtime.hip) and the kernels
// (decode_attention.hip).  Nothing here is part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

#include "host_layout.h"

namespace llmp {

// Largest number of split-K partitions per KV head a decode call may use.
constexpr int kMaxSplits = 1024;
// Largest GQA group (query heads per KV head) any decode kernel ships.
constexpr int kMaxGroup = 8;
// Tokens per launch of the token-batched projections (the MFMA's N).
constexpr int kTokBatch = 16;

// Arguments of one split-K decode launch.  All pointers are device pointers.  The kernels
// derive the step plan (window start, rows per split, effective splits, RoPE row) from the
// position, which comes from `pos` or, when d_pos is set, from device memory at run time (a
// captured graph then replays at whatever position the caller stored there).
struct DecodeArgs {
    const float* q;        // [Hq*D] raw query projection
    const float* k;        // [Hkv*D] raw key projection
    const float* v;        // [Hkv*D] value projection
    float* kc;             // fp32 cache: layer K plane [Hkv][max_seq][D]
    float* vc;             // fp32 cache: layer V plane [Hkv][max_seq][D]
    signed char* kq;       // Q8_0 cache: K quants [Hkv][max_seq][D]
    float* ks;             // Q8_0 cache: K block scales [Hkv][max_seq][D/32]
    signed char* vq;
    float* vs;
    const float* cos_t;    // RoPE table [max_seq][half_rope] or nullptr (NoPE)
    const float* sin_t;
    const float* qnw;      // QK-norm weights [D] or nullptr
    const float* knw;
    const float* sinks;    // [Hq] attention-sink logits times log2(e), or nullptr
    const float* gate;     // [Hq*D] output gate (out *= sigmoid(gate)), or nullptr
    float* out;            // [Hq*D] final output (written directly when one split runs)
    float* part_o;         // [Hkv][splits][G][D] unnormalised split outputs
    float* part_ml;        // [Hkv][splits][G][2] split (max, sum) in the log2 domain
    const int* d_pos;      // device position (tokenParams[0]) or nullptr to use `pos`
    int* range;            // range exponents of the layer's rows [Hkv][K, V] (raised by the append)
    int kv_rep;            // virtual KV heads per cached KV head (grid y = n_kv_heads * kv_rep)
    int* done;             // per virtual KV head: split workgroups of the current call that have
                           // written their partials (zero between calls; dk::combine_if_last)
    int fused;             // 1: the split kernel merges the splits itself (else decode_reduce_kernel)
    long long head_stride; // floats between consecutive KV heads of a plane (max_seq*D)
    int pos;               // position of the new token (row appended) when d_pos is null
    int max_seq;           // cache rows; a device position outside [0, max_seq) is a no-op
    int window;            // > 0: attend to the last `window` rows; 0: all rows
    int splits;            // grid size: most splits per KV head (fewer run for short rows)
    int half_rope;         // rotated pairs per head
    int rope_type;         // 0 NORMAL, 2 NEOX
    int q8_trunc;          // Q8_0 append: 1 = truncate (8-lane SIMD contract), 0 = round half up
    int norm_seq;          // 1: K-norm sums squares sequentially (RMSNorm.apply with offsets)
    int v_norm;            // 1: the V row is RMS-normalised without weights before the append
    int no_append;         // 1: shared-KV layer: row `pos` is already cached, k/v are unused
    float eps;             // QK-norm epsilon
    float qk_scale;        // factor folded into q: scale*log2(e), or scale when soft-capping
    float softcap;         // 0 = off
    float softcap_log2e;   // softcap * log2(e)
    float inv_softcap;     // 1 / softcap
};

// Launches the split-K kernel for head_dim D and GQA group G = Hq/Hkv on grid
// (splits, Hkv) with `waves` (2, 4 or 8) waves per workgroup requested, over an fp32
// (q8 = false) or Q8_0 (q8 = true) cache.  Returns hipErrorInvalidValue for an unsupported
// shape.  With splits > 1, launch_decode_reduce must follow.
hipError_t launch_decode_split(const DecodeArgs& a, int head_dim, int group, int n_kv_heads,
                               int waves, bool q8, hipStream_t stream);
// Waves per workgroup the split kernel actually runs with for a request of `waves` (some
// shapes only ship 4-wave workgroups); 0 for an unsupported shape.
int decode_split_waves(int head_dim, int group, int waves, bool q8);
// Workgroups of that kernel resident per CU at once (registers and LDS), 0 on error.
int decode_split_blocks_per_cu(int head_dim, int group, int waves, bool q8);
// Launches the log-sum-exp combine of the splits: one block per query head.
// Whether a decode launch with `splits` splits of `waves`-wave workgroups merges its splits
// inside the split kernel: when the last workgroup's merge takes one round of loads
// (dk::combine_if_last with at most dk::kMergeBatch splits per thread group).
bool decode_fused_merge(int head_dim, int group, int waves, int splits);
hipError_t launch_decode_reduce(const DecodeArgs& a, int head_dim, int group, int n_heads,
                                hipStream_t stream);
// True when a decode kernel exists for (head_dim, group) (host_layout.h decode_group_ok; larger
// groups run through kernel_group's divisor, DecodeArgs::kv_rep).
bool decode_shape_supported(int head_dim, int group);

namespace pk {
struct PrefillArgs;
}
// Prefill, three launches: exact K/V append of all prompt tokens (one workgroup per token);
// tile images (the fp16 hi/lo split of key tiles [tile0, tile0 + n_tiles) of every KV head,
// V transposed) into `ws`; the MFMA causal attention over those images.  All return
// hipErrorInvalidValue for an unsupported shape.
hipError_t launch_prefill_append(const pk::PrefillArgs& a, int head_dim, hipStream_t stream);
hipError_t launch_prefill_tiles(const pk::PrefillArgs& a, int head_dim, void* ws, int tile0,
                                int n_tiles, int row_end, hipStream_t stream);
hipError_t launch_prefill_attn(const pk::PrefillArgs& a, int head_dim, int group, const void* ws,
                               int tile0, int n_tiles, int n_cu, int ksplit, hipStream_t stream);
// Key splits of a prefill call (1 unless the query blocks alone leave CUs idle: short prompts
// after a long cached prefix, speculative verification); ksplit > 1 writes partials to
// a.part_o / a.part_ml ([ksplit][P][Hq][D] and [..][2] floats) and adds a combine launch.
constexpr int kMaxPrefillSplits = 64;
int prefill_key_splits(int P, int pos0, int window, int n_kv_heads, int group, int head_dim,
                       int n_cu);
// Keys per tile and bytes per tile image (per KV head) for head_dim; 0 if unsupported.
int prefill_tile_keys(int head_dim);
size_t prefill_tile_bytes(int head_dim);

// Plain 16-byte-per-thread copy kernel.
hipError_t launch_copy(void* dst, const void* src, size_t bytes, hipStream_t stream);

namespace gk {
struct GemvArgs;
}
// Weights per lane unit of a GGML type's projection kernel (0 = no kernel for that type).
int gemv_unit(int ggml_type);
// y = W x over one to three row segments of one GGML type (optional fused pre-RMSNorm of x,
// optional residual epilogue); hipErrorInvalidValue for an unsupported type or shape.
// q8_input: Q4_K and Q8_0 rows take the Q8_1-quantised input and int8 dot products (the
// reference GPU's default matvecs); other types are unaffected.
hipError_t launch_gemv(const gk::GemvArgs& a, int ggml_type, bool q8_input, hipStream_t stream);
// The same over segments of two types in one launch (GemvSeg::fmt 0: first_type, 1: second);
// supported for first_type Q4_K with second_type Q6_K.
bool gemv_pair_supported(int first_type, int second_type);
hipError_t launch_gemv_pair(const gk::GemvArgs& a, int first_type, int second_type, bool q8_input,
                            hipStream_t stream);
// x += rscale? * rmsnorm(xb, w) over dim values, for n_tokens rows dim floats apart (one
// workgroup per row).
hipError_t launch_post_norm_residual(const float* xb, const float* w, float eps, float rscale,
                                     float* x, int dim, int n_tokens, hipStream_t stream);

namespace tk {
struct ProjTokArgs;
}
// Token-batched projections on the matrix cores (proj_tok_kernels.h): the GGML types with a
// kernel, the two-type pairs one launch takes (GemvSeg-like TokSeg::fmt 0 and 1), and the
// launch (second_type < 0: one type); hipErrorInvalidValue for an unsupported type or shape.
// Per-token factors of a token-batched projection (tk::tok_prep_kernel): sc[2t] = the RMSNorm
// factor r (1 without norm_w) and sc[2t + 1] = the range exponent of the largest x*w (or x),
// for t < n_tokens (<= kTokBatch).
hipError_t launch_tok_prep(const float* x, long long x_pitch, int cols, const float* norm_w, float eps,
                           float* sc, int n_tokens, hipStream_t stream);
bool proj_tok_supported(int ggml_type);
bool proj_tok_pair_supported(int first_type, int second_type);
// q8: the types the reference GPU runs on its Q8_1 input (proj_tok_q8_routed) take the staged
// quants of a.q8b / q8d / q8s (launch_tok_q8); the others keep the fp32 input.
hipError_t launch_proj_tok(const tk::ProjTokArgs& a, int first_type, int second_type, bool q8,
                           hipStream_t stream);
bool proj_tok_q8_routed(int ggml_type);
// The Q8_1 input of n_tokens rows for the int8 formats (tk::tok_q8_kernel): the single-token
// kernel's staged norm and quantiser, written in the B-operand layout (q8b: cols/32 * 64
// uint4, q8d and q8s: cols/32 * kTokBatch floats), kTokBatch slots (zeros past n_tokens); with
// sc, also launch_tok_prep's per-token factors.
hipError_t launch_tok_q8(const float* x, long long x_pitch, int cols, const float* norm_w, float eps,
                         int n_tokens, void* q8b, float* q8d, float* q8s, float* sc, hipStream_t stream);

}  // namespace llmp
