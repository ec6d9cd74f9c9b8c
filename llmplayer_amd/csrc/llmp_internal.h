// Internal declarations shared by the runtime (llmp_runtime.hip) and the kernels
// (decode_attention.hip).  Nothing here is part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace llmp {

// Largest number of split-K partitions per KV head a decode call may use.
constexpr int kMaxSplits = 1024;

// Arguments of one split-K decode launch.  All pointers are device pointers.
struct DecodeArgs {
    const float* q;        // [Hq*D] raw query projection
    const float* k;        // [Hkv*D] raw key projection
    const float* v;        // [Hkv*D] value projection
    float* kc;             // layer K plane [Hkv][max_seq][D]
    float* vc;             // layer V plane [Hkv][max_seq][D]
    const float* cos_row;  // RoPE table row of `pos` (half_rope floats) or nullptr (NoPE)
    const float* sin_row;
    const float* qnw;      // QK-norm weights [D] or nullptr
    const float* knw;
    float* out;            // [Hq*D] final output (written directly when splits == 1)
    float* part_o;         // [Hkv][splits][G][D] unnormalised split outputs
    float* part_ml;        // [Hkv][splits][G][2] split (max, sum) in the log2 domain
    long long head_stride; // floats between consecutive KV heads of a plane (max_seq*D)
    int pos;               // position of the new token (row appended)
    int t_start;           // first attended position
    int rows_per_split;    // rows of [t_start, pos] per split
    int splits;            // number of splits per KV head
    int half_rope;         // rotated pairs per head
    int rope_type;         // 0 NORMAL, 2 NEOX
    float eps;             // QK-norm epsilon
    float qk_scale;        // factor folded into q: scale*log2(e), or scale when soft-capping
    float softcap;         // 0 = off
    float softcap_log2e;   // softcap * log2(e)
    float inv_softcap;     // 1 / softcap
};

// Launches the split-K kernel for head_dim D and GQA group G = Hq/Hkv on grid
// (splits, Hkv) with `waves` (4 or 8) waves per workgroup.  Returns hipErrorInvalidValue for
// an unsupported shape.  With splits > 1, launch_decode_reduce must follow.
hipError_t launch_decode_split(const DecodeArgs& a, int head_dim, int group, int n_kv_heads,
                               int waves, hipStream_t stream);
// Launches the log-sum-exp combine of the splits: one block per query head.
hipError_t launch_decode_reduce(const DecodeArgs& a, int head_dim, int group, int n_heads,
                                hipStream_t stream);
// True when a decode kernel exists for (head_dim, group).
bool decode_shape_supported(int head_dim, int group);

namespace pk {
struct PrefillArgs;
}
// Prefill: exact K/V append of all prompt tokens (one workgroup per token), then the MFMA
// causal attention.  Both return hipErrorInvalidValue for an unsupported shape.
hipError_t launch_prefill_append(const pk::PrefillArgs& a, int head_dim, hipStream_t stream);
hipError_t launch_prefill_attn(const pk::PrefillArgs& a, int head_dim, int group,
                               hipStream_t stream);

// Plain 16-byte-per-thread copy kernel.
hipError_t launch_copy(void* dst, const void* src, size_t bytes, hipStream_t stream);

}  // namespace llmp
