// Split-K flash-decoding kernels for one new token, gfx950 (CDNA4, wave64).  Included by
// decode_attention.hip, which instantiates the shapes the library ships.
//
// One workgroup = (split j, KV head g): it owns rows [t_start + j*R, ...) of that KV head and
// every query head of its GQA group (Hq/Hkv heads), so each KV byte is read from HBM once per
// layer-call.  It also does the per-token prep of the reference's separate kernels
// (rmsnorm_per_head, rope_apply, kv_cache_update: CudaForwardPass.java:1529-1564) for its own
// heads.  With more than one split, a second small kernel merges the splits (log-sum-exp
// combine); a layer-call is one or two launches.
//
// Bit-exactness of the appended K row: it is computed with the CPU path's float step order --
// sum of squares in the SimdVectorOps.dot order (8 FMA lanes, lanes summed left to right,
// SimdVectorOps.java:17-31), r = 1/(float)sqrt((double)(ss/D + eps)) (Attention.java:390),
// x = (x*r)*w (SimdVectorOps.java:150-162), and the rotation x0*c - x1*s, x0*s + x1*c with
// separately rounded products (RoPE.java:145-170, SimdVectorOps.java:165-186).  The library
// is compiled with -ffp-contract=off so none of these is fused; fmaf is explicit where the
// attention math wants a fused multiply-add.
//
// Streaming: the device cache is head-major [kv_head][pos][D], so a split's K (and V) rows
// are one contiguous span.  LPR lanes share a row; lane j of a row group loads the 16-byte
// chunks j, j+LPR, ... of the row, so one wave-wide load instruction covers RPW = 64/LPR rows
// with LPR*16 contiguous bytes per row.  Scores are reduced across the LPR lanes of a row with
// DPP (quad_perm, row_half_mirror, row_mirror); each row group keeps its own online-softmax
// state (max, sum, output slice) in registers; groups and waves are merged once at the end
// through cross-lane shuffles and LDS.  Decode is HBM-bound (Hq/(2*Hkv) flop/byte), so no
// MFMA is used.
#pragma once

#include "llmp_internal.h"

namespace llmp {
namespace dk {

constexpr float kLog2e = 1.4426950408889634f;
// Finite "minus infinity" for running maxima, so that exp2(m_old - m_new) never sees
// (-inf) - (-inf).  Masked scores use a true -inf, which exp2 maps to 0.
constexpr float kNegBig = -1.0e30f;
// Lazy rescaling: a running max is only raised (and o, l rescaled) once some lane of the wave
// sees a score more than this many log2 units above it, so exp2(s - m) stays <= 2^8 and the
// rescale multiplies are skipped on most trips.  O/L is unchanged: both use the same max.
constexpr float kLazyMargin = 8.0f;


// DPP controls (CDNA3/CDNA4 ISA): quad_perm, row_half_mirror, row_mirror.
constexpr int kDppQuadXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppRowMirror = 0x140;      // lane i <- lane 15-i within each row of 16
constexpr int kDppRowHalfMirror = 0x141;  // lane i <- lane 7-i within each half row

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// One step of a cross-lane reduction over the lanes of equal residue mod OFF (OFF a power of
// two, 4..32), all in VGPRs: offsets 16 and 32 exchange whole rows / half-waves with the
// gfx950 permlane swaps (the pair's two values come back in both lanes, combined in the same
// order there); smaller offsets rotate the 16-lane row by OFF with DPP, which pairs lanes of
// the same residue, so steps OFF, 2*OFF, ..., 8 leave the residue class's total in every lane.
template <int OFF, bool MAX>
__device__ __forceinline__ float lane_step(float x) {
    static_assert(OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32, "offset 4, 8, 16 or 32");
    float a, b;
    if constexpr (OFF >= 16) {
        const unsigned u = __builtin_bit_cast(unsigned, x);
        const auto r = OFF == 32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                                 : __builtin_amdgcn_permlane16_swap(u, u, false, false);
        a = __builtin_bit_cast(float, (unsigned)r[0]);
        b = __builtin_bit_cast(float, (unsigned)r[1]);
    } else {
        a = x;
        b = dpp<0x120 + OFF>(x);  // row_ror:OFF
    }
    return MAX ? fmaxf(a, b) : a + b;
}

// Sum over the LPR consecutive lanes that share a row.  Every lane ends with the same value
// (each step adds the same two operands, in either order).
template <int LPR>
__device__ __forceinline__ float row_group_sum(float x) {
    static_assert(LPR == 4 || LPR == 8 || LPR == 16 || LPR == 32 || LPR == 64,
                  "rows are shared by 4 to 64 lanes");
    x = x + dpp<kDppQuadXor1>(x);
    x = x + dpp<kDppQuadXor2>(x);
    if constexpr (LPR >= 8) x = x + dpp<kDppRowHalfMirror>(x);
    if constexpr (LPR >= 16) x = x + dpp<kDppRowMirror>(x);
    if constexpr (LPR >= 32) x = lane_step<16, false>(x);
    if constexpr (LPR >= 64) x = lane_step<32, false>(x);
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Range exponents of the stored rows.  The multi-token kernels split cache rows into fp16
// hi/lo parts, which hold magnitudes below 65504; rows with larger values are scaled by 2^-E
// first.  E(x) = max(0, floor(log2|x|) - 14), from the biased exponent: 0 for |x| < 2^15, and
// |x| * 2^-E(x) < 2^15 for every finite x.  Every writer of cache rows raises the exponents
// of the KV head it stores to (range[2*kvh] for K, range[2*kvh + 1] for V), so they bound
// every row of the layer until the cache is cleared.  The atomics only run when a row holds
// such a value.
__device__ __forceinline__ unsigned abs_bits(float x) { return __float_as_uint(x) & 0x7FFFFFFFu; }
__device__ __forceinline__ int range_exp_of_bits(unsigned ab) {
    const int e = (int)(ab >> 23) - 141;
    return e > 0 ? e : 0;
}
__device__ __forceinline__ void note_range(int* range, int kvh, unsigned kbits, unsigned vbits) {
    const int ek = range_exp_of_bits(kbits), ev = range_exp_of_bits(vbits);
    if (ek > 0) atomicMax(range + 2 * kvh, ek);
    if (ev > 0) atomicMax(range + 2 * kvh + 1, ev);
}


// Final normalisation of one output element of query head hq from its merged (max M,
// sum L, unnormalised O) in the log2 domain: an attention sink (log2-domain logit) joins the
// max and the sum with no value (softmaxWithSink, Qwen3MoEInferenceEngine.java:562-575), then
// the optional output gate multiplies by sigmoid(gate) (Qwen35InferenceEngine.java:580-583).
__device__ __forceinline__ float finish_output(float M, float L, float O, const float* sinks,
                                               const float* gate, int hq, long long gate_idx) {
    if (sinks != nullptr) {
        const float sk = sinks[hq];
        const float Mn = fmaxf(M, sk);
        const float f = fast_exp2(M - Mn);
        O = O * f;
        L = __builtin_fmaf(L, f, fast_exp2(sk - Mn));
    }
    float r = O / L;
    if (gate != nullptr) {
        const float e = expf(-gate[gate_idx]);
        r = r * (1.0f / (1.0f + e));
    }
    return r;
}

typedef float native_f4 __attribute__((ext_vector_type(4)));

// 16-byte load; NT marks it non-temporal (streamed once, no reuse expected).
template <bool NT>
__device__ __forceinline__ float4 load4(const float4* p) {
    if constexpr (NT) {
        const native_f4 v = __builtin_nontemporal_load(reinterpret_cast<const native_f4*>(p));
        return make_float4(v.x, v.y, v.z, v.w);
    } else {
        return *p;
    }
}

// Lane layout of a K/V row.  fp32 rows: lane j of a row group holds the 16-byte chunks
// j, j+LPR, ... (LPR*16 contiguous bytes per wave-wide load).  Q8_0 rows (CONTIG): lane j
// holds the 16 contiguous quants 16j..16j+15, i.e. half of one 32-value scale block.
template <int D, int EPL, bool CONTIG = false>
struct Frag {
    static constexpr int LPR = D / EPL;   // lanes per row
    static constexpr int RPW = 64 / LPR;  // rows per wave-wide load
    static constexpr int C4 = EPL / 4;    // 16-byte fp32 chunks per lane per row
    // Dimension held by lane j (within its row group) at element e.
    static __device__ __forceinline__ int dim(int j, int e) {
        return CONTIG ? j * EPL + e : (e >> 2) * (LPR * 4) + j * 4 + (e & 3);
    }
};

typedef unsigned int native_u4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ uint4 load_u4(const uint4* p) {
    if constexpr (NT) {
        const native_u4 v = __builtin_nontemporal_load(reinterpret_cast<const native_u4*>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return *p;
    }
}

// 16 signed bytes -> floats.
__device__ __forceinline__ void unpack_q8(const uint4& w, float (&f)[16]) {
    const unsigned d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int b = 0; b < 4; ++b) f[4 * i + b] = (float)(int)(signed char)(d[i] >> (8 * b));
}

// Online-softmax update of one row group over U Q8_0 rows: s = scale_k * (q . quants_k),
// o += (p * scale_v) * quants_v (KVCache.dotK / saxpyV in Q8_0 mode, KVCache.java:187-210).
template <int D, int G, int U, bool LAZY = false>
__device__ __forceinline__ void accumulate_rows_q8(const float (&qr)[G][16],
                                                   const float (&kq)[U][16], const float (&ksc)[U],
                                                   const float (&vq)[U][16], const float (&vsc)[U],
                                                   const bool (&valid)[U], float (&m)[G],
                                                   float (&l)[G], float (&o)[G][16],
                                                   const DecodeArgs& a) {
    constexpr int LPR = D / 16;
    float s[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float acc = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; ++e) acc = __builtin_fmaf(qr[h][e], kq[u][e], acc);
            s[u][h] = row_group_sum<LPR>(acc * ksc[u]);
        }
    }
    if (a.softcap > 0.0f) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int h = 0; h < G; ++h) s[u][h] = a.softcap_log2e * tanhf(s[u][h] * a.inv_softcap);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float mx = m[h];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            s[u][h] = valid[u] ? s[u][h] : -__builtin_inff();
            mx = fmaxf(mx, s[u][h]);
        }
        float lsum = l[h];
        if (!LAZY || __any(mx > m[h] + kLazyMargin)) {
            const float alpha = fast_exp2(m[h] - mx);
            m[h] = mx;
            lsum = lsum * alpha;
#pragma unroll
            for (int e = 0; e < 16; ++e) o[h][e] = o[h][e] * alpha;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float p = fast_exp2(s[u][h] - m[h]);
            lsum = lsum + p;
            const float w = p * vsc[u];
#pragma unroll
            for (int e = 0; e < 16; ++e) o[h][e] = __builtin_fmaf(w, vq[u][e], o[h][e]);
        }
        l[h] = lsum;
    }
}

// Math.round(float): nearest int, ties toward +infinity (exact for |y| < 2^22).
__device__ __forceinline__ int round_half_up(float y) {
    float r = floorf(y);
    const float frac = y - r;
    if (frac >= 0.5f) r = r + 1.0f;
    return (int)r;
}

// Q8_0 quantisation (KVCache.quantizeBlocksScalar, KVCache.java:218-243; SimdQ8KvOps.quantize,
// SimdQ8KvOps.java:86-117): per 32-value block scale = maxAbs/127, and each value becomes
// clamp(r(x * (1/scale)), -128, 127), where r rounds half up, or truncates toward zero when
// `trunc` is set (the 8-lane SIMD contract).  A zero block has inverse scale 0.
__device__ __forceinline__ float q8_block_scale(const float* x) {
    float mx = 0.0f;
    for (int i = 0; i < 32; ++i) {
        const float v = x[i];
        const float av = v >= 0.0f ? v : -v;
        mx = av > mx ? av : mx;
    }
    return mx / 127.0f;
}
__device__ __forceinline__ float q8_inv_scale(float scale) {
    return scale != 0.0f ? 1.0f / scale : 0.0f;
}
__device__ __forceinline__ int q8_code(float x, float inv, bool trunc) {
    const float y = x * inv;
    int v = trunc ? (int)y : round_half_up(y);   // |y| <= 127.x: the cast is in range
    return v > 127 ? 127 : (v < -128 ? -128 : v);
}

// Q8_0 quantisation of one row of D fp32 values staged in LDS, by the whole workgroup;
// results in LDS (q: D bytes, sc: D/32 floats).
template <int D, int NTHR>
__device__ void quantize_row_lds(const float* x, signed char* q, float* sc, float* s_inv, int tid,
                                 bool trunc) {
    for (int b = tid; b < D / 32; b += NTHR) {
        const float scale = q8_block_scale(x + 32 * b);
        sc[b] = scale;
        s_inv[b] = q8_inv_scale(scale);
    }
    __syncthreads();
    for (int i = tid; i < D; i += NTHR) q[i] = (signed char)q8_code(x[i], s_inv[i / 32], trunc);
    __syncthreads();
}

// Online-softmax update of one row group with U rows: s = (q . K_t) in the log2 domain,
// masked rows get -inf; o and l are rescaled once per call.
template <int D, int G, int EPL, int U, bool LAZY = false>
__device__ __forceinline__ void accumulate_rows(const float (&qr)[G][EPL],
                                                const float4 (&kf)[U][EPL / 4],
                                                const float4 (&vf)[U][EPL / 4],
                                                const bool (&valid)[U], float (&m)[G],
                                                float (&l)[G], float (&o)[G][EPL],
                                                const DecodeArgs& a) {
    using F = Frag<D, EPL>;
    float s[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float acc = 0.0f;
#pragma unroll
            for (int c = 0; c < F::C4; ++c) {
                acc = __builtin_fmaf(qr[h][4 * c + 0], kf[u][c].x, acc);
                acc = __builtin_fmaf(qr[h][4 * c + 1], kf[u][c].y, acc);
                acc = __builtin_fmaf(qr[h][4 * c + 2], kf[u][c].z, acc);
                acc = __builtin_fmaf(qr[h][4 * c + 3], kf[u][c].w, acc);
            }
            s[u][h] = row_group_sum<F::LPR>(acc);
        }
    }
    if (a.softcap > 0.0f) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int h = 0; h < G; ++h) s[u][h] = a.softcap_log2e * tanhf(s[u][h] * a.inv_softcap);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float mx = m[h];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            s[u][h] = valid[u] ? s[u][h] : -__builtin_inff();
            mx = fmaxf(mx, s[u][h]);
        }
        float lsum = l[h];
        if (!LAZY || __any(mx > m[h] + kLazyMargin)) {
            const float alpha = fast_exp2(m[h] - mx);
            m[h] = mx;
            lsum = lsum * alpha;
#pragma unroll
            for (int e = 0; e < EPL; ++e) o[h][e] = o[h][e] * alpha;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float p = fast_exp2(s[u][h] - m[h]);
            lsum = lsum + p;
#pragma unroll
            for (int c = 0; c < F::C4; ++c) {
                o[h][4 * c + 0] = __builtin_fmaf(p, vf[u][c].x, o[h][4 * c + 0]);
                o[h][4 * c + 1] = __builtin_fmaf(p, vf[u][c].y, o[h][4 * c + 1]);
                o[h][4 * c + 2] = __builtin_fmaf(p, vf[u][c].z, o[h][4 * c + 2]);
                o[h][4 * c + 3] = __builtin_fmaf(p, vf[u][c].w, o[h][4 * c + 3]);
            }
        }
        l[h] = lsum;
    }
}

// Per-token prep parameters shared by the decode and prefill kernels.
struct HeadPrep {
    const float* qnw;      // QK-norm weights for query heads [D] or nullptr (no QK-norm)
    const float* knw;      // QK-norm weights for key heads [D]
    float eps;
    const float* cos_row;  // RoPE row of the token's position, or nullptr (NoPE)
    const float* sin_row;
    int half_rope;
    int rope_type;         // 0 NORMAL, 2 NEOX
};

// The same parameters with the weights and the RoPE row staged in LDS (pointers in the LDS
// address space, so the prep reads them with LDS loads; a null pointer means "absent").
typedef __attribute__((address_space(3))) const float* lds_cptr;
struct HeadPrepLds {
    lds_cptr qnw;
    lds_cptr knw;
    float eps;
    lds_cptr cos_row;
    lds_cptr sin_row;
    int half_rope;
    int rope_type;
};

__device__ __forceinline__ HeadPrep head_prep(const DecodeArgs& a, int pos) {
    const long long row = (long long)pos * a.half_rope;
    return HeadPrep{a.qnw, a.knw, a.eps, a.cos_t ? a.cos_t + row : nullptr,
                    a.sin_t ? a.sin_t + row : nullptr, a.half_rope, a.rope_type};
}

// Position of this step: the host value, or the device word (read once per thread; all
// threads read the same value).
__device__ __forceinline__ int step_position(const DecodeArgs& a) {
    return a.d_pos != nullptr ? *a.d_pos : a.pos;
}

// Kernel arguments are read with scalar loads at their first use, and a field first used
// after a branch (the position checks, the split's early exit) waits for another round trip
// to the argument segment: three rounds, ~1.3 us per workgroup, measured at the Llama-3.2-3B
// shape.  Naming every field the prologue reads at entry puts them in one round.
__device__ __forceinline__ void load_args_now(const DecodeArgs& a) {
    asm volatile("" ::"s"(a.q), "s"(a.k), "s"(a.v), "s"(a.kc), "s"(a.vc), "s"(a.kq), "s"(a.ks),
                 "s"(a.vq), "s"(a.vs), "s"(a.cos_t), "s"(a.sin_t));
    asm volatile("" ::"s"(a.qnw), "s"(a.knw), "s"(a.sinks), "s"(a.gate), "s"(a.out),
                 "s"(a.part_o), "s"(a.part_ml), "s"(a.d_pos), "s"(a.head_stride));
    asm volatile("" ::"s"(a.pos), "s"(a.max_seq), "s"(a.window), "s"(a.splits), "s"(a.half_rope),
                 "s"(a.rope_type), "s"(a.q8_trunc), "s"(a.norm_seq), "s"(a.v_norm),
                 "s"(a.no_append), "s"(a.eps), "s"(a.qk_scale));
    asm volatile("" ::"s"(a.softcap), "s"(a.softcap_log2e), "s"(a.inv_softcap), "s"(a.range),
                 "s"(a.kv_rep));
}
// The merge arguments too (the kernel instances that can merge their splits).
__device__ __forceinline__ void load_merge_args_now(const DecodeArgs& a) {
    asm volatile("" ::"s"(a.done), "s"(a.fused));
}

// ---- merge of the splits, in the split kernel ------------------------------------------------
// A call with S > 1 splits leaves every workgroup's partial state (unnormalised o, max, sum)
// of its G query heads in part_o / part_ml.  With DecodeArgs::fused the workgroup that
// finishes last per virtual KV head merges them and writes the output (no second launch); the
// host fuses only where that merge is one round of loads and measured faster than
// decode_reduce_kernel's launch (decode_fused_merge): with more splits per thread group the
// last workgroup's rounds of loads from the coherence point cost more (C3 at 4k, 16 splits
// per group: 13.2 -> 15.5 us per layer-call; at 32k, 24 splits of 8-wave workgroups in 5
// groups: 45.5 -> 45.0 us).  The workgroups of a KV head
// may run on different XCDs, each with its own L2, so the partials move through the device's
// coherence point: they are written and read with agent-scope relaxed atomic accesses (stores
// and loads that bypass the non-coherent L2 state, 4 or 8 bytes each).  A workgroup waits for
// its partial stores to complete before it counts itself done on the KV head's counter; the
// one that brings the count to S has observed every other workgroup's count, issued after
// their stores completed, so its loads see all partials.  It re-arms the counter for the next
// call.  (A device-scope fence per workgroup instead would write back the whole L2 of each
// workgroup's XCD: measured 13 -> 35 us per C3 layer-call at 4k.)
//
// The merge is the log-sum-exp combine of decode_reduce_kernel: per float4 column of the G
// heads, the splits are taken in NP groups of threads (group p: splits p, p + NP, ..., the
// first kMergeBatch of them loaded at once, any further merged online), and the groups' states
// are merged through LDS.  `scratch`: LDS of at least combine_scratch_floats<NTHR>() floats that
// the caller no longer reads.
constexpr int kMergeBatch = 8;
template <int NTHR>
constexpr int combine_scratch_floats() { return 6 * NTHR; }   // float4 o + float2 (m, l) per thread

__device__ __forceinline__ void store_partial(float* p, float v, int fused) {
    if (fused)
        __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *p = v;
}
__device__ __forceinline__ float2 load_partial2(const float* p) {   // 8-byte aligned
    const unsigned long long u = __hip_atomic_load(reinterpret_cast<const unsigned long long*>(p),
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __builtin_bit_cast(float2, u);
}

template <int D, int G, int NTHR>
__device__ __forceinline__ void combine_if_last(const DecodeArgs& a, int vkh, int S, int tid,
                                                float* scratch) {
    __shared__ int s_last;
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this thread's partial stores completed
    __syncthreads();
    if (tid == 0) {
        s_last = __hip_atomic_fetch_add(a.done + vkh, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
        if (s_last) __hip_atomic_store(a.done + vkh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;
    constexpr int NC = G * D / 4;                      // float4 columns of the G heads
    constexpr int NP = NTHR >= NC ? NTHR / NC : 1;     // split groups
    const int h0 = vkh * G;
    float4* s_o = reinterpret_cast<float4*>(scratch);                 // [NP][NC]
    float2* s_ml = reinterpret_cast<float2*>(scratch + 4 * NTHR);     // [NP][NC]
    // One column c over the splits p, p + NP, ...: (m, l, o).
    auto merge_col = [&](int c, int p, float& m, float& l, float4& o) {
        const int h = c / (D / 4), c4 = c - h * (D / 4);
        const long long slot0 = (long long)vkh * S * G + h;   // split j: slot0 + j*G
        m = kNegBig;
        l = 0.0f;
        o = make_float4(0.f, 0.f, 0.f, 0.f);
        float2 mlj[kMergeBatch], oa[kMergeBatch], ob[kMergeBatch];
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
            const int jj = p + u * NP;
            const long long slot = slot0 + (long long)(jj < S ? jj : 0) * G;
            mlj[u] = load_partial2(a.part_ml + 2 * slot);
            oa[u] = load_partial2(a.part_o + slot * D + 4 * c4);
            ob[u] = load_partial2(a.part_o + slot * D + 4 * c4 + 2);
        }
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) m = fmaxf(m, p + u * NP < S ? mlj[u].x : kNegBig);
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
            const float sj = p + u * NP < S ? fast_exp2(mlj[u].x - m) : 0.0f;
            l = __builtin_fmaf(mlj[u].y, sj, l);
            o.x = __builtin_fmaf(oa[u].x, sj, o.x);
            o.y = __builtin_fmaf(oa[u].y, sj, o.y);
            o.z = __builtin_fmaf(ob[u].x, sj, o.z);
            o.w = __builtin_fmaf(ob[u].y, sj, o.w);
        }
        for (int jj = p + kMergeBatch * NP; jj < S; jj += NP) {
            const long long slot = slot0 + (long long)jj * G;
            const float2 mq = load_partial2(a.part_ml + 2 * slot);
            const float2 qa = load_partial2(a.part_o + slot * D + 4 * c4);
            const float2 qb = load_partial2(a.part_o + slot * D + 4 * c4 + 2);
            const float mn = fmaxf(m, mq.x);
            const float so = fast_exp2(m - mn), sq = fast_exp2(mq.x - mn);
            l = __builtin_fmaf(l, so, mq.y * sq);
            o.x = __builtin_fmaf(o.x, so, qa.x * sq);
            o.y = __builtin_fmaf(o.y, so, qa.y * sq);
            o.z = __builtin_fmaf(o.z, so, qb.x * sq);
            o.w = __builtin_fmaf(o.w, so, qb.y * sq);
            m = mn;
        }
    };
    auto store_col = [&](int c, float M, float L, const float4& O) {
        const int h = c / (D / 4), d0 = 4 * (c - h * (D / 4));
        const long long row = (long long)(h0 + h) * D + d0;
        float4 r;
        r.x = finish_output(M, L, O.x, a.sinks, a.gate, h0 + h, row);
        r.y = finish_output(M, L, O.y, a.sinks, a.gate, h0 + h, row + 1);
        r.z = finish_output(M, L, O.z, a.sinks, a.gate, h0 + h, row + 2);
        r.w = finish_output(M, L, O.w, a.sinks, a.gate, h0 + h, row + 3);
        reinterpret_cast<float4*>(a.out + row)[0] = r;
    };
    if constexpr (NP == 1) {
        for (int c = tid; c < NC; c += NTHR) {
            float m, l;
            float4 o;
            merge_col(c, 0, m, l, o);
            store_col(c, m, l, o);
        }
    } else {
        const int c = tid % NC, p = tid / NC;
        const bool act = p < NP;
        float m, l;
        float4 o;
        merge_col(c, act ? p : 0, m, l, o);
        if (act) {
            s_o[p * NC + c] = o;
            s_ml[p * NC + c] = make_float2(m, l);
        }
        __syncthreads();
        if (p == 0) {
            float M = s_ml[c].x;
#pragma unroll
            for (int q = 1; q < NP; ++q) M = fmaxf(M, s_ml[q * NC + c].x);
            float L = 0.0f;
            float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int q = 0; q < NP; ++q) {
                const float sc = fast_exp2(s_ml[q * NC + c].x - M);
                L = __builtin_fmaf(s_ml[q * NC + c].y, sc, L);
                const float4 x = s_o[q * NC + c];
                O.x = __builtin_fmaf(x.x, sc, O.x);
                O.y = __builtin_fmaf(x.y, sc, O.y);
                O.z = __builtin_fmaf(x.z, sc, O.z);
                O.w = __builtin_fmaf(x.w, sc, O.w);
            }
            store_col(c, M, L, O);
        }
    }
}


// 1/rms of D values in the order of RMSNorm.apply with offsets (RMSNorm.java:24-35, the
// Gemma 4 engine's QK-norm and V-norm): one thread sums the squares sequentially, unfused,
// then r = 1/(float)sqrt(ss/D + eps).
template <int D>
__device__ __forceinline__ float seq_rms_inv(const float* x, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < D; ++i) ss = ss + x[i] * x[i];
    float v = ss / (float)D;
    v = v + eps;
    return 1.0f / (float)__builtin_sqrt((double)v);
}

// Exact prep of `nh` heads staged in LDS (x: nh*D floats): QK-norm with weights p.qnw for
// heads < n_w0 and p.knw for the others, then RoPE.  The sum of squares follows
// SimdVectorOps.dot's 8-lane FMA order, or with `seq` RMSNorm.apply's sequential one.  Must
// be called by the whole workgroup (NTHR threads).
//
// Every phase loads its LDS operands before it computes: a chain that waits for each load in
// turn costs an LDS round trip per step (head_dim 256: 32 dependent reads per partial sum).
// The scaling and the rotation run as one pass over (head, pair) slots: slot i < half_rope is
// the rotated pair (2i, 2i+1) (NORMAL) or (i, half_rope + i) (NEOX); every other slot is the
// unrotated pair (2i, 2i+1), so each element is read and written once.  The float steps are
// those of the CPU path: (x * r) * w, then x0*c - x1*s and x0*s + x1*c.
template <int D, int NTHR, class HP = HeadPrep>
__device__ void prep_heads_lds(float* x, int nh, int n_w0, float* s_acc, float* s_r,
                               const HP& p, int tid, bool seq = false) {
    const bool norm = p.qnw != nullptr;
    const bool rope = p.cos_row != nullptr;
    if (norm && seq) {
        for (int t = tid; t < nh; t += NTHR) s_r[t] = seq_rms_inv<D>(x + t * D, p.eps);
        __syncthreads();
    } else if (norm) {
        constexpr int NV = D / 8;                       // values per partial sum
        constexpr int CH = NV % 8 == 0 ? 8 : NV;        // loaded ahead of their FMAs
        for (int t = tid; t < nh * 8; t += NTHR) {
            const int hh = t >> 3, ln = t & 7;
            const float* xh = x + hh * D + ln;
            float acc = 0.0f;
#pragma unroll
            for (int k0 = 0; k0 < NV; k0 += CH) {
                float v[CH];
#pragma unroll
                for (int k = 0; k < CH; ++k) v[k] = xh[8 * (k0 + k)];
#pragma unroll
                for (int k = 0; k < CH; ++k) acc = __builtin_fmaf(v[k], v[k], acc);
            }
            s_acc[t] = acc;
        }
        __syncthreads();
        for (int t = tid; t < nh; t += NTHR) {
            const float* ac = s_acc + t * 8;
            float ss = ac[0];
#pragma unroll
            for (int ln = 1; ln < 8; ++ln) ss = ss + ac[ln];
            float v = ss / (float)D;
            v = v + p.eps;
            const float r = (float)__builtin_sqrt((double)v);
            s_r[t] = 1.0f / r;
        }
        __syncthreads();
    }
    if (!norm && !rope) return;
    constexpr int HALF = D / 2;
    constexpr int SL = 4;   // slots per thread per round, loaded together
    const int n_slots = nh * HALF;
    const int half = rope ? p.half_rope : 0;
    const bool neox = p.rope_type != 0;
    for (int base = tid; base < n_slots; base += SL * NTHR) {
        float v0[SL], v1[SL], w0[SL], w1[SL], r[SL], c[SL], sn[SL];
        int o0[SL], o1[SL];
#pragma unroll
        for (int k = 0; k < SL; ++k) {
            // a slot past the end re-reads this thread's own first slot (its result is dropped),
            // so no thread reads an element another thread rewrites in this round
            const int slot = base + k * NTHR < n_slots ? base + k * NTHR : base;
            const int hh = slot / HALF, i = slot - hh * HALF;
            const bool rot = i < half;
            const int i0 = (rot && neox) ? i : 2 * i;
            const int i1 = (rot && neox) ? half + i : 2 * i + 1;
            o0[k] = hh * D + i0;
            o1[k] = hh * D + i1;
            v0[k] = x[o0[k]];
            v1[k] = x[o1[k]];
            if (norm) {
                const auto w = (hh < n_w0) ? p.qnw : p.knw;
                r[k] = s_r[hh];
                w0[k] = w[i0];
                w1[k] = w[i1];
            }
            if (rope) {
                const int ic = rot ? i : 0;
                c[k] = p.cos_row[ic];
                sn[k] = p.sin_row[ic];
            }
        }
#pragma unroll
        for (int k = 0; k < SL; ++k) {
            if (base + k * NTHR >= n_slots) break;
            const int i = (base + k * NTHR) % HALF;
            float a0 = v0[k], a1 = v1[k];
            if (norm) {
                const float xs0 = a0 * r[k], xs1 = a1 * r[k];
                a0 = xs0 * w0[k];
                a1 = xs1 * w1[k];
            }
            if (i < half) {
                const float t0 = a0 * c[k], t1 = a1 * sn[k], t2 = a0 * sn[k], t3 = a1 * c[k];
                a0 = t0 - t1;
                a1 = t2 + t3;
            }
            x[o0[k]] = a0;
            x[o1[k]] = a1;
        }
    }
    __syncthreads();
}

// Rotation of the lane's own q slice in registers (no QK-norm; NORMAL pairs sit inside one
// 16-byte chunk, NEOX pairs (i, i+D/2) in chunks c and c+C4/2 of the same lane).  The lane's
// EPL/2 cos/sin factors are loaded first (rope_lane_factors) so that their loads are in flight
// with the other prologue loads, then applied (rope_registers).
template <int D, int EPL, bool CONTIG = false>
__device__ __forceinline__ void rope_lane_factors(float (&cs)[EPL / 2], float (&sn)[EPL / 2],
                                                  int j, const HeadPrep& a) {
    using F = Frag<D, EPL, CONTIG>;
    const int half = a.half_rope;
    if (a.rope_type == 0) {
#pragma unroll
        for (int c = 0; c < F::C4; ++c)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int i = F::dim(j, 4 * c + 2 * p) / 2;
                const int ii = i < half ? i : 0;   // pairs at or beyond half_rope keep their values
                cs[2 * c + p] = a.cos_row[ii];
                sn[2 * c + p] = a.sin_row[ii];
            }
    } else if constexpr (!CONTIG) {
#pragma unroll
        for (int c = 0; c < F::C4 / 2; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = c * F::LPR * 4 + j * 4 + e;   // < D/2 = half
                cs[4 * c + e] = a.cos_row[i];
                sn[4 * c + e] = a.sin_row[i];
            }
    }
}

template <int D, int G, int EPL, bool CONTIG = false>
__device__ __forceinline__ void rope_registers(float (&qr)[G][EPL], int j, const float (&cs)[EPL / 2],
                                               const float (&sn)[EPL / 2], const HeadPrep& a) {
    using F = Frag<D, EPL, CONTIG>;
    const int half = a.half_rope;
    if (a.rope_type == 0) {
#pragma unroll
        for (int c = 0; c < F::C4; ++c) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const bool rot = F::dim(j, 4 * c + 2 * p) / 2 < half;
                const float cv = cs[2 * c + p], sv = sn[2 * c + p];
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    const float v0 = qr[h][4 * c + 2 * p], v1 = qr[h][4 * c + 2 * p + 1];
                    const float t0 = v0 * cv, t1 = v1 * sv, t2 = v0 * sv, t3 = v1 * cv;
                    const float r0 = t0 - t1, r1 = t2 + t3;
                    qr[h][4 * c + 2 * p] = rot ? r0 : v0;
                    qr[h][4 * c + 2 * p + 1] = rot ? r1 : v1;
                }
            }
        }
    } else if constexpr (!CONTIG) {  // NEOX, fp32 layout: dims i, i + D/2 in chunks c, c + C4/2
#pragma unroll
        for (int c = 0; c < F::C4 / 2; ++c) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float cv = cs[4 * c + e], sv = sn[4 * c + e];
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    const float v0 = qr[h][4 * c + e], v1 = qr[h][4 * (c + F::C4 / 2) + e];
                    const float t0 = v0 * cv, t1 = v1 * sv, t2 = v0 * sv, t3 = v1 * cv;
                    qr[h][4 * c + e] = t0 - t1;
                    qr[h][4 * (c + F::C4 / 2) + e] = t2 + t3;
                }
            }
        }
    }
}

// The new token's K and V rows of KV head kvh, staged for the append by the whole workgroup:
// k (sk) exactly QK-normed and rotated like the CPU path, v (sv) V-normed when the layer asks
// for it (Gemma 4's weightless V-norm: its sequential sum runs on another wave than the
// K-norm's thread 0, and is applied after the K prep's barriers).
template <int D, int NTHR>
__device__ void stage_new_row(const DecodeArgs& a, int kvh, float* sk, float* sv, float* s_acc,
                              float* s_r, float* s_vr, const HeadPrep& hp, int tid) {
    for (int i = tid; i < D; i += NTHR) {
        sk[i] = a.k[kvh * D + i];
        sv[i] = a.v[kvh * D + i];
    }
    __syncthreads();
    if (a.v_norm != 0 && tid == (NTHR > 64 ? 64 : 0)) *s_vr = seq_rms_inv<D>(sv, a.eps);
    prep_heads_lds<D, NTHR>(sk, 1, 0, s_acc, s_r, hp, tid, a.norm_seq != 0);
    if (a.v_norm != 0) {
        __syncthreads();
        for (int i = tid; i < D; i += NTHR) sv[i] = sv[i] * *s_vr;
        __syncthreads();
    }
}

// Q8_0 append of the staged row pos (KVCache.storeK/storeV in Q8_0 mode): quantised into LDS
// (kq/ks, vq/vs) and written to the cache.
// store: false for the workgroups of a KV head's further virtual heads (DecodeArgs::kv_rep),
// which quantise the row for their own use and leave the cache write to the first one.
template <int D, int NTHR>
__device__ void append_row_q8(const DecodeArgs& a, int kvh, int pos, const float* sk,
                              const float* sv, signed char* kq, float* ks, signed char* vq,
                              float* vs, float* s_inv, int tid, bool store) {
    quantize_row_lds<D, NTHR>(sk, kq, ks, s_inv, tid, a.q8_trunc != 0);
    quantize_row_lds<D, NTHR>(sv, vq, vs, s_inv, tid, a.q8_trunc != 0);
    if (!store) return;
    signed char* kqp = a.kq + (long long)kvh * a.head_stride + (long long)pos * D;
    signed char* vqp = a.vq + (long long)kvh * a.head_stride + (long long)pos * D;
    float* ksp = a.ks + (long long)kvh * (a.head_stride / 32) + (long long)pos * (D / 32);
    float* vsp = a.vs + (long long)kvh * (a.head_stride / 32) + (long long)pos * (D / 32);
    unsigned kb = 0, vb = 0;   // the dequantised values stay within the fp32 rows' range
    for (int i = tid; i < D; i += NTHR) {
        kqp[i] = kq[i];
        vqp[i] = vq[i];
        kb = max(kb, abs_bits(sk[i]));
        vb = max(vb, abs_bits(sv[i]));
    }
    note_range(a.range, kvh, kb, vb);
    for (int b = tid; b < D / 32; b += NTHR) {
        ksp[b] = ks[b];
        vsp[b] = vs[b];
    }
}

// Cached rows of one loop trip of a lane group: rows base + u*RPW + grp, u < U (masked past
// cache_end, with the address clamped into the cache), as 16-byte fp32 chunks, or as 16 quants
// and their block scale (Q8_0).
template <int D, int EPL, int U, bool Q8>
struct TripRows {
    static constexpr int C4 = EPL / 4;
    float4 k[Q8 ? 1 : U][C4], v[Q8 ? 1 : U][C4];
    uint4 kw[Q8 ? U : 1], vw[Q8 ? U : 1];
    float ksc[Q8 ? U : 1], vsc[Q8 ? U : 1];
    bool valid[U];
};

template <int D, int EPL, int U, bool NT, bool Q8>
__device__ __forceinline__ void load_trip(TripRows<D, EPL, U, Q8>& r, const DecodeArgs& a,
                                          int kvh, int base, int cache_end, int grp, int j) {
    using F = Frag<D, EPL, Q8>;
    const int last = cache_end > 0 ? cache_end - 1 : 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int t = base + u * F::RPW + grp;
        r.valid[u] = t < cache_end;
        const long long tt = r.valid[u] ? t : last;
        if constexpr (!Q8) {
            const float4* kp =
                reinterpret_cast<const float4*>(a.kc + (long long)kvh * a.head_stride + tt * D) + j;
            const float4* vp =
                reinterpret_cast<const float4*>(a.vc + (long long)kvh * a.head_stride + tt * D) + j;
#pragma unroll
            for (int c = 0; c < F::C4; ++c) r.k[u][c] = load4<NT>(kp + c * F::LPR);
#pragma unroll
            for (int c = 0; c < F::C4; ++c) r.v[u][c] = load4<NT>(vp + c * F::LPR);
        } else {
            const long long h = (long long)kvh * a.head_stride, hs = (long long)kvh * (a.head_stride / 32);
            r.kw[u] = load_u4<NT>(reinterpret_cast<const uint4*>(a.kq + h + tt * D) + j);
            r.vw[u] = load_u4<NT>(reinterpret_cast<const uint4*>(a.vq + h + tt * D) + j);
            r.ksc[u] = a.ks[hs + tt * (D / 32) + (j >> 1)];
            r.vsc[u] = a.vs[hs + tt * (D / 32) + (j >> 1)];
        }
    }
}

template <int D, int G, int EPL, int U, bool Q8, bool LAZY>
__device__ __forceinline__ void consume_trip(const TripRows<D, EPL, U, Q8>& r,
                                             const float (&qr)[G][EPL], float (&m)[G],
                                             float (&l)[G], float (&o)[G][EPL],
                                             const DecodeArgs& a) {
    if constexpr (!Q8) {
        accumulate_rows<D, G, EPL, U, LAZY>(qr, r.k, r.v, r.valid, m, l, o, a);
    } else {
        float kq[U][16], vq[U][16];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            unpack_q8(r.kw[u], kq[u]);
            unpack_q8(r.vw[u], vq[u]);
        }
        accumulate_rows_q8<D, G, U, LAZY>(qr, kq, r.ksc, vq, r.vsc, r.valid, m, l, o, a);
    }
}

template <int D, int G, int EPL, int U, int WAVES, bool NT, bool Q8 = false, bool LAZY = Q8>
__global__ __launch_bounds__(WAVES * 64) void decode_split_kernel(DecodeArgs a) {
    static_assert(!Q8 || EPL == 16, "Q8_0 rows are read 16 quants per lane");
    using F = Frag<D, EPL, Q8>;
    using Trip = TripRows<D, EPL, U, Q8>;
    constexpr int NTHR = WAVES * 64;
    constexpr int LPR = F::LPR, RPW = F::RPW, C4 = F::C4;
    constexpr int ROWS_WAVE = U * RPW;
    constexpr int ROWS_BLOCK = WAVES * ROWS_WAVE;
    constexpr int WPT = (D + NTHR - 1) / NTHR;   // per-thread elements of a D-vector

    // s_x: G query heads then the group's K head (post norm and RoPE).
    __shared__ float s_x[(G + 1) * D];
    __shared__ float s_v[D];
    __shared__ float s_acc[(G + 1) * 8];
    __shared__ float s_r[G + 1];
    __shared__ float s_cs[D / 2], s_sn[D / 2], s_qw[D], s_kw[D];
    __shared__ float s_vr;
    __shared__ __align__(16) signed char s_kq[Q8 ? D : 16], s_vq[Q8 ? D : 16];
    __shared__ float s_ks[D / 32], s_vs[D / 32], s_inv[D / 32];
    // Merge of the workgroup's partial softmax states (section 5): with LDS_MERGE every row
    // group of every wave leaves its raw (m, l, o) in LDS (NPART partials); otherwise the row
    // groups of a wave are merged in VGPRs first (WAVES partials).
    // The LDS budget for it is 32 KB, or 64 KB for head_dim >= 256 at 4 waves, where the VGPR
    // count (G * EPL values of o per lane) already allows no more than 2 waves per SIMD
    // (Gemma-3 at 8k: -1 to -2 % per layer-call against the lane-exchange merge).
    constexpr int NPART_LDS = WAVES * RPW;
    constexpr bool LDS_MERGE = NPART_LDS * G * D * 4 <= (D >= 256 && WAVES == 4 ? 65536 : 32768);
    constexpr int NPART = LDS_MERGE ? NPART_LDS : WAVES;
    // The weight pass of the LDS merge gives one thread to each (partial, head) pair.
    static_assert(!LDS_MERGE || NPART * G <= NTHR, "LDS merge needs a thread per partial and head");
    __shared__ float s_m[NPART * G];
    __shared__ float s_l[NPART * G];
    __shared__ float s_w[LDS_MERGE ? NPART * G : 1];
    __shared__ float s_ML[LDS_MERGE ? 2 * G : 1];
    __shared__ float s_o[NPART * G * D];
    // The merge of the splits (combine_if_last), compiled into the 2- and 8-wave instances only
    // (decode_fused_merge never picks it for 4-wave workgroups, whose code stays without it),
    // reuses s_o when it is large enough.
    constexpr bool CAN_FUSE = WAVES != 4;
    constexpr bool CMB_ALIAS = NPART * G * D >= combine_scratch_floats<NTHR>();
    __shared__ float s_cmb[(CMB_ALIAS || !CAN_FUSE) ? 1 : combine_scratch_floats<NTHR>()];

    const int tid = threadIdx.x;
    const int split = blockIdx.x;
    // Grid y runs over virtual KV heads: kv_rep of them share each cached KV head (groups of
    // more than 8 query heads run as kv_rep groups of G), so the query heads, the partials and
    // the grid use vkh, the cache uses kvh, and the first virtual head alone appends.
    const int vkh = blockIdx.y;
    const int kvh = vkh / a.kv_rep;
    const bool store = vkh == kvh * a.kv_rep;
    const int h0 = vkh * G;
    // Step plan from the position (host value or device word).  A device position outside
    // the cache leaves everything untouched; splits beyond the rows of this step exit.
    load_args_now(a);
    if constexpr (CAN_FUSE) load_merge_args_now(a);
    const int pos = step_position(a);
    if (pos < 0 || pos >= a.max_seq) return;
    const StepPlan sp = plan_step(pos, a.window, a.splits);
    if (split >= sp.splits) return;
    const HeadPrep hp = head_prep(a, pos);
    const int row_begin = sp.start + split * sp.rows_per_split;
    const int row_end = min(row_begin + sp.rows_per_split, pos + 1);
    // The split holding row `pos` appends it, unless the layer shares another layer's KV
    // (row `pos` is then already cached and streamed like the others).
    const bool has_pos = (row_end == pos + 1) && a.no_append == 0;
    const int cache_end = has_pos ? pos : row_end;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int grp = lane / LPR, j = lane - grp * LPR;

    // 1. Every load of the prologue is issued before any of them is waited for, then the
    //    wave's first trip of cached rows, so the prep's memory latency overlaps the stream's:
    //    the lane's q slice (in the streaming layout), its RoPE factors (register path), the
    //    RoPE row and norm weights for the LDS prep, and the new k/v row (appending split).
    //    Without QK-norm and with RoPE pairs inside a lane, q is rotated in registers;
    //    otherwise it is prepared in LDS with the exact QK-norm order.
    const bool rope = a.cos_t != nullptr, qkn = a.qnw != nullptr;
    // NEOX pairs (i, i + D/2) share a lane only when the lane's chunks split evenly in halves
    const bool pairs_in_lane = a.rope_type == 0 || (!Q8 && C4 % 2 == 0 && 2 * a.half_rope == D);
    const bool reg_prologue = !qkn && (!rope || pairs_in_lane);
    const bool lds_prep = !reg_prologue || has_pos;
    float qr[G][EPL];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int c = 0; c < C4; ++c) {
            const float4 x = *reinterpret_cast<const float4*>(a.q + (h0 + h) * D + F::dim(j, 4 * c));
            qr[h][4 * c + 0] = x.x;
            qr[h][4 * c + 1] = x.y;
            qr[h][4 * c + 2] = x.z;
            qr[h][4 * c + 3] = x.w;
        }
    float rcs[EPL / 2], rsn[EPL / 2];
    if (reg_prologue && rope) rope_lane_factors<D, EPL, Q8>(rcs, rsn, j, hp);
    float cw[WPT], sw[WPT], qw[WPT], kw[WPT], kn[WPT], vn[WPT];
    if (lds_prep) {
#pragma unroll
        for (int r = 0; r < WPT; ++r) {
            const int i = tid + r * NTHR;
            const int ic = rope ? min(i, max(a.half_rope - 1, 0)) : 0;
            cw[r] = rope ? hp.cos_row[ic] : 0.0f;
            sw[r] = rope ? hp.sin_row[ic] : 0.0f;
            qw[r] = qkn ? a.qnw[min(i, D - 1)] : 0.0f;
            kw[r] = qkn ? a.knw[min(i, D - 1)] : 0.0f;
        }
    }
    if (has_pos) {
#pragma unroll
        for (int r = 0; r < WPT; ++r) {
            const int i = min(tid + r * NTHR, D - 1);
            kn[r] = a.k[kvh * D + i];
            vn[r] = a.v[kvh * D + i];
        }
    }
    const int first = row_begin + wave * ROWS_WAVE;
    const int ntrips = first < cache_end ? (cache_end - first + ROWS_BLOCK - 1) / ROWS_BLOCK : 0;
    Trip ta, tb;
    load_trip<D, EPL, U, NT, Q8>(ta, a, kvh, first, cache_end, grp, j);

    // 2. The LDS prep (one barrier for all staged inputs): q heads (LDS path) and the new K
    //    head (appending split) normalised and rotated in the CPU path's float step order, the
    //    V row V-normed when asked; then the append itself, before the stream.
    if (lds_prep) {
        if (!reg_prologue && wave == 0 && grp == 0) {
#pragma unroll
            for (int h = 0; h < G; ++h)
#pragma unroll
                for (int e = 0; e < EPL; ++e) s_x[h * D + F::dim(j, e)] = qr[h][e];
        }
#pragma unroll
        for (int r = 0; r < WPT; ++r) {
            const int i = tid + r * NTHR;
            if (i < a.half_rope) {
                s_cs[i] = cw[r];
                s_sn[i] = sw[r];
            }
            if (i < D) {
                s_qw[i] = qw[r];
                s_kw[i] = kw[r];
                if (has_pos) {
                    s_x[G * D + i] = kn[r];
                    s_v[i] = vn[r];
                }
            }
        }
        __syncthreads();
        const lds_cptr lnull = nullptr;
        const HeadPrepLds hl{qkn ? (lds_cptr)s_qw : lnull, qkn ? (lds_cptr)s_kw : lnull, a.eps,
                             rope ? (lds_cptr)s_cs : lnull, rope ? (lds_cptr)s_sn : lnull,
                             a.half_rope, a.rope_type};
        // Gemma 4's weightless V-norm: its serial sum runs on another wave than the K-norm's.
        if (has_pos && a.v_norm != 0 && tid == (NTHR > 64 ? 64 : 0)) s_vr = seq_rms_inv<D>(s_v, a.eps);
        const bool seq = a.norm_seq != 0;
        if (!reg_prologue && has_pos && !seq) {
            prep_heads_lds<D, NTHR>(s_x, G + 1, G, s_acc, s_r, hl, tid);
        } else {
            if (!reg_prologue) prep_heads_lds<D, NTHR>(s_x, G, G, s_acc, s_r, hl, tid);
            if (has_pos) prep_heads_lds<D, NTHR>(s_x + G * D, 1, 0, s_acc, s_r, hl, tid, seq);
        }
        if (has_pos) {
            if (a.v_norm != 0) {
                __syncthreads();
                for (int i = tid; i < D; i += NTHR) s_v[i] = s_v[i] * s_vr;
                __syncthreads();
            }
            // KVCache.storeK/storeV: the exact fp32 rows, or their Q8_0 quantisation.
            if constexpr (!Q8) {
              if (store) {
                float* kplane = a.kc + (long long)kvh * a.head_stride + (long long)pos * D;
                float* vplane = a.vc + (long long)kvh * a.head_stride + (long long)pos * D;
                unsigned kb = 0, vb = 0;
                for (int i = tid; i < D; i += NTHR) {
                    const float kx = s_x[G * D + i], vx = s_v[i];
                    kplane[i] = kx;
                    vplane[i] = vx;
                    kb = max(kb, abs_bits(kx));
                    vb = max(vb, abs_bits(vx));
                }
                note_range(a.range, kvh, kb, vb);
              }
            } else {
                append_row_q8<D, NTHR>(a, kvh, pos, s_x + G * D, s_v, s_kq, s_ks, s_vq, s_vs, s_inv, tid,
                                       store);
            }
        }
        if (!reg_prologue) {
#pragma unroll
            for (int h = 0; h < G; ++h)
#pragma unroll
                for (int e = 0; e < EPL; ++e) qr[h][e] = s_x[h * D + F::dim(j, e)];
        }
    }
    if (reg_prologue && rope) rope_registers<D, G, EPL, Q8>(qr, j, rcs, rsn, hp);
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < EPL; ++e) qr[h][e] = qr[h][e] * a.qk_scale;

    float m[G], l[G], o[G][EPL];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m[h] = kNegBig;
        l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) o[h][e] = 0.0f;
    }

    // 3. Stream the cached rows [row_begin, cache_end), one trip prefetched in registers.  The
    //    trips run in pairs with one exit: a branch between the two halves would join the loop
    //    head with the second buffer's loads in flight, and the wait placed there would drain
    //    the prefetch on every trip.  (The last pair's refill reads masked, clamped rows.
    //    Peeling the last trips to skip it raised the register count by up to 40 VGPRs and cost
    //    an occupancy step at most shapes; pointing its rows at the cache-resident query vector
    //    measured 0.2 us faster at 4k but 0.6 us slower at 32k.)
    int base = first;
    for (int i = 0; i + 1 < ntrips; i += 2) {
        load_trip<D, EPL, U, NT, Q8>(tb, a, kvh, base + ROWS_BLOCK, cache_end, grp, j);
        consume_trip<D, G, EPL, U, Q8, LAZY>(ta, qr, m, l, o, a);
        load_trip<D, EPL, U, NT, Q8>(ta, a, kvh, base + 2 * ROWS_BLOCK, cache_end, grp, j);
        consume_trip<D, G, EPL, U, Q8, LAZY>(tb, qr, m, l, o, a);
        base += 2 * ROWS_BLOCK;
    }
    if (ntrips & 1) consume_trip<D, G, EPL, U, Q8, LAZY>(ta, qr, m, l, o, a);

    // 4. Row `pos` as the cache now holds it, from LDS (row group 0 of wave 0).
    if (has_pos && wave == 0) {
        if constexpr (!Q8) {
            float4 kf[1][C4], vf[1][C4];
            bool valid[1] = {grp == 0};
#pragma unroll
            for (int c = 0; c < C4; ++c) {
                const int d0 = F::dim(j, 4 * c);
                kf[0][c] = make_float4(s_x[G * D + d0], s_x[G * D + d0 + 1], s_x[G * D + d0 + 2],
                                       s_x[G * D + d0 + 3]);
                vf[0][c] = make_float4(s_v[d0], s_v[d0 + 1], s_v[d0 + 2], s_v[d0 + 3]);
            }
            accumulate_rows<D, G, EPL, 1>(qr, kf, vf, valid, m, l, o, a);
        } else {
            float kq[1][16], vq[1][16], ksc[1], vsc[1];
            bool valid[1] = {grp == 0};
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                kq[0][e] = (float)s_kq[16 * j + e];
                vq[0][e] = (float)s_vq[16 * j + e];
            }
            ksc[0] = s_ks[j >> 1];
            vsc[0] = s_vs[j >> 1];
            accumulate_rows_q8<D, G, 1>(qr, kq, ksc, vq, vsc, valid, m, l, o, a);
        }
    }

    // 5. Merge the partial states.  LDS_MERGE: each row group writes its raw (m, l, o); the
    //    per-(partial, head) weights 2^(m - M) are computed once, then each output element is
    //    a weighted sum over the NPART partials.  Otherwise the row groups of each wave are
    //    merged with lane exchanges first (the state of 8-wave workgroups and of large groups
    //    does not fit in 32 KB of LDS).
    if constexpr (LDS_MERGE) {
        const int pidx = wave * RPW + grp;
#pragma unroll
        for (int h = 0; h < G; ++h) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) s_o[(pidx * G + h) * D + F::dim(j, e)] = o[h][e];
            if (j == 0) {
                s_m[pidx * G + h] = m[h];
                s_l[pidx * G + h] = l[h];
            }
        }
        __syncthreads();
        if (tid < NPART * G) {
            const int h = tid % G;
            float M = s_m[h];
#pragma unroll
            for (int q = 1; q < NPART; ++q) M = fmaxf(M, s_m[q * G + h]);
            s_w[tid] = fast_exp2(s_m[tid] - M);
            if (tid < G) {
                float L = 0.0f;
#pragma unroll
                for (int q = 0; q < NPART; ++q)
                    L = __builtin_fmaf(s_l[q * G + h], fast_exp2(s_m[q * G + h] - M), L);
                s_ML[2 * h] = M;
                s_ML[2 * h + 1] = L;
            }
        }
        __syncthreads();
        for (int idx = tid; idx < G * D; idx += NTHR) {
            const int h = idx / D, d = idx - h * D;
            const float M = s_ML[2 * h], L = s_ML[2 * h + 1];
            float O = 0.0f;
#pragma unroll
            for (int q = 0; q < NPART; ++q)
                O = __builtin_fmaf(s_o[(q * G + h) * D + d], s_w[q * G + h], O);
            if (sp.splits == 1) {
                a.out[(h0 + h) * D + d] =
                    finish_output(M, L, O, a.sinks, a.gate, h0 + h, (long long)(h0 + h) * D + d);
            } else {
                const long long slot = ((long long)vkh * sp.splits + split) * G + h;
                store_partial(a.part_o + slot * D + d, O, CAN_FUSE && a.fused);
                if (d == 0) {
                    store_partial(a.part_ml + 2 * slot, M, CAN_FUSE && a.fused);
                    store_partial(a.part_ml + 2 * slot + 1, L, CAN_FUSE && a.fused);
                }
            }
        }
    } else {
        // 5. Merge the row groups of each wave (lanes j, j+LPR, ...), then the waves via LDS.
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float mw = m[h];
            if constexpr (LPR <= 4) mw = lane_step<4, true>(mw);
            if constexpr (LPR <= 8) mw = lane_step<8, true>(mw);
            if constexpr (LPR <= 16) mw = lane_step<16, true>(mw);
            if constexpr (LPR <= 32) mw = lane_step<32, true>(mw);
            const float sc = fast_exp2(m[h] - mw);
            float lw = l[h] * sc;
            if constexpr (LPR <= 4) lw = lane_step<4, false>(lw);
            if constexpr (LPR <= 8) lw = lane_step<8, false>(lw);
            if constexpr (LPR <= 16) lw = lane_step<16, false>(lw);
            if constexpr (LPR <= 32) lw = lane_step<32, false>(lw);
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                float x = o[h][e] * sc;
                if constexpr (LPR <= 4) x = lane_step<4, false>(x);
                if constexpr (LPR <= 8) x = lane_step<8, false>(x);
                if constexpr (LPR <= 16) x = lane_step<16, false>(x);
                if constexpr (LPR <= 32) x = lane_step<32, false>(x);
                o[h][e] = x;
            }
            m[h] = mw;
            l[h] = lw;
        }
        if (grp == 0) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
#pragma unroll
                for (int e = 0; e < EPL; ++e) s_o[(wave * G + h) * D + F::dim(j, e)] = o[h][e];
                if (j == 0) {
                    s_m[wave * G + h] = m[h];
                    s_l[wave * G + h] = l[h];
                }
            }
        }
        __syncthreads();

        for (int idx = tid; idx < G * D; idx += NTHR) {
            const int h = idx / D, d = idx - h * D;
            float M = s_m[h];
#pragma unroll
            for (int w = 1; w < WAVES; ++w) M = fmaxf(M, s_m[w * G + h]);
            float L = 0.0f, O = 0.0f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                const float sc = fast_exp2(s_m[w * G + h] - M);
                L = __builtin_fmaf(s_l[w * G + h], sc, L);
                O = __builtin_fmaf(s_o[(w * G + h) * D + d], sc, O);
            }
            if (sp.splits == 1) {
                a.out[(h0 + h) * D + d] =
                    finish_output(M, L, O, a.sinks, a.gate, h0 + h, (long long)(h0 + h) * D + d);
            } else {
                const long long slot = ((long long)vkh * sp.splits + split) * G + h;
                store_partial(a.part_o + slot * D + d, O, CAN_FUSE && a.fused);
                if (d == 0) {
                    store_partial(a.part_ml + 2 * slot, M, CAN_FUSE && a.fused);
                    store_partial(a.part_ml + 2 * slot + 1, L, CAN_FUSE && a.fused);
                }
            }
        }
    }
    if constexpr (CAN_FUSE) {
        if (sp.splits > 1 && a.fused) combine_if_last<D, G, NTHR>(a, vkh, sp.splits, tid, CMB_ALIAS ? s_o : s_cmb);
    }
}

// ---- Q8_0 cache, scores on the matrix cores --------------------------------------------------
// The same split-K decode over a Q8_0 cache (GQA groups of up to 4 query heads), with the
// scores as int8 matrix products: per 16-key tile and 32-dim scale block, one
// v_mfma_i32_16x16x64_i8 multiplies the tile's K quants (B operand, read straight from the
// cache) by the query's int8 parts (A operand).  Up to head_dim 128 the 64-deep product
// covers two scale blocks of K (a lane's B operand is 16 contiguous quants: dims
// 64p + 16(l/16) .. +15), and the A operand of block 2p carries the query parts in lane groups
// 0-1 only, that of block 2p+1 in groups 2-3 only, so each product is one block's dot
// product: the 16-byte loads halve the K load instructions of a tile against four 8-byte
// pieces 32 bytes apart.  At head_dim 256 the two zero-padded operands per pair cost the
// registers of an occupancy step, and a v_mfma_i32_16x16x32_i8 per block takes the 8-byte
// pieces (dims 32b + 8(l/16) .. +7).  Each (query head, block) of the scaled query
// is held as q = s * (Q1 + (Q2 + Q3/F)/F) with s = max|q|/127 and F = 254, Q1..Q3 int8, which
// represents q to 2^-23 of the block maximum; the three integer dot products with the quants
// are exact, so a score  sum_b ks_b * s_b * (D1 + (D2 + D3/F)/F)  rounds at the fp32 level of
// KVCache.dotK in Q8_0 mode (KVCache.java:187-195).  Rows of A are (head, part) = 4*head +
// part, so the accumulator lane (key l%16, head l/16) holds a head's three part sums for its
// key.  The online softmax runs per 16-key tile in that layout (tile max over a DPP row); the
// probabilities go through LDS to the V lanes, which accumulate o += (p * vscale) * quants in
// fp32 as KVCache.saxpyV does (KVCache.java:201-210), 16 quants per lane.
typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef unsigned int native_u2 __attribute__((ext_vector_type(2)));

constexpr float kQPartF = 254.0f;
constexpr float kQPartInvF = 1.0f / 254.0f;

template <bool NT>
__device__ __forceinline__ uint2 load_u2(const uint2* p) {
    if constexpr (NT) {
        const native_u2 v = __builtin_nontemporal_load(reinterpret_cast<const native_u2*>(p));
        return make_uint2(v.x, v.y);
    } else {
        return *p;
    }
}

// The raw bytes one lane holds of a 16-key tile.
template <int D>
struct Q8Tile {
    static constexpr int NB = D / 32;     // scale blocks per row
    static constexpr int LPR = D / 16;    // V lanes per key (16 quants each)
    static constexpr int KPL = 64 / LPR;  // keys per wave-wide V load
    static constexpr int UV = 16 / KPL;   // V loads per tile
    static constexpr int NP = D / 64;     // 64-dim pairs of scale blocks
    static constexpr bool K64 = D <= 128; // 16x16x64 products (else one 16x16x32 per block)
    uint4 k[K64 ? NP : 1];    // K64: quants of key l%16, dims 64p + 16(l/16) .. +15
    uint2 k8[K64 ? 1 : NB];   // else: dims 32b + 8(l/16) .. +7
    float ks[NB];  // K block scales of key l%16
    uint4 v[UV];   // V quants of key u*KPL + l/LPR, dims 16(l%LPR) .. +15
    float vs[UV];  // its V block scale
};

// Loads of keys t0 .. t0+15 (rows past `last` read row `last` and are masked by the caller).
template <int D, bool NT>
__device__ __forceinline__ void q8_tile_load(Q8Tile<D>& t, const signed char* kq, const float* ks,
                                             const signed char* vq, const float* vs, int t0,
                                             int last, int lane) {
    using T = Q8Tile<D>;
    const int kr = min(t0 + (lane & 15), last);
    if constexpr (T::K64) {
        const signed char* krow = kq + (long long)kr * D + 16 * (lane >> 4);
#pragma unroll
        for (int p = 0; p < T::NP; ++p) t.k[p] = load_u4<NT>(reinterpret_cast<const uint4*>(krow + 64 * p));
    } else {
        const signed char* krow = kq + (long long)kr * D + 8 * (lane >> 4);
#pragma unroll
        for (int b = 0; b < T::NB; ++b) t.k8[b] = load_u2<NT>(reinterpret_cast<const uint2*>(krow + 32 * b));
    }
    const float* ksr = ks + (long long)kr * T::NB;
    if constexpr (T::NB % 4 == 0) {
#pragma unroll
        for (int c = 0; c < T::NB / 4; ++c) {
            const float4 x = *reinterpret_cast<const float4*>(ksr + 4 * c);
            t.ks[4 * c + 0] = x.x;
            t.ks[4 * c + 1] = x.y;
            t.ks[4 * c + 2] = x.z;
            t.ks[4 * c + 3] = x.w;
        }
    } else {
        static_assert(T::NB == 2, "head_dim 64, 128 or 256");
        const float2 x = *reinterpret_cast<const float2*>(ksr);
        t.ks[0] = x.x;
        t.ks[1] = x.y;
    }
    const int j = lane % T::LPR;
#pragma unroll
    for (int u = 0; u < T::UV; ++u) {
        const int vr = min(t0 + u * T::KPL + lane / T::LPR, last);
        t.v[u] = load_u4<NT>(reinterpret_cast<const uint4*>(vq + (long long)vr * D) + j);
        t.vs[u] = vs[(long long)vr * T::NB + (j >> 1)];
    }
}

// Int8 parts of the scaled query heads x ([G][D] fp32 in LDS), computed once per workgroup:
// parts [3][G][D] bytes, block scales qs [G][NB].  Value i of a pass sits in the 32-lane group
// that holds its whole block, so the block maximum is a cross-lane reduction.
template <int D, int G, int NTHR>
__device__ __forceinline__ void q8_query_split(const float* x, float qk_scale, signed char* parts,
                                               float* qs, int tid) {
    static_assert((G * D) % 32 == 0 && NTHR % 64 == 0, "blocks fill whole 32-lane groups");
    for (int i0 = 0; i0 < G * D; i0 += NTHR) {
        const int i = i0 + tid;
        const bool in = i < G * D;
        const float x0 = in ? x[i] * qk_scale : 0.0f;
        float mx = fabsf(x0);
        mx = fmaxf(mx, dpp<kDppQuadXor1>(mx));
        mx = fmaxf(mx, dpp<kDppQuadXor2>(mx));
        mx = fmaxf(mx, dpp<kDppRowHalfMirror>(mx));
        mx = fmaxf(mx, dpp<kDppRowMirror>(mx));
        mx = lane_step<16, true>(mx);
        const float sc = mx / 127.0f;
        const float inv = sc != 0.0f ? 1.0f / sc : 0.0f;
        const float v = x0 * inv;
        const float q1 = fminf(fmaxf(rintf(v), -127.0f), 127.0f);
        const float r1 = (v - q1) * kQPartF;
        const float q2 = fminf(fmaxf(rintf(r1), -127.0f), 127.0f);
        const float r2 = (r1 - q2) * kQPartF;
        const float q3 = fminf(fmaxf(rintf(r2), -127.0f), 127.0f);
        if (in) {
            parts[i] = (signed char)(int)q1;
            parts[G * D + i] = (signed char)(int)q2;
            parts[2 * G * D + i] = (signed char)(int)q3;
            if ((i & 31) == 0) qs[i >> 5] = sc;
        }
    }
}

// The lane's A operands, row l%16 = (head (l%16)/4, part l%4); rows of absent heads and
// part 3 are zero.  16x16x64 (D <= 128): two per 64-dim pair p, dims 64p + 16(l/16) .. +15,
// held in aq0[p] by lane groups 0-1 (block 2p) and in aq1[p] by groups 2-3 (block 2p+1), zero
// elsewhere.  16x16x32: one per block b in aq8[b], dims 32b + 8(l/16) .. +7.
template <int D, int G>
__device__ __forceinline__ void q8_query_operands(const signed char* parts, int lane,
                                                  v4i_t (&aq0)[D / 64], v4i_t (&aq1)[D / 64]) {
    const int row = lane & 15, h = row >> 2, part = row & 3, g = lane >> 4;
    const bool live = h < G && part < 3;
    const signed char* src = parts + (live ? part * G * D + h * D : 0) + 16 * g;
    const v4i_t z = {0, 0, 0, 0};
#pragma unroll
    for (int p = 0; p < D / 64; ++p) {
        const v4i_t w = *reinterpret_cast<const v4i_t*>(src + 64 * p);
        aq0[p] = (live && g < 2) ? w : z;
        aq1[p] = (live && g >= 2) ? w : z;
    }
}
template <int D, int G>
__device__ __forceinline__ void q8_query_operands8(const signed char* parts, int lane, long (&aq)[D / 32]) {
    const int row = lane & 15, h = row >> 2, part = row & 3;
    const bool live = h < G && part < 3;
    const signed char* src = parts + (live ? part * G * D + h * D : 0) + 8 * (lane >> 4);
#pragma unroll
    for (int b = 0; b < D / 32; ++b) {
        const long w = *reinterpret_cast<const long*>(src + 32 * b);
        aq[b] = live ? w : 0;
    }
}

// Orders one wave's LDS writes before its later LDS reads of other lanes' data.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
}

template <int D, int G, int WAVES, bool NT>
__global__ __launch_bounds__(WAVES * 64) void decode_q8_mfma_kernel(DecodeArgs a) {
    static_assert(G >= 1 && G <= 4, "A rows hold 4 heads x (3 parts + 1)");
    using T = Q8Tile<D>;
    constexpr int NB = T::NB, LPR = T::LPR, KPL = T::KPL, UV = T::UV;
    constexpr int NTHR = WAVES * 64;
    constexpr int TSTEP = WAVES * 16;

    __shared__ float s_x[(G + 1) * D];
    __shared__ float s_v[D];
    __shared__ float s_acc[(G + 1) * 8];
    __shared__ float s_r[G + 1];
    __shared__ float s_qs[G * NB];
    __shared__ __align__(16) signed char s_qp[3 * G * D];
    __shared__ float4 s_p[WAVES * 16];  // per wave and key slot: p of heads 0..3
    __shared__ float4 s_al[WAVES];      // per wave: rescale factors of heads 0..3
    __shared__ float s_m[WAVES * G];
    __shared__ float s_l[WAVES * G];
    __shared__ float s_o[WAVES * G * D];
    constexpr bool CAN_FUSE = WAVES != 4;   // as in decode_split_kernel
    constexpr bool CMB_ALIAS = WAVES * G * D >= combine_scratch_floats<NTHR>();
    __shared__ float s_cmb[(CMB_ALIAS || !CAN_FUSE) ? 1 : combine_scratch_floats<NTHR>()];

    const int tid = threadIdx.x;
    const int split = blockIdx.x;
    const int vkh = blockIdx.y;          // virtual KV head (see decode_split_kernel)
    const int kvh = vkh / a.kv_rep;
    const bool store = vkh == kvh * a.kv_rep;
    const int h0 = vkh * G;
    load_args_now(a);
    if constexpr (CAN_FUSE) load_merge_args_now(a);
    const int pos = step_position(a);
    if (pos < 0 || pos >= a.max_seq) return;
    const StepPlan sp = plan_step(pos, a.window, a.splits);
    if (split >= sp.splits) return;
    const HeadPrep hp = head_prep(a, pos);
    const int row_begin = sp.start + split * sp.rows_per_split;
    const int row_end = min(row_begin + sp.rows_per_split, pos + 1);
    const bool has_pos = (row_end == pos + 1) && a.no_append == 0;
    const int cache_end = has_pos ? pos : row_end;
    // The wave index is wave-uniform: from an SGPR, the tile loop's branches are scalar.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;

    const signed char* kqp = a.kq + (long long)kvh * a.head_stride;
    const signed char* vqp = a.vq + (long long)kvh * a.head_stride;
    const float* ksp = a.ks + (long long)kvh * (a.head_stride / 32);
    const float* vsp = a.vs + (long long)kvh * (a.head_stride / 32);
    const int last = cache_end > 0 ? cache_end - 1 : 0;

    // 1. The query prep's inputs are requested first and the wave's first two tiles right
    //    after them: the load counter completes in order, so the prologue waits for its own
    //    loads alone while the tiles stream in.
    static_assert(D <= NTHR, "one RoPE pair and one norm weight per thread");
    constexpr int QPT = (G * D + NTHR - 1) / NTHR;
    float qv[QPT];
#pragma unroll
    for (int r = 0; r < QPT; ++r) qv[r] = a.q[h0 * D + min(tid + r * NTHR, G * D - 1)];
    const bool rope = hp.cos_row != nullptr, qkn = hp.qnw != nullptr;
    const int ci = min(tid, max(hp.half_rope - 1, 0));
    const float cs = (rope ? hp.cos_row : a.q)[rope ? ci : 0];
    const float sn = (rope ? hp.sin_row : a.q)[rope ? ci : 0];
    const float qw = (qkn ? hp.qnw : a.q)[qkn ? tid % D : 0];
    T ta, tb;
    int t0 = row_begin + wave * 16;
    q8_tile_load<D, NT>(ta, kqp, ksp, vqp, vsp, t0, last, lane);

    // 2. Query heads: exact prep in LDS, the scale folded in, split into int8 parts.
    __shared__ float s_cs[D / 2], s_sn[D / 2], s_qw[D];
#pragma unroll
    for (int r = 0; r < QPT; ++r)
        if (tid + r * NTHR < G * D) s_x[tid + r * NTHR] = qv[r];
    if (tid < hp.half_rope) {
        s_cs[tid] = cs;
        s_sn[tid] = sn;
    }
    if (tid < D) s_qw[tid] = qw;
    __syncthreads();
    const lds_cptr lnull = nullptr;
    const HeadPrepLds hl{qkn ? (lds_cptr)s_qw : lnull, qkn ? (lds_cptr)s_qw : lnull, hp.eps,
                         rope ? (lds_cptr)s_cs : lnull, rope ? (lds_cptr)s_sn : lnull,
                         hp.half_rope, hp.rope_type};
    prep_heads_lds<D, NTHR>(s_x, G, G, s_acc, s_r, hl, tid);
    q8_query_split<D, G, NTHR>(s_x, a.qk_scale, s_qp, s_qs, tid);
    __syncthreads();
    v4i_t aq0[T::K64 ? T::NP : 1], aq1[T::K64 ? T::NP : 1];
    long aq8[T::K64 ? 1 : NB];
    if constexpr (T::K64)
        q8_query_operands<D, G>(s_qp, lane, aq0, aq1);
    else
        q8_query_operands8<D, G>(s_qp, lane, aq8);
    const int qh = lane >> 4;  // head of the lane's scores
    float sq[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) sq[b] = qh < G ? s_qs[qh * NB + b] : 0.0f;

    // 3. Stream the cached rows in 16-key tiles, one tile ahead in registers.
    float M = kNegBig, lsum = 0.0f;
    float o[G][16];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[h][e] = 0.0f;
    float4* sp_w = s_p + wave * 16;
    float* al_w = reinterpret_cast<float*>(s_al + wave);

    auto consume = [&](const T& t, int base, int end) {
        float s = 0.0f;
#pragma unroll
        for (int b = 0; b < NB; ++b) {   // blocks in order
            v4i_t d;
            if constexpr (T::K64)
                d = __builtin_amdgcn_mfma_i32_16x16x64_i8((b & 1) ? aq1[b >> 1] : aq0[b >> 1],
                                                          __builtin_bit_cast(v4i_t, t.k[b >> 1]),
                                                          v4i_t{0, 0, 0, 0}, 0, 0, 0);
            else
                d = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq8[b], __builtin_bit_cast(long, t.k8[b]),
                                                          v4i_t{0, 0, 0, 0}, 0, 0, 0);
            const float f = (float)d[0] + ((float)d[1] + (float)d[2] * kQPartInvF) * kQPartInvF;
            s = __builtin_fmaf(f, t.ks[b] * sq[b], s);
        }
        if (a.softcap > 0.0f) s = a.softcap_log2e * tanhf(s * a.inv_softcap);
        s = base + (lane & 15) < end ? s : -__builtin_inff();
        float mt = fmaxf(s, dpp<kDppQuadXor1>(s));
        mt = fmaxf(mt, dpp<kDppQuadXor2>(mt));
        mt = fmaxf(mt, dpp<kDppRowHalfMirror>(mt));
        mt = fmaxf(mt, dpp<kDppRowMirror>(mt));
        const bool rescale = __any(mt > M + kLazyMargin);
        if (rescale) {
            const float mn = fmaxf(M, mt);
            const float al = fast_exp2(M - mn);
            M = mn;
            lsum = lsum * al;
            if ((lane & 15) == 0) al_w[qh] = al;
        }
        const float p = fast_exp2(s - M);
        lsum = lsum + p;
        reinterpret_cast<float*>(sp_w)[(lane & 15) * 4 + qh] = p;
        wave_lds_sync();
        if (rescale) {
            const float4 al4 = *reinterpret_cast<const float4*>(al_w);
            const float al[4] = {al4.x, al4.y, al4.z, al4.w};
#pragma unroll
            for (int h = 0; h < G; ++h)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[h][e] = o[h][e] * al[h];
        }
#pragma unroll
        for (int u = 0; u < UV; ++u) {
            const float4 p4 = sp_w[u * KPL + lane / LPR];
            const float pw[4] = {p4.x, p4.y, p4.z, p4.w};
            float w[G];
#pragma unroll
            for (int h = 0; h < G; ++h) w[h] = pw[h] * t.vs[u];
            const unsigned dw[4] = {t.v[u].x, t.v[u].y, t.v[u].z, t.v[u].w};
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const float vf = (float)(int)(signed char)(dw[c] >> (8 * b));
#pragma unroll
                    for (int h = 0; h < G; ++h)
                        o[h][4 * c + b] = __builtin_fmaf(w[h], vf, o[h][4 * c + b]);
                }
        }
        wave_lds_sync();
    };

    // Tiles in pairs, so that the loop has one exit (a break between the two halves would
    // join the loop head with the second buffer's loads in flight, and the wait inserted
    // there would drain the prefetch on every trip); an odd last tile follows.  (Peeling the
    // last pair so that its unused refill is not fetched costs this kernel 20-30 VGPRs and an
    // occupancy step at most shapes, so the refill stays.)
    const int ntiles = t0 < cache_end ? (cache_end - t0 + TSTEP - 1) / TSTEP : 0;
    for (int i = 0; i + 1 < ntiles; i += 2) {
        q8_tile_load<D, NT>(tb, kqp, ksp, vqp, vsp, t0 + TSTEP, last, lane);
        consume(ta, t0, cache_end);
        q8_tile_load<D, NT>(ta, kqp, ksp, vqp, vsp, t0 + 2 * TSTEP, last, lane);
        consume(tb, t0 + TSTEP, cache_end);
        t0 += 2 * TSTEP;
    }
    if (ntiles & 1) consume(ta, t0, cache_end);

    // 4. The split that owns row pos appends it and takes it from LDS as a one-key tile.
    if (has_pos) {
        __shared__ float s_vr;
        __shared__ __align__(16) signed char s_kq[D], s_vq[D];
        __shared__ float s_ks[NB], s_vs[NB], s_inv[NB];
        stage_new_row<D, NTHR>(a, kvh, s_x + G * D, s_v, s_acc, s_r, &s_vr, hp, tid);
        append_row_q8<D, NTHR>(a, kvh, pos, s_x + G * D, s_v, s_kq, s_ks, s_vq, s_vs, s_inv, tid, store);
        if (wave == 0) {
            T t;
            const bool k0 = (lane & 15) == 0;
            if constexpr (T::K64) {
#pragma unroll
                for (int p = 0; p < T::NP; ++p)
                    t.k[p] = k0 ? *reinterpret_cast<const uint4*>(s_kq + 64 * p + 16 * (lane >> 4))
                                : make_uint4(0u, 0u, 0u, 0u);
            } else {
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    t.k8[b] = k0 ? *reinterpret_cast<const uint2*>(s_kq + 32 * b + 8 * (lane >> 4))
                                 : make_uint2(0u, 0u);
            }
#pragma unroll
            for (int b = 0; b < NB; ++b) t.ks[b] = k0 ? s_ks[b] : 0.0f;
            const bool v0 = lane < LPR;
            t.v[0] = v0 ? *reinterpret_cast<const uint4*>(s_vq + 16 * lane) : make_uint4(0u, 0u, 0u, 0u);
            t.vs[0] = v0 ? s_vs[lane >> 1] : 0.0f;
#pragma unroll
            for (int u = 1; u < UV; ++u) {
                t.v[u] = make_uint4(0u, 0u, 0u, 0u);
                t.vs[u] = 0.0f;
            }
            consume(t, pos, pos + 1);
        }
    }

    // 5. Merge within the wave: sums over the key slots of a head (one DPP row) and over the
    //    V lanes of equal dims, then across waves through LDS.
    const float L = row_group_sum<16>(lsum);
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            float x = o[h][e];
            if constexpr (LPR <= 4) x = lane_step<4, false>(x);
            if constexpr (LPR <= 8) x = lane_step<8, false>(x);
            if constexpr (LPR <= 16) x = lane_step<16, false>(x);
            x = lane_step<32, false>(x);
            o[h][e] = x;
        }
    if (lane < LPR) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int e = 0; e < 16; ++e) s_o[(wave * G + h) * D + 16 * lane + e] = o[h][e];
    }
    if ((lane & 15) == 0 && qh < G) {
        s_m[wave * G + qh] = M;
        s_l[wave * G + qh] = L;
    }
    __syncthreads();

    for (int idx = tid; idx < G * D; idx += NTHR) {
        const int h = idx / D, d = idx - h * D;
        float Mx = s_m[h];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) Mx = fmaxf(Mx, s_m[w * G + h]);
        float Ls = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float sc = fast_exp2(s_m[w * G + h] - Mx);
            Ls = __builtin_fmaf(s_l[w * G + h], sc, Ls);
            O = __builtin_fmaf(s_o[(w * G + h) * D + d], sc, O);
        }
        if (sp.splits == 1) {
            a.out[(h0 + h) * D + d] =
                finish_output(Mx, Ls, O, a.sinks, a.gate, h0 + h, (long long)(h0 + h) * D + d);
        } else {
            const long long slot = ((long long)vkh * sp.splits + split) * G + h;
            store_partial(a.part_o + slot * D + d, O, CAN_FUSE && a.fused);
            if (d == 0) {
                store_partial(a.part_ml + 2 * slot, Mx, CAN_FUSE && a.fused);
                store_partial(a.part_ml + 2 * slot + 1, Ls, CAN_FUSE && a.fused);
            }
        }
    }
    if constexpr (CAN_FUSE) {
        if (sp.splits > 1 && a.fused) combine_if_last<D, G, NTHR>(a, vkh, sp.splits, tid, CMB_ALIAS ? s_o : s_cmb);
    }
}

// Combine of the splits: one block per query head; thread (column c, split group p) owns
// float4 column c of the head's output for the splits p, p+NP, ...  A thread's first
// kReduceBatch splits are loaded at once (one memory round trip), any further ones merge
// online; the per-group maxima and sums are merged through LDS.
constexpr int kReduceThreads = 256;
constexpr int kReduceBatch = 12;   // splits per thread loaded up front (96 splits at head_dim 128)

// CB workgroups per query head (blockIdx.y), each owning D/CB of the columns: with many splits
// per head the loads of one workgroup would take several rounds (CB is picked on the host so
// that every thread's splits fit in one batch).
template <int D, int CB = 1>
__global__ __launch_bounds__(kReduceThreads) void decode_reduce_kernel(DecodeArgs a, int G) {
    static_assert((D / 4) % CB == 0, "whole float4 columns per workgroup");
    constexpr int NC = D / 4 / CB;            // float4 columns of this workgroup
    constexpr int NP = kReduceThreads / NC;   // split groups
    __shared__ float s_m[NP], s_l[NP];
    __shared__ float4 s_o[NP][NC];
    const int hq = blockIdx.x;
    const int kvh = hq / G, h = hq - kvh * G;
    const int tid = threadIdx.x;
    const int cl = tid % NC, p = tid / NC;
    const int c = (CB > 1 ? (int)blockIdx.y * NC : 0) + cl;   // float4 column of the head
    const bool act = p < NP;   // NC need not divide the block: the spare threads only sync
    load_args_now(a);
    const int pos = step_position(a);
    if (pos < 0 || pos >= a.max_seq) return;
    const int S = plan_step(pos, a.window, a.splits).splits;
    if (S == 1) return;   // the split kernel wrote the output directly
    const long long slot0 = (long long)kvh * S * G + h;  // slot of split j: slot0 + j*G

    // This thread's first kReduceBatch splits: every load issued at once (masked entries
    // read split 0 and drop out), then one max and one weighted sum.
    float m = kNegBig, l = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    {
        float mj[kReduceBatch], lj[kReduceBatch];
        float4 oj[kReduceBatch];
#pragma unroll
        for (int u = 0; u < kReduceBatch; ++u) {
            const int jj = p + u * NP;
            const long long slot = slot0 + (long long)(jj < S ? jj : 0) * G;
            mj[u] = a.part_ml[2 * slot];
            lj[u] = a.part_ml[2 * slot + 1];
            oj[u] = reinterpret_cast<const float4*>(a.part_o + slot * D)[c];
        }
#pragma unroll
        for (int u = 0; u < kReduceBatch; ++u) m = fmaxf(m, p + u * NP < S ? mj[u] : kNegBig);
#pragma unroll
        for (int u = 0; u < kReduceBatch; ++u) {
            const float sj = p + u * NP < S ? fast_exp2(mj[u] - m) : 0.0f;
            l = __builtin_fmaf(lj[u], sj, l);
            o.x = __builtin_fmaf(oj[u].x, sj, o.x);
            o.y = __builtin_fmaf(oj[u].y, sj, o.y);
            o.z = __builtin_fmaf(oj[u].z, sj, o.z);
            o.w = __builtin_fmaf(oj[u].w, sj, o.w);
        }
    }
    // Splits beyond the batch: online merge.
#pragma unroll 4
    for (int jj = p + kReduceBatch * NP; jj < S; jj += NP) {
        const long long slot = slot0 + (long long)jj * G;
        const float mj = a.part_ml[2 * slot], lj = a.part_ml[2 * slot + 1];
        const float4 oj = reinterpret_cast<const float4*>(a.part_o + slot * D)[c];
        const float mn = fmaxf(m, mj);
        const float so = fast_exp2(m - mn), sj = fast_exp2(mj - mn);
        l = __builtin_fmaf(l, so, lj * sj);
        o.x = __builtin_fmaf(o.x, so, oj.x * sj);
        o.y = __builtin_fmaf(o.y, so, oj.y * sj);
        o.z = __builtin_fmaf(o.z, so, oj.z * sj);
        o.w = __builtin_fmaf(o.w, so, oj.w * sj);
        m = mn;
    }
    if (act && cl == 0) {
        s_m[p] = m;
        s_l[p] = l;
    }
    if (act) s_o[p][cl] = o;
    __syncthreads();
    if (p == 0) {
        float M = s_m[0];
        for (int q = 1; q < NP; ++q) M = fmaxf(M, s_m[q]);
        float L = 0.0f;
        float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int q = 0; q < NP; ++q) {
            const float sc = fast_exp2(s_m[q] - M);
            L = __builtin_fmaf(s_l[q], sc, L);
            const float4 x = s_o[q][cl];
            O.x = __builtin_fmaf(x.x, sc, O.x);
            O.y = __builtin_fmaf(x.y, sc, O.y);
            O.z = __builtin_fmaf(x.z, sc, O.z);
            O.w = __builtin_fmaf(x.w, sc, O.w);
        }
        const long long g0 = (long long)hq * D + 4 * c;
        O.x = finish_output(M, L, O.x, a.sinks, a.gate, hq, g0);
        O.y = finish_output(M, L, O.y, a.sinks, a.gate, hq, g0 + 1);
        O.z = finish_output(M, L, O.z, a.sinks, a.gate, hq, g0 + 2);
        O.w = finish_output(M, L, O.w, a.sinks, a.gate, hq, g0 + 3);
        reinterpret_cast<float4*>(a.out + (long long)hq * D)[c] = O;
    }
}

}  // namespace dk
}  // namespace llmp
