// Prefill attention for P prompt tokens at positions pos0..pos0+P-1, gfx950.
//
// The reference has no batched prefill: the prompt runs as P sequential single-token forwards
// (LLMEngine.java:478-480, InferenceEngine.prefill at InferenceEngine.java:374-381), so query i
// attends to rows [start(i), pos0+i] of a cache that already holds rows < pos0+i.  This path
// computes the same result in three launches:
//
//  1. prefill_append_kernel: one workgroup per token takes its k/v (fp32, or bf16 widened to
//     fp32), applies the exact QK-norm + RoPE of the decode path and writes the K/V rows
//     (bit-identical to P appends by the CPU path).
//  2. prefill_tile_kernel: once per (key tile, KV head), the fp16 hi/lo split of the tile's K
//     rows and of its V rows (transposed) into a workspace image laid out like the LDS tile.
//  3. prefill_attn2_kernel: causal flash attention on MFMA.  A workgroup owns one KV head and
//     16*NB query positions of all G query heads of that KV head; each wave owns 16 positions
//     of HPW query heads.  Tile images stream into two LDS buffers (tile i+2 is fetched into
//     registers while tile i is consumed); per 64-key tile a wave computes S^T = K Q^T and
//     O^T += V^T P^T with v_mfma_f32_16x16x32_f16 and an online softmax in the accumulator
//     layout.  Workgroups are ranked by key count and dispatched heaviest-first in the first
//     half of the grid, lightest-first in the second, so co-resident workgroups balance.
//
// Precision: Q and K are post-RoPE fp32, so each operand is split into hi = fp16(x) and
// lo = fp16(x - hi), and a product uses three MFMAs (hi*hi + hi*lo + lo*hi): ~2^-21 relative
// per term (a bf16 split would give ~2^-16), which keeps the output within ~1e-6 of the
// fp32 CPU path.  P V uses the same split for P and for V (rows written from bf16 inputs have
// lo = 0 within fp16's normal range).  The split needs |x| < 65504 for the K and V rows and the
// scaled query (the range fp16 KV caches assume); P <= 1.
//
// Layout facts of v_mfma_f32_16x16x32_f16 (and _bf16) used here (checked on MI355X): lane i holds
// A[i%16][8*(i/16)+j] and B[8*(i/16)+j][i%16] (j < 8) and D[4*(i/16)+j][i%16] (j < 4).
// S^T's D fragment (lane: query i%16, keys 4*(i/16)+j of a 16-key tile) is fed back as the B
// operand of the P V product without moving data across lanes: the 32 keys of an MFMA step
// are taken in the order {4q..4q+3 of tile 2c, 4q..4q+3 of tile 2c+1} (q = i/16), and V^T is
// stored in LDS in that key order, so its A operand is one 16-byte read.
#pragma once

#include <type_traits>

#include "decode_kernels.h"

namespace llmp {
namespace pk {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short short8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr float kNegBig = dk::kNegBig;

// Keys per LDS tile: 64, or 32 for head_dim 256 (keeps the fp16 hi/lo tile under 80 KB).
template <int D>
constexpr int tile_keys() { return D >= 256 ? 32 : 64; }

struct PrefillArgs {
    const void* q;            // [P][Hq*D]: bf16 bits, or fp32 when in_f32
    const void* k;            // [P][Hkv*D]
    const void* v;            // [P][Hkv*D]
    int in_f32;               // 1: q/k/v are fp32 projections (the CPU path's), 0: bf16 bits
    float* kc;                // fp32 cache: layer K plane [Hkv][max_seq][D]
    float* vc;
    signed char* kq;          // Q8_0 cache (when set): K quants [Hkv][max_seq][D]
    float* ks;                // Q8_0 cache: K block scales [Hkv][max_seq][D/32]
    signed char* vq;
    float* vs;
    long long head_stride;    // max_seq*D (elements of one KV head's rows)
    int* range;               // range exponents of the layer's rows [Hkv][K, V] (dk::note_range)
    int q8_trunc;             // Q8_0 append: 1 = truncate (8-lane SIMD contract), 0 = round half up
    int norm_seq;             // 1: K-norm sums squares sequentially (RMSNorm.apply with offsets)
    int v_norm;               // 1: V rows RMS-normalised without weights before the append
    const float* cos_t;       // RoPE table [max_seq][half] or nullptr (NoPE)
    const float* sin_t;
    const float* qnw;         // QK-norm weights or nullptr
    const float* knw;
    const float* sinks;       // [Hq] attention-sink logits times log2(e), or nullptr
    const float* gate;        // fp32 [P][Hq*D] output gate, or nullptr
    float* out;               // fp32 [P][Hq*D]
    float* part_o;            // split-K partials [ksplit][P][Hq][D] (ksplit > 1)
    float* part_ml;           // split-K (max, sum) [ksplit][P][Hq][2]
    int pos0, P, Hq, Hkv;
    int kv_rep;               // virtual KV heads per cached KV head in the attention grid (groups of
                              // more than 8 query heads run as kv_rep groups of Hq/(Hkv*kv_rep))
    int half_rope, rope_type;
    int window;               // > 0: attend to the last `window` rows (local layer)
    float eps;
    float qk_scale;           // folded into q: scale*log2(e), or scale when soft-capping
    float softcap, softcap_log2e, inv_softcap;
};

__device__ __forceinline__ float bf16_to_f32(unsigned short b) {
    return __uint_as_float((unsigned)b << 16);
}
// Element i of a prompt input array: fp32 as is, or bf16 bits widened to fp32 (exact).
__device__ __forceinline__ float in_val(const void* p, long long i, int f32) {
    return f32 ? static_cast<const float*>(p)[i]
               : bf16_to_f32(static_cast<const unsigned short*>(p)[i]);
}
// ---- 1. exact K/V append, one workgroup per token --------------------------------------------
// Every input of the workgroup (its K and V rows, the RoPE row, the K-norm weights) is requested
// in one pass and staged in LDS, so the append costs one memory round trip before its stores.
// LDS floats: Hkv*(2*D + 10) + 2*Hkv*D/32 + 2*D (prefill_append_lds).
// At most 64 VGPRs (8 waves per SIMD): a long prompt's workgroups then all fit on the chip at
// once (2048 four-wave workgroups at 8 waves per SIMD), where 7 waves per SIMD left a second
// round of workgroups behind the first.
template <int D, int NTHR>
__global__ __launch_bounds__(NTHR) __attribute__((amdgpu_waves_per_eu(8)))
void prefill_append_kernel(PrefillArgs a) {
    extern __shared__ float s_dyn[];
    const int kvd = a.Hkv * D;
    float* s_k = s_dyn;                    // Hkv*D
    float* s_acc = s_k + kvd;              // Hkv*8
    float* s_r = s_acc + a.Hkv * 8;        // Hkv
    float* s_v = s_r + a.Hkv;              // Hkv*D
    float* s_vr = s_v + kvd;               // Hkv
    float* s_inv = s_vr + a.Hkv;           // 2*Hkv*D/32
    float* s_cs = s_inv + 2 * kvd / 32;    // D/2: cos row
    float* s_sn = s_cs + D / 2;            // D/2: sin row
    float* s_w = s_sn + D / 2;             // D: K-norm weights
    const int i = blockIdx.x, tid = threadIdx.x;
    const int pos = a.pos0 + i;
    const bool rope = a.cos_t != nullptr, qkn = a.qnw != nullptr;
    if (!qkn && a.v_norm == 0 && a.kq == nullptr) {
        // fp32 cache, no QK-norm or V-norm: each thread rotates whole (head, pair) slots in
        // registers, with the slot map and float steps of prep_heads_lds (no LDS, no barrier).
        constexpr int HALF = D / 2;
        const int half = rope ? a.half_rope : 0;
        const bool neox = a.rope_type != 0;
        for (int sl = tid; sl < a.Hkv * HALF; sl += NTHR) {
            const int h = sl / HALF, p = sl - h * HALF;
            const bool rot = p < half;
            const int i0 = (rot && neox) ? p : 2 * p, i1 = (rot && neox) ? half + p : 2 * p + 1;
            const long long in0 = (long long)i * kvd + (long long)h * D;
            float k0 = in_val(a.k, in0 + i0, a.in_f32), k1 = in_val(a.k, in0 + i1, a.in_f32);
            const float v0 = in_val(a.v, in0 + i0, a.in_f32), v1 = in_val(a.v, in0 + i1, a.in_f32);
            if (rot) {
                const float c = a.cos_t[(long long)pos * a.half_rope + p];
                const float sn = a.sin_t[(long long)pos * a.half_rope + p];
                const float t0 = k0 * c, t1 = k1 * sn, t2 = k0 * sn, t3 = k1 * c;
                k0 = t0 - t1;
                k1 = t2 + t3;
            }
            const long long off = (long long)h * a.head_stride + (long long)pos * D;
            a.kc[off + i0] = k0;
            a.kc[off + i1] = k1;
            a.vc[off + i0] = v0;
            a.vc[off + i1] = v1;
            dk::note_range(a.range, h, max(dk::abs_bits(k0), dk::abs_bits(k1)),
                           max(dk::abs_bits(v0), dk::abs_bits(v1)));
        }
        return;
    }
    for (int e = tid; e < kvd; e += NTHR) {
        s_k[e] = in_val(a.k, (long long)i * kvd + e, a.in_f32);
        s_v[e] = in_val(a.v, (long long)i * kvd + e, a.in_f32);
    }
    if (rope) {
        for (int e = tid; e < a.half_rope; e += NTHR) {
            s_cs[e] = a.cos_t[(long long)pos * a.half_rope + e];
            s_sn[e] = a.sin_t[(long long)pos * a.half_rope + e];
        }
    }
    if (qkn && a.knw != nullptr)
        for (int e = tid; e < D; e += NTHR) s_w[e] = a.knw[e];
    __syncthreads();
    const dk::lds_cptr lnull = nullptr;
    const dk::HeadPrepLds hp{qkn ? (dk::lds_cptr)s_w : lnull, qkn ? (dk::lds_cptr)s_w : lnull,
                             a.eps, rope ? (dk::lds_cptr)s_cs : lnull,
                             rope ? (dk::lds_cptr)s_sn : lnull, a.half_rope, a.rope_type};
    dk::prep_heads_lds<D, NTHR>(s_k, a.Hkv, 0, s_acc, s_r, hp, tid, a.norm_seq != 0);
    if (a.v_norm != 0) {   // Gemma 4's weightless V-norm, sequential order (RMSNorm.applyNoScale)
        for (int h = tid; h < a.Hkv; h += NTHR) s_vr[h] = dk::seq_rms_inv<D>(s_v + h * D, a.eps);
        __syncthreads();
        for (int e = tid; e < kvd; e += NTHR) s_v[e] = s_v[e] * s_vr[e / D];
        __syncthreads();
    }
    if (a.kq == nullptr) {
        for (int e = tid; e < kvd; e += NTHR) {
            const int h = e / D, d = e - h * D;
            const long long off = (long long)h * a.head_stride + (long long)pos * D + d;
            a.kc[off] = s_k[e];
            a.vc[off] = s_v[e];
            dk::note_range(a.range, h, dk::abs_bits(s_k[e]), dk::abs_bits(s_v[e]));
        }
        return;
    }
    // Q8_0: the K and V rows are quantised block by block exactly like a decode append
    // (KVCache.storeK/storeV over a Q8_0 cache, KVCache.java:164-179).  Blocks [0, nb) are K's,
    // [nb, 2nb) V's; 4 consecutive codes are stored as one 32-bit word.
    const int nb = kvd / 32, bph = D / 32;
    for (int b = tid; b < 2 * nb; b += NTHR) {
        const bool is_v = b >= nb;
        const int bb = is_v ? b - nb : b, h = bb / bph;
        const float scale = dk::q8_block_scale((is_v ? s_v : s_k) + 32 * bb);
        s_inv[b] = dk::q8_inv_scale(scale);
        (is_v ? a.vs : a.ks)[(long long)h * (a.head_stride / 32) + (long long)pos * bph +
                             (bb - h * bph)] = scale;
    }
    __syncthreads();
    const bool trunc = a.q8_trunc != 0;
    for (int w = tid; w < 2 * kvd / 4; w += NTHR) {
        const bool is_v = w >= kvd / 4;
        const int e = 4 * (is_v ? w - kvd / 4 : w), h = e / D, d = e - h * D;
        const float* x = (is_v ? s_v : s_k) + e;
        const float inv = s_inv[(is_v ? nb : 0) + e / 32];
        unsigned word = 0, xb = 0;   // the dequantised values stay within the fp32 rows' range
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            word |= (unsigned)(dk::q8_code(x[j], inv, trunc) & 0xFF) << (8 * j);
            xb = max(xb, dk::abs_bits(x[j]));
        }
        dk::note_range(a.range, h, is_v ? 0u : xb, is_v ? xb : 0u);
        *reinterpret_cast<unsigned*>((is_v ? a.vq : a.kq) + (long long)h * a.head_stride +
                                     (long long)pos * D + d) = word;
    }
}

// Dynamic LDS bytes of prefill_append_kernel.
inline size_t prefill_append_lds(int Hkv, int D) {
    const size_t f = (size_t)Hkv * (2 * D + 10) + 2 * (size_t)Hkv * D / 32 + 2 * (size_t)D;
    return f * sizeof(float);
}

// ---- LDS tile layout (also the workspace image of a tile) -------------------------------------
// LDS tile: K hi/lo [TK keys][D] fp16, V^T hi/lo [D][TK] fp16, then one flag word.  Within
// each 32-key chunk of a V^T row the keys are stored in the order the P V MFMA takes them
// (vt_group_pos): the 8 keys {4q..4q+3, 16+4q..16+4q+3} a lane group q feeds to one MFMA are
// contiguous, so a lane reads its A operand with one 16-byte load.
//
// Bank conflicts.  The MFMA operand reads are ds_read_b128 of 16 rows x 4 consecutive 16-byte
// chunks (lane l: row l%16, chunk 4s + l/16).  On gfx950 the LDS serves such a read in 4
// cycles of 16 lanes over 64 four-byte banks; a cycle takes the lanes of one half-wave whose
// 4-lane quad index (bits 2-4 of the lane) has a given parity (measured with
// SQ_LDS_BANK_CONFLICT: lanes 0-3, 12-15, 20-23 and 24-27 share a cycle).  With 16-byte row
// padding the 16 rows of a cycle collide in pairs (every read took 8 cycles instead of 4).
// Instead the chunk index of a row is XOR-ed with the row (koff / voff): rows of 8 or more
// chunks with r mod min(chunks, 16), the 4-chunk V^T rows of 32-key tiles with (r/2) mod 4,
// which spreads each cycle's 16 reads over all 64 banks; no padding.  head_dim 96 (12 chunks, not
// a power of two) keeps a padded pitch of 14 chunks, which is conflict-free as well.
template <int D, int TKEYS = tile_keys<D>()>
struct alignas(16) TileLds {
    static constexpr int TK = TKEYS;
    static constexpr int KCH = D / 8;                          // 16-byte chunks of a K row
    static constexpr bool KSWZ = (KCH & (KCH - 1)) == 0;
    static constexpr int KP = KSWZ ? D : D + 16;               // K row pitch (fp16 elements)
    static constexpr int VCH = TK / 8;                         // 16-byte chunks of a V^T row
    static constexpr int VP = TK;                              // V^T row pitch
    unsigned short kh[TK * KP];
    unsigned short kl[TK * KP];
    unsigned short vh[D * VP];
    unsigned short vl[D * VP];
    // flag[0] (set by the image builder): nonzero when some V lo part of the tile exceeds
    // 2^-24 in magnitude; the other words are unused.
    unsigned flag[4];
    // Offset (fp16 elements) of element e of K row r, and of element e of V^T row d.
    static __device__ __forceinline__ int koff(int r, int e) {
        if constexpr (KSWZ)
            return r * KP + ((((e >> 3) ^ (r & (KCH >= 16 ? 15 : KCH - 1))) << 3) | (e & 7));
        else
            return r * KP + e;
    }
    static __device__ __forceinline__ int voff(int d, int e) {
        const int sw = VCH >= 8 ? (d & 7) : ((d >> 1) & (VCH - 1));
        return d * VP + ((((e >> 3) ^ sw) << 3) | (e & 7));
    }
};

// ---- 2. Tile images ----------------------------------------------------------------------------
// The fp16 hi/lo split of a key tile does not depend on the query block, so it is done once per
// (tile, KV head) into a workspace image laid out exactly like TileLds.

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

// Two fp32 values -> packed fp16 (round to nearest even, v_cvt_pk_f16_f32).
__device__ __forceinline__ unsigned pack_f16(float x, float y) {
    return __builtin_bit_cast(unsigned, __builtin_convertvector(floatx2{x, y}, f16x2));
}
// Split of two values: hi = fp16(x), lo = fp16(x - hi), packed in pairs: hi + lo holds x to
// ~2^-22 of |x| (or 2^-25 absolute below fp16's normal range).  Each lo half comes from one
// mixed-precision FMA, hi(f16) * -1 + x(f32), which forms the difference exactly and rounds it
// once to fp16 into its half of the register: the same bits as rounding the exact fp32
// difference, in 3 instructions per pair instead of 6.
__device__ __forceinline__ void split_pair(float x, float y, unsigned& hi, unsigned& lo) {
    hi = pack_f16(x, y);
    unsigned r;
    asm("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(hi), "v"(x));
    asm("v_fma_mixhi_f16 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "+v"(r) : "v"(hi), "v"(y));
    lo = r;
}
// True when either fp16 half of a packed lo pair is larger in magnitude than 2^-24 (fp16's
// smallest subnormal): rows written from bf16 inputs never are.
__device__ __forceinline__ bool lo_significant(unsigned lo) {
    return (lo & 0x7FFFu) > 1u || ((lo >> 16) & 0x7FFFu) > 1u;
}

// Position within a 32-key chunk of V^T of the 4 keys 4*g..4*g+3 (g < 8): groups 0-3 (keys
// 0-15) go to 8*g, groups 4-7 (keys 16-31) to 8*(g-4)+4.
__device__ __forceinline__ int vt_group_pos(int g) { return g < 4 ? 8 * g : 8 * (g - 4) + 4; }
// Element offset within a V^T row of the 4 keys 4*rq..4*rq+3 of a tile.
__device__ __forceinline__ int vt_keys_off(int rq) { return 32 * (rq >> 3) + vt_group_pos(rq & 7); }

template <int D>
constexpr int tile_img_u4() { return (int)(sizeof(TileLds<D>) / 16); }
// A tile image carries one flag (TileLds::flag): nonzero when some V lo part exceeds 2^-24 in
// magnitude.  Where it is zero the P V product drops its V-lo MFMA: the terms it would add are
// below 2^-24 * sum(P) / l <= 2^-24 of the output.

// One KV head's rows in the cache: fp32 rows (f), or Q8_0 quants (q) and block scales (s).
struct HeadRows {
    const float* f;
    const signed char* q;
    const float* s;
};
template <bool Q8>
__device__ __forceinline__ HeadRows head_rows(float* f, signed char* q, float* s,
                                              const PrefillArgs& a, int kvh) {
    if constexpr (Q8)
        return {nullptr, q + (long long)kvh * a.head_stride, s + (long long)kvh * (a.head_stride / 32)};
    else
        return {f + (long long)kvh * a.head_stride, nullptr, nullptr};
}
template <bool Q8>
__device__ __forceinline__ HeadRows k_rows(const PrefillArgs& a, int kvh) {
    return head_rows<Q8>(a.kc, a.kq, a.ks, a, kvh);
}
template <bool Q8>
__device__ __forceinline__ HeadRows v_rows(const PrefillArgs& a, int kvh) {
    return head_rows<Q8>(a.vc, a.vq, a.vs, a, kvh);
}

// Dims 4*c4 .. 4*c4+3 of row r, as loaded: fp32 values, or for Q8_0 the four quants (one
// 32-bit word, bit pattern in element 0) and their block's scale (element 1).  chunk_values
// turns a loaded chunk into fp32 values (quant * scale), so loads can be issued before any
// of the arithmetic.
template <int D, bool Q8>
__device__ __forceinline__ floatx4 load_chunk(const HeadRows& h, int r, int c4) {
    if constexpr (Q8) {
        const unsigned w = *reinterpret_cast<const unsigned*>(h.q + (long long)r * D + 4 * c4);
        return floatx4{__builtin_bit_cast(float, w), h.s[(long long)r * (D / 32) + (c4 >> 3)],
                       0.0f, 0.0f};
    } else {
        return reinterpret_cast<const floatx4*>(h.f + (long long)r * D)[c4];
    }
}
// 2^e as a float for -126 <= e <= 127, built from its exponent bits (integer operations, so a
// uniform e stays in scalar registers): the range scale factors of dk::note_range.
__device__ __forceinline__ float pow2i(int e) { return __uint_as_float((unsigned)(127 + e) << 23); }
// 1 / f for f a power of two given by pow2i (exact).
__device__ __forceinline__ float pow2_inv(float f) { return __uint_as_float(0x7F000000u - __float_as_uint(f)); }

template <bool Q8>
__device__ __forceinline__ floatx4 chunk_values(floatx4 x) {
    if constexpr (Q8) {
        const unsigned w = __float_as_uint(x[0]);
        const float sc = x[1];
        return floatx4{(float)(signed char)(w & 0xFF) * sc, (float)(signed char)((w >> 8) & 0xFF) * sc,
                       (float)(signed char)((w >> 16) & 0xFF) * sc, (float)(signed char)(w >> 24) * sc};
    } else {
        return x;
    }
}

// Image of keys [tau*TK, tau*TK + TK) of KV head blockIdx.y, tau = tile0 + blockIdx.x, at
// ws[(kvh * n_tiles + blockIdx.x) * tile_img_u4<D>()], from fp32 or (Q8) dequantised Q8_0 rows,
// scaled by 2^-E of the head's range exponents (E = 0, no scaling, unless some stored value
// reached 2^15) so that every split part is finite.  Rows at or past row_end (never attended)
// repeat row row_end - 1 so that every staged value is finite.
template <int D, int NTHR, bool Q8>
__global__ __launch_bounds__(NTHR) void prefill_tile_kernel(PrefillArgs a, uint4* ws, int tile0,
                                                            int n_tiles, int row_end) {
    using T = TileLds<D>;
    constexpr int TK = T::TK;
    // The image has the LDS tile's layout; each thread writes its converted chunks to it
    // directly (no staging through LDS, so no copy-out pass behind a barrier).
    T& t = *reinterpret_cast<T*>(ws + ((size_t)blockIdx.y * n_tiles + blockIdx.x) * tile_img_u4<D>());
    const int tid = threadIdx.x, kvh = blockIdx.y;
    const int r0 = (tile0 + (int)blockIdx.x) * TK;
    const HeadRows kr = k_rows<Q8>(a, kvh), vr = v_rows<Q8>(a, kvh);
    const float fk = pow2i(-a.range[2 * kvh]), fv = pow2i(-a.range[2 * kvh + 1]);
    // K rows: work item (row r, dims 4*c4 .. 4*c4+3), c4 fastest across lanes, so the loads
    // are row-contiguous and the 8-byte stores of 16 lanes fill one image row.
    // V^T: work item (keys 4*rq .. 4*rq+3, dims 4*c4 .. 4*c4+3), rq fastest across lanes: each
    // dim row gets the 4 keys as one 8-byte store, and the TK/4 lanes that share a dim chunk
    // write one V^T row's TK keys together; a load instruction reads 64/(TK/4) consecutive
    // 16-byte chunks of TK/4 rows.
    // Every global load of a thread is issued before any of its math (one memory round trip).
    constexpr int KI = TK * (D / 4) / NTHR, VI = (TK / 4) * (D / 4) / NTHR;
    static_assert(KI * NTHR == TK * (D / 4) && VI * NTHR == (TK / 4) * (D / 4),
                  "tile work must divide evenly over the threads");
    floatx4 kx[KI], vx[VI][4];
#pragma unroll
    for (int i = 0; i < KI; ++i) {
        const int e = tid + i * NTHR;
        const int r = e / (D / 4), c4 = e - r * (D / 4);
        kx[i] = load_chunk<D, Q8>(kr, min(r0 + r, row_end - 1), c4);
    }
#pragma unroll
    for (int i = 0; i < VI; ++i) {
        const int e = tid + i * NTHR;
        const int c4 = e / (TK / 4), rq = e - c4 * (TK / 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) vx[i][j] = load_chunk<D, Q8>(vr, min(r0 + 4 * rq + j, row_end - 1), c4);
    }
#pragma unroll
    for (int i = 0; i < KI; ++i) {
        const int e = tid + i * NTHR;
        const int r = e / (D / 4), c4 = e - r * (D / 4);
        const floatx4 x = chunk_values<Q8>(kx[i]) * fk;
        unsigned h0, l0, h1, l1;
        split_pair(x[0], x[1], h0, l0);
        split_pair(x[2], x[3], h1, l1);
        *reinterpret_cast<uint2*>(&t.kh[T::koff(r, 4 * c4)]) = make_uint2(h0, h1);
        *reinterpret_cast<uint2*>(&t.kl[T::koff(r, 4 * c4)]) = make_uint2(l0, l1);
    }
    bool vlo = false;
#pragma unroll
    for (int i = 0; i < VI; ++i) {
        const int e = tid + i * NTHR;
        const int c4 = e / (TK / 4), rq = e - c4 * (TK / 4);
        const floatx4 vv[4] = {chunk_values<Q8>(vx[i][0]) * fv, chunk_values<Q8>(vx[i][1]) * fv,
                               chunk_values<Q8>(vx[i][2]) * fv, chunk_values<Q8>(vx[i][3]) * fv};   // [key][dim]
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            unsigned h0, l0, h1, l1;
            split_pair(vv[0][u], vv[1][u], h0, l0);
            split_pair(vv[2][u], vv[3][u], h1, l1);
            vlo = vlo || lo_significant(l0) || lo_significant(l1);
            const int d = 4 * c4 + u;
            *reinterpret_cast<uint2*>(&t.vh[T::voff(d, vt_keys_off(rq))]) = make_uint2(h0, h1);
            *reinterpret_cast<uint2*>(&t.vl[T::voff(d, vt_keys_off(rq))]) = make_uint2(l0, l1);
        }
    }
    const unsigned any_vlo = __syncthreads_or(vlo ? 1 : 0) ? 1u : 0u;
    if (tid == 0) t.flag[0] = any_vlo;
}

// ---- 3. Double-buffered MFMA attention ------------------------------------------------------
// Largest value of an int over the wave (prologue use only: lane exchanges through LDS).
__device__ __forceinline__ int wave_max_int(int x) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) x = max(x, __shfl_xor(x, off));
    return __builtin_amdgcn_readfirstlane(x);
}

// Query fragment of one lane for MFMA B operands: dims 32*s + 8*grp + j of query token qi
// (clamped into range), head hq, as fp32 (or widened from bf16), QK-normed, rotated, scaled,
// then split.  NEOX partners (d, d + half) usually sit in other lanes, so each element reads
// its partner from the input and normalises it exactly as the partner's own lane does; any
// rotated width (partial RoPE) works the same way.  The scaled queries of the wave are divided
// by 2^eq before their split, eq the range exponent of the largest magnitude among them (0
// below 2^15; wave-uniform, so the factor that restores the scores stays in scalar registers);
// the scores are multiplied back.
template <int D>
__device__ __forceinline__ void query_fragment(const PrefillArgs& a, int qi, int hq, int qpos,
                                               int grp, f16x8 (&qh)[D / 32],
                                               f16x8 (&ql)[D / 32], int& eq) {
    constexpr int KS = D / 32;
    float qf[KS][8];
    const long long q0 = (long long)qi * a.Hq * D + (long long)hq * D;
    // A lane's 8 elements per step are contiguous and 16-byte aligned (D is a multiple of 32):
    // one 16-byte load per step for bf16 inputs, two for fp32.
    if (a.in_f32) {
        const float* qp = static_cast<const float*>(a.q) + q0;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const float4 x0 = *reinterpret_cast<const float4*>(qp + 32 * s + 8 * grp);
            const float4 x1 = *reinterpret_cast<const float4*>(qp + 32 * s + 8 * grp + 4);
            qf[s][0] = x0.x; qf[s][1] = x0.y; qf[s][2] = x0.z; qf[s][3] = x0.w;
            qf[s][4] = x1.x; qf[s][5] = x1.y; qf[s][6] = x1.z; qf[s][7] = x1.w;
        }
    } else {
        const unsigned short* qp = static_cast<const unsigned short*>(a.q) + q0;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const uint4 w = *reinterpret_cast<const uint4*>(qp + 32 * s + 8 * grp);
            const unsigned u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                qf[s][2 * j] = __uint_as_float(u[j] << 16);
                qf[s][2 * j + 1] = __uint_as_float(u[j] & 0xFFFF0000u);
            }
        }
    }
    float r = 1.0f;
    if (a.qnw != nullptr) {
        float ss = 0.0f;
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(qf[s][j], qf[s][j], ss);
        ss = dk::lane_step<16, false>(ss);
        ss = dk::lane_step<32, false>(ss);
        r = 1.0f / sqrtf(ss / (float)D + a.eps);
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int j = 0; j < 8; ++j) qf[s][j] = (qf[s][j] * r) * a.qnw[32 * s + 8 * grp + j];
    }
    if (a.cos_t != nullptr) {
        const float* cr = a.cos_t + (long long)qpos * a.half_rope;
        const float* sr = a.sin_t + (long long)qpos * a.half_rope;
        const int half = a.half_rope;
        if (a.rope_type == 0) {
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                // the lane's 4 pairs are consecutive table entries: one 16-byte load each for
                // cos and sin when all 4 rotate and the rows are 16-byte aligned
                const int i0 = 16 * s + 4 * grp;
                float cv[4], sv[4];
                if ((half & 3) == 0 && i0 + 3 < half) {
                    const float4 c4 = *reinterpret_cast<const float4*>(cr + i0);
                    const float4 s4 = *reinterpret_cast<const float4*>(sr + i0);
                    cv[0] = c4.x; cv[1] = c4.y; cv[2] = c4.z; cv[3] = c4.w;
                    sv[0] = s4.x; sv[1] = s4.y; sv[2] = s4.z; sv[3] = s4.w;
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const bool rot = i0 + u < half;
                        cv[u] = cr[rot ? i0 + u : 0];
                        sv[u] = sr[rot ? i0 + u : 0];
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int j = 2 * u;
                    const bool rot = i0 + u < half;
                    const float c = cv[u], sn = sv[u];
                    const float v0 = qf[s][j], v1 = qf[s][j + 1];
                    const float t0 = v0 * c, t1 = v1 * sn, t2 = v0 * sn, t3 = v1 * c;
                    qf[s][j] = rot ? t0 - t1 : v0;
                    qf[s][j + 1] = rot ? t2 + t3 : v1;
                }
            }
        } else {  // NEOX: pairs (i, i + half) for i < half; dims >= 2*half keep their values
#pragma unroll
            for (int s = 0; s < KS; ++s)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int d = 32 * s + 8 * grp + j;
                    if (d < 2 * half) {
                        const bool first = d < half;
                        const int i = first ? d : d - half, pd = first ? d + half : d - half;
                        float pv = in_val(a.q, q0 + pd, a.in_f32);
                        if (a.qnw != nullptr) pv = (pv * r) * a.qnw[pd];
                        const float v0 = first ? qf[s][j] : pv, v1 = first ? pv : qf[s][j];
                        const float c = cr[i], sn = sr[i];
                        const float t0 = v0 * c, t1 = v1 * sn, t2 = v0 * sn, t3 = v1 * c;
                        qf[s][j] = first ? t0 - t1 : t2 + t3;
                    }
                }
        }
    }
    float qmax = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            qf[s][j] = qf[s][j] * a.qk_scale;
            qmax = fmaxf(qmax, fabsf(qf[s][j]));
        }
    eq = wave_max_int(dk::range_exp_of_bits(dk::abs_bits(qmax)));
    const float fq = pow2i(-eq);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        unsigned hh[4], ll[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            split_pair(qf[s][2 * j] * fq, qf[s][2 * j + 1] * fq, hh[j], ll[j]);
        qh[s] = __builtin_bit_cast(f16x8, make_uint4(hh[0], hh[1], hh[2], hh[3]));
        ql[s] = __builtin_bit_cast(f16x8, make_uint4(ll[0], ll[1], ll[2], ll[3]));
    }
}

// Copies of a tile image between global memory, registers and LDS: thread tid moves 16-byte
// chunks tid, tid + NTHR, ...
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <int PER, int NTHR, int IMG>
__device__ __forceinline__ void img_load(u32x4 (&stage)[PER], const uint4* src, int tid) {
    const u32x4* s = reinterpret_cast<const u32x4*>(src);
#pragma unroll
    for (int r = 0; r < PER; ++r) {
        const int idx = tid + r * NTHR;
        stage[r] = s[idx < IMG ? idx : IMG - 1];   // chunks past the image: a valid duplicate
    }
}
template <int PER, int NTHR, int IMG>
__device__ __forceinline__ void img_store(const u32x4 (&stage)[PER], void* dst, int tid) {
    u32x4* d = static_cast<u32x4*>(dst);
#pragma unroll
    for (int r = 0; r < PER; ++r) {
        const int idx = tid + r * NTHR;
        if (r + 1 < PER || idx < IMG) d[idx] = stage[r];
    }
}

// Direct staging from the fp32 cache (short prompts after a long prefix, where each key tile
// feeds only a few workgroups and building images first would re-convert the whole prefix on
// every call).  K: items (row, 4-dim chunk), the chunk index fastest across lanes so every load
// reads whole rows; V: items (4 keys, 4-dim chunk), stored transposed as 8-byte runs, the key
// group fastest across lanes (as in prefill_tile_kernel).  Rows at or past row_lim repeat row
// row_lim (never attended, finite).
// Keys per LDS tile of the direct-staging launches: 32, so two workgroups' double-buffered
// tiles fit in a CU's 160 KB of LDS (64-key tiles of head_dim 128 take 136 KB per workgroup).
template <int D>
constexpr int direct_tile_keys() { return 32; }

template <int D, int NTHR, int TK_ = direct_tile_keys<D>()>
struct RawTile {
    static constexpr int TK = TK_;
    static constexpr int NK = TK * (D / 4), NV = (TK / 4) * (D / 4);
    static constexpr int KI = (NK + NTHR - 1) / NTHR, VI = (NV + NTHR - 1) / NTHR;
};

template <int D, int NTHR, int KI, int VI, bool Q8, int TK = direct_tile_keys<D>()>
__device__ __forceinline__ void raw_load(floatx4 (&kx)[KI], floatx4 (&vx)[VI][4],
                                         const HeadRows& kr, const HeadRows& vr, int t0,
                                         int row_lim, int tid) {
    using R = RawTile<D, NTHR, TK>;
    static_assert(KI == R::KI && VI == R::VI, "staging register counts");
#pragma unroll
    for (int i = 0; i < R::KI; ++i) {
        const int e = min(tid + i * NTHR, R::NK - 1);
        const int r = e / (D / 4), c4 = e - r * (D / 4);
        kx[i] = load_chunk<D, Q8>(kr, min(t0 + r, row_lim), c4);
    }
#pragma unroll
    for (int i = 0; i < R::VI; ++i) {
        const int e = min(tid + i * NTHR, R::NV - 1);
        const int c4 = e / (TK / 4), rq = e - c4 * (TK / 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) vx[i][j] = load_chunk<D, Q8>(vr, min(t0 + 4 * rq + j, row_lim), c4);
    }
}

// The rows are scaled by fk (K) and fv (V), the head's 2^-E range factors (1 unless a stored
// value reached 2^15), before the split.
template <int D, int NTHR, int KI, int VI, bool Q8, int TK = direct_tile_keys<D>()>
__device__ __forceinline__ void raw_store(const floatx4 (&kx)[KI], const floatx4 (&vx)[VI][4],
                                          TileLds<D, TK>& t, int tid, float fk, float fv) {
    using R = RawTile<D, NTHR, TK>;
    static_assert(KI == R::KI && VI == R::VI, "staging register counts");
    using T = TileLds<D, TK>;
#pragma unroll
    for (int i = 0; i < R::KI; ++i) {
        const int e = tid + i * NTHR;
        if (i + 1 < R::KI || e < R::NK) {
            const int r = e / (D / 4), c4 = e - r * (D / 4);
            const floatx4 x = chunk_values<Q8>(kx[i]) * fk;
            unsigned h0, l0, h1, l1;
            split_pair(x[0], x[1], h0, l0);
            split_pair(x[2], x[3], h1, l1);
            *reinterpret_cast<uint2*>(&t.kh[T::koff(r, 4 * c4)]) = make_uint2(h0, h1);
            *reinterpret_cast<uint2*>(&t.kl[T::koff(r, 4 * c4)]) = make_uint2(l0, l1);
        }
    }
#pragma unroll
    for (int i = 0; i < R::VI; ++i) {
        const int e = tid + i * NTHR;
        if (i + 1 < R::VI || e < R::NV) {
            const int c4 = e / (TK / 4), rq = e - c4 * (TK / 4);
            const floatx4 vv[4] = {chunk_values<Q8>(vx[i][0]) * fv, chunk_values<Q8>(vx[i][1]) * fv,
                                   chunk_values<Q8>(vx[i][2]) * fv, chunk_values<Q8>(vx[i][3]) * fv};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                unsigned h0, l0, h1, l1;
                split_pair(vv[0][u], vv[1][u], h0, l0);
                split_pair(vv[2][u], vv[3][u], h1, l1);
                const int d = 4 * c4 + u;
                *reinterpret_cast<uint2*>(&t.vh[T::voff(d, vt_keys_off(rq))]) = make_uint2(h0, h1);
                *reinterpret_cast<uint2*>(&t.vl[T::voff(d, vt_keys_off(rq))]) = make_uint2(l0, l1);
            }
        }
    }
}

// Workgroup: KV head blockIdx.y, query tokens [i0, i0 + 16*NB) of its G query heads.  Wave:
// 16 tokens (sub-block sb) x HPW query heads (head group hg), so each K/V fragment read from
// LDS feeds HPW heads' MFMAs.  Tiles [tile0, tile0 + n_tiles) of the layer are in `ws`.
// Waves per SIMD the register allocation must leave room for: with head_dim 64 image tiles
// as many as the LDS lets run at once (two 8-wave workgroups per CU: 4 waves per SIMD, at
// most 128 VGPRs each; key halves: one 16-wave workgroup); other shapes are not constrained.
template <int D, int G, int NB, int HPW, bool DIRECT, int KH>
constexpr int attn_waves_per_eu() {
    if (!(D == 64 && G >= 2 && !DIRECT)) return 1;
    constexpr int waves = KH * (G / HPW) * NB;
    constexpr int per_cu = (160 * 1024) / (2 * KH * (int)sizeof(TileLds<D>));   // LDS-bound
    constexpr int w = per_cu * waves / 4;
    return w < 1 ? 1 : (w > 4 ? 4 : w);
}

template <int D, int G, int NB, int HPW, bool DIRECT = false, bool Q8 = false, int KH = 1>
__global__ __launch_bounds__(KH * (G / HPW) * NB * 64)
__attribute__((amdgpu_waves_per_eu(attn_waves_per_eu<D, G, NB, HPW, DIRECT, KH>())))
void prefill_attn2_kernel(PrefillArgs a,
                                                                            const uint4* ws,
                                                                            int tile0, int n_tiles,
                                                                            int ksplit) {
    using T = TileLds<D, DIRECT ? direct_tile_keys<D>() : tile_keys<D>()>;
    constexpr int HG = G / HPW;
    constexpr int WH = HG * NB;           // waves of one key half
    constexpr int NTHR = WH * 64;         // threads of one key half (all of them when KH = 1)
    constexpr int KS = D / 32, DT = D / 16, TK = T::TK, NKT = TK / 16, NC = TK / 32;
    constexpr int IMG = tile_img_u4<D>();
    constexpr int PER = (IMG + NTHR - 1) / NTHR;
    static_assert(G % HPW == 0, "heads per wave must divide the group");
    static_assert(KH == 1 || (KH == 2 && !DIRECT), "key halves stage tile images");
    __shared__ T buf[2 * KH];

    // KH = 2: two halves of WH waves each take the same queries; half 0 the first half of the
    // item's key tiles, half 1 the second, in lockstep (one barrier per tile pair), each with
    // its own two LDS buffers; half 1 hands its state to half 0 through LDS at the end.  The
    // heaviest query block's chain is halved, with no partials in global memory.
    const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int half = KH == 2 ? wave_all / WH : 0, wave = wave_all - half * WH;
    const int tid = threadIdx.x - half * NTHR;   // thread index within the half
    const int col = lane & 15, grp = lane >> 4;
    const int nblk = (a.P + 16 * NB - 1) / (16 * NB);
    // Grid x: nblk*Hkv items ranked by key count (rank r: block nblk-1-r/Hkv, head r%Hkv).
    // The first half of the grid takes ranks heaviest-first, the second half lightest-first,
    // so the two workgroups a CU holds at once carry about equal total work.  Grid y: split
    // of the item's key tiles (ksplit > 1 writes partials for prefill_combine_kernel).
    // With key halves a workgroup fills a CU alone: plain heaviest-first order, and the
    // dispatcher hands each freed CU the next item.
    // Items run over virtual KV heads vkh (kv_rep per cached KV head kvh): the query heads
    // are vkh's, the key rows and tiles kvh's.
    const int hkv_v = a.Hkv * a.kv_rep;
    const int n_items = nblk * hkv_v, L = (int)blockIdx.x, mid = (n_items + 1) / 2;
    const int rank = KH == 2 ? L : (L < mid ? L : n_items - 1 - (L - mid));
    const int vkh = rank % hkv_v;
    const int kvh = vkh / a.kv_rep;
    const int blk = nblk - 1 - rank / hkv_v;
    const int ks = blockIdx.y;
    const int i0 = blk * 16 * NB;
    const int sb = wave / HG, hg = wave - sb * HG;
    const int qi = i0 + 16 * sb + col;
    const bool q_ok = qi < a.P;
    const int qpos = a.pos0 + (q_ok ? qi : a.P - 1);
    const int qstart = a.window > 0 ? max(0, qpos - a.window + 1) : 0;

    // Key range of the workgroup and of this wave's 16 queries.
    const int last_tok = min(i0 + 16 * NB, a.P) - 1;
    const int kend = a.pos0 + last_tok + 1;
    const int kbeg = a.window > 0 ? max(0, a.pos0 + i0 - a.window + 1) : 0;
    const int t_all0 = kbeg / TK, t_all1 = (kend - 1) / TK;
    const int per = (t_all1 - t_all0 + ksplit) / ksplit;            // tiles per split
    const int t_first = t_all0 + ks * per, t_last = min(t_all1, t_first + per - 1);
    // This half's tiles [tb, tb + nh) and the workgroup's trip count n_iter (half 0's).
    const int n_split = max(0, t_last - t_first + 1);
    const int n_iter = KH == 2 ? (n_split + 1) / 2 : n_split;
    const int tb = t_first + (half ? n_iter : 0);
    const int nh = half ? n_split - n_iter : n_iter;
    const int w_lo = a.pos0 + i0 + 16 * sb;           // first query position of the wave
    const bool w_full = i0 + 16 * sb + 15 < a.P;
    const int w_start_max = a.window > 0 ? max(0, w_lo + 15 - a.window + 1) : 0;

    const uint4* img = ws + (size_t)kvh * n_tiles * IMG;
    const HeadRows kr = k_rows<Q8>(a, kvh), vr = v_rows<Q8>(a, kvh);   // DIRECT staging
    // Range exponents of the head's rows: the tiles hold K * 2^-ek and V * 2^-ev (the images
    // are built scaled; direct staging scales as it splits), restored on the scores and on the
    // output.  Both are 0 unless a stored value reached 2^15.
    const int ek = a.range[2 * kvh], ev = a.range[2 * kvh + 1];
    const float fk = pow2i(-ek), fv = pow2i(-ev);
    using RT = RawTile<D, NTHR, T::TK>;
    u32x4 stage[DIRECT ? 1 : PER];
    floatx4 kx[RT::KI], vx[RT::VI][4];   // used by DIRECT staging only
    // (Always multiplying measured fewer registers than a uniform branch between a scaled and
    // an unscaled copy of the staging.)
    auto stage_direct = [&](auto& dst) {   // generic: instantiated by DIRECT launches only
        raw_store<D, NTHR, RT::KI, RT::VI, Q8, T::TK>(kx, vx, dst, tid, fk, fv);
    };
    floatx4 o[HPW][DT];
    float m[HPW], l[HPW];
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
#pragma unroll
        for (int d = 0; d < DT; ++d) o[hh][d] = floatx4{0.f, 0.f, 0.f, 0.f};
        m[hh] = kNegBig;
        l[hh] = 0.0f;
    }

    // The first tile's loads go out before the query fragments are read and prepared, so the
    // two memory round trips of the prologue overlap.
    const bool has_keys = nh > 0;   // a split past the item's last tile: neutral partial
    T* hbuf = buf + 2 * half;
    if (has_keys) {
        if constexpr (DIRECT)
            raw_load<D, NTHR, RT::KI, RT::VI, Q8, T::TK>(kx, vx, kr, vr, tb * TK, kend - 1, tid);
        else
            img_load<PER, NTHR, IMG>(stage, img + (size_t)(tb - tile0) * IMG, tid);
    }
    f16x8 qh[HPW][KS], ql[HPW][KS];
    // Per query head of the wave: fs = 2^(ek + eq), the factor that restores the scores'
    // scale.  The tiles' scores stay in units of fs (soft-capped ones are divided by it again)
    // and fs is applied where the exponent's argument is formed and to the tile maximum: exact
    // scalings by a power of two, so with ek = eq = 0 every value is bit for bit what it is
    // without the range scaling.
    float fs[HPW];
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
        int eq;
        query_fragment<D>(a, q_ok ? qi : a.P - 1, vkh * G + hg * HPW + hh, qpos, grp, qh[hh], ql[hh], eq);
        fs[hh] = pow2i(min(ek + eq, 127));
    }
    if (has_keys) {
        if constexpr (DIRECT) {
            stage_direct(hbuf[0]);
            if (nh > 1)
                raw_load<D, NTHR, RT::KI, RT::VI, Q8, T::TK>(kx, vx, kr, vr, (tb + 1) * TK, kend - 1, tid);
        } else {
            img_store<PER, NTHR, IMG>(stage, &hbuf[0], tid);
            if (nh > 1) img_load<PER, NTHR, IMG>(stage, img + (size_t)(tb + 1 - tile0) * IMG, tid);
        }
    }
    if (n_iter > 0) __syncthreads();
    for (int it = 0; it < n_iter; ++it) {
      // half 1 sits out the last trip when the split has an odd tile count (still at the barrier)
      if (KH == 1 || it < nh) {
        const int tile = tb + it;
        const T& t = hbuf[it & 1];
        const int t0 = tile * TK;
        // S^T = K Q^T per 16-key sub-tile: lane holds keys 4*grp + j of sub-tile kt.
        floatx4 st[HPW][NKT];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
            floatx4 acc[HPW];
#pragma unroll
            for (int hh = 0; hh < HPW; ++hh) acc[hh] = floatx4{0.f, 0.f, 0.f, 0.f};
            const int krow = kt * 16 + col;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const int ko = T::koff(krow, 32 * s + 8 * grp);
                const f16x8 kh = *reinterpret_cast<const f16x8*>(&t.kh[ko]);
                const f16x8 kl = *reinterpret_cast<const f16x8*>(&t.kl[ko]);
#pragma unroll
                for (int hh = 0; hh < HPW; ++hh) {
                    acc[hh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[hh][s], acc[hh], 0, 0, 0);
                    acc[hh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[hh][s], acc[hh], 0, 0, 0);
                    acc[hh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[hh][s], acc[hh], 0, 0, 0);
                }
            }
#pragma unroll
            for (int hh = 0; hh < HPW; ++hh) st[hh][kt] = acc[hh];
        }
        // Soft-cap; causal/window/range mask only on tiles that cross a boundary of this wave.
        if (a.softcap > 0.0f) {
#pragma unroll
            for (int hh = 0; hh < HPW; ++hh) {
                const float isc = a.inv_softcap * fs[hh], rfs = pow2_inv(fs[hh]);
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        st[hh][kt][j] = (a.softcap_log2e * tanhf(st[hh][kt][j] * isc)) * rfs;
            }
        }
        const bool interior = w_full && t0 + TK - 1 <= w_lo && t0 >= w_start_max;
        if (!interior) {
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int key = t0 + kt * 16 + 4 * grp + j;
                    const bool ok = q_ok && key <= qpos && key >= qstart && key < kend;
#pragma unroll
                    for (int hh = 0; hh < HPW; ++hh)
                        st[hh][kt][j] = ok ? st[hh][kt][j] : -__builtin_inff();
                }
        }
#pragma unroll
        for (int hh = 0; hh < HPW; ++hh) {
            float mt = kNegBig;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                for (int j = 0; j < 4; ++j) mt = fmaxf(mt, st[hh][kt][j]);
            mt = dk::lane_step<16, true>(mt);
            mt = dk::lane_step<32, true>(mt);
            mt = mt * fs[hh];
            // Rescaled on every tile, with no branch: alpha is exactly 1 where the running max
            // did not grow.  A branch on "some row grew" split the loop body into blocks the
            // scheduler could not interleave (C5 P = 2048: 86.2 -> 84.0 us per call; 16-token
            // verification at 32k: 72.4 -> 67.6 us).
            {
                const float mn = fmaxf(m[hh], mt);
                const float alpha = dk::fast_exp2(m[hh] - mn);
                m[hh] = mn;
                l[hh] = l[hh] * alpha;
#pragma unroll
                for (int d = 0; d < DT; ++d) o[hh][d] = o[hh][d] * alpha;
            }
            const float mn = m[hh];
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float p = dk::fast_exp2(__builtin_fmaf(st[hh][kt][j], fs[hh], -mn));
                    l[hh] = l[hh] + p;
                    st[hh][kt][j] = p;
                }
        }
        // O^T += V^T P^T: B operand = P in the key order {32c+4grp..+3, 32c+16+4grp..+3}.
        // Tiles whose V lo parts are all within 2^-24 (rows written from bf16 inputs) skip the
        // V-lo MFMA and its LDS reads.  Direct staging does not flag its tiles.
        const bool tile_vlo =
            DIRECT || __builtin_amdgcn_readfirstlane(t.flag[0]) != 0;
        auto pv = [&](auto has_lo) {
            constexpr bool HL = decltype(has_lo)::value;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            f16x8 ph[HPW], pl[HPW];
#pragma unroll
            for (int hh = 0; hh < HPW; ++hh) {
                unsigned h0, l0, h1, l1, h2, l2, h3, l3;
                split_pair(st[hh][2 * c][0], st[hh][2 * c][1], h0, l0);
                split_pair(st[hh][2 * c][2], st[hh][2 * c][3], h1, l1);
                split_pair(st[hh][2 * c + 1][0], st[hh][2 * c + 1][1], h2, l2);
                split_pair(st[hh][2 * c + 1][2], st[hh][2 * c + 1][3], h3, l3);
                ph[hh] = __builtin_bit_cast(f16x8, make_uint4(h0, h1, h2, h3));
                pl[hh] = __builtin_bit_cast(f16x8, make_uint4(l0, l1, l2, l3));
            }
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                const int dim = d * 16 + col;
                const int k0 = 32 * c + 8 * grp;   // keys {32c+4grp..+3, 32c+16+4grp..+3}
                const int vo = T::voff(dim, k0);
                const f16x8 vh = *reinterpret_cast<const f16x8*>(&t.vh[vo]);
#pragma unroll
                for (int hh = 0; hh < HPW; ++hh) {
                    o[hh][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph[hh], o[hh][d], 0, 0, 0);
                    o[hh][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl[hh], o[hh][d], 0, 0, 0);
                }
                if constexpr (HL) {
                    const f16x8 vl = *reinterpret_cast<const f16x8*>(&t.vl[vo]);
#pragma unroll
                    for (int hh = 0; hh < HPW; ++hh)
                        o[hh][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph[hh], o[hh][d], 0, 0, 0);
                }
            }
        }
        };
        if (tile_vlo) pv(std::true_type{});
        else pv(std::false_type{});
        // Next buffer: tile+1 (already in registers) to LDS, tile+2 loads in flight.  The
        // buffer written here was last read before the previous iteration's barrier.
        if (it + 1 < nh) {
            if constexpr (DIRECT) {
                stage_direct(hbuf[(it + 1) & 1]);
                if (it + 2 < nh)
                    raw_load<D, NTHR, RT::KI, RT::VI, Q8, T::TK>(kx, vx, kr, vr, (tile + 2) * TK, kend - 1, tid);
            } else {
                img_store<PER, NTHR, IMG>(stage, &hbuf[(it + 1) & 1], tid);
                if (it + 2 < nh)
                    img_load<PER, NTHR, IMG>(stage, img + (size_t)(tile + 2 - tile0) * IMG, tid);
            }
        }
      }
        __syncthreads();
    }
    if constexpr (KH == 2) {
        // Half 1's state (m, l per lane, o) to half 0 through the tile buffers, whose last
        // reads ended at the loop's final barrier; half 0 merges it into its own.
        constexpr int XS = HPW * (2 + 4 * DT);   // floats per lane
        static_assert((size_t)WH * 64 * XS * sizeof(float) <= sizeof(buf), "exchange fits the tiles");
        float* xch = reinterpret_cast<float*>(&buf[0]) + (size_t)(wave * 64 + lane) * XS;
        if (half == 1) {
#pragma unroll
            for (int hh = 0; hh < HPW; ++hh) {
                xch[hh * (2 + 4 * DT)] = m[hh];
                xch[hh * (2 + 4 * DT) + 1] = l[hh];
#pragma unroll
                for (int d = 0; d < DT; ++d)
#pragma unroll
                    for (int j = 0; j < 4; ++j) xch[hh * (2 + 4 * DT) + 2 + 4 * d + j] = o[hh][d][j];
            }
        }
        __syncthreads();
        if (half == 1) return;
#pragma unroll
        for (int hh = 0; hh < HPW; ++hh) {
            const float mb = xch[hh * (2 + 4 * DT)], lb = xch[hh * (2 + 4 * DT) + 1];
            const float mn = fmaxf(m[hh], mb);
            const float sa = dk::fast_exp2(m[hh] - mn), sb2 = dk::fast_exp2(mb - mn);
            l[hh] = __builtin_fmaf(l[hh], sa, lb * sb2);
#pragma unroll
            for (int d = 0; d < DT; ++d)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    o[hh][d][j] = __builtin_fmaf(o[hh][d][j], sa, xch[hh * (2 + 4 * DT) + 2 + 4 * d + j] * sb2);
            m[hh] = mn;
        }
    }
    const float fvs = pow2i(ev);   // V's range factor, restored on the output (exact)
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
        float lt = dk::lane_step<16, false>(l[hh]);
        lt = dk::lane_step<32, false>(lt);
        if (q_ok && ksplit > 1) {
            // Unnormalised partial of split ks: o for this lane's dims, (max, sum) per row.
            const int hq = vkh * G + hg * HPW + hh;
            const long long slot = ((long long)ks * a.P + qi) * a.Hq + hq;
#pragma unroll
            for (int d = 0; d < DT; ++d)
                *reinterpret_cast<float4*>(a.part_o + slot * D + d * 16 + 4 * grp) =
                    make_float4(o[hh][d][0] * fvs, o[hh][d][1] * fvs, o[hh][d][2] * fvs,
                                o[hh][d][3] * fvs);
            if (grp == 0) *reinterpret_cast<float2*>(a.part_ml + 2 * slot) = make_float2(m[hh], lt);
        } else if (q_ok) {
            const int hq = vkh * G + hg * HPW + hh;
            const long long row = (long long)qi * a.Hq * D + (long long)hq * D;
            float* op = a.out + row;
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                const int d0 = d * 16 + 4 * grp;
                float4 r;
                r.x = dk::finish_output(m[hh], lt, o[hh][d][0], a.sinks, a.gate, hq, row + d0) * fvs;
                r.y = dk::finish_output(m[hh], lt, o[hh][d][1], a.sinks, a.gate, hq, row + d0 + 1) * fvs;
                r.z = dk::finish_output(m[hh], lt, o[hh][d][2], a.sinks, a.gate, hq, row + d0 + 2) * fvs;
                r.w = dk::finish_output(m[hh], lt, o[hh][d][3], a.sinks, a.gate, hq, row + d0 + 3) * fvs;
                reinterpret_cast<float4*>(op + d0)[0] = r;
            }
        }
    }
}


// ---- 4. Split-K combine -------------------------------------------------------------------------
// One block per (token, query head) row.  Thread (column c, split group p) owns float4 column
// c of the row for the splits p, p + NP, ...; its loads are independent of the running max,
// so they are all in flight together.  The NP group results merge through LDS, then sinks and
// the output gate apply (the same merge as decode_reduce_kernel).
constexpr int kCombineThreads = 256;

template <int D>
__global__ __launch_bounds__(kCombineThreads) void prefill_combine_kernel(PrefillArgs a,
                                                                          int ksplit) {
    constexpr int NC = D / 4, NP = kCombineThreads / NC;
    __shared__ float s_m[NP], s_l[NP];
    __shared__ float4 s_o[NP][NC];
    const long long rows = (long long)a.P * a.Hq;
    const long long row = blockIdx.x;                 // token * Hq + head
    const int tid = threadIdx.x, c = tid % NC, p = tid / NC;
    const bool act = p < NP;   // NC need not divide the block: the spare threads only sync
    const int hq = (int)(row % a.Hq);
    float m = kNegBig, l = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
    for (int s = p; s < ksplit; s += NP) {
        const long long slot = (long long)s * rows + row;
        const float2 ml = *reinterpret_cast<const float2*>(a.part_ml + 2 * slot);
        const float4 x = reinterpret_cast<const float4*>(a.part_o + slot * D)[c];
        const float mn = fmaxf(m, ml.x);
        const float so = dk::fast_exp2(m - mn), sx = dk::fast_exp2(ml.x - mn);
        l = __builtin_fmaf(l, so, ml.y * sx);
        o.x = __builtin_fmaf(o.x, so, x.x * sx);
        o.y = __builtin_fmaf(o.y, so, x.y * sx);
        o.z = __builtin_fmaf(o.z, so, x.z * sx);
        o.w = __builtin_fmaf(o.w, so, x.w * sx);
        m = mn;
    }
    if (act && c == 0) {
        s_m[p] = m;
        s_l[p] = l;
    }
    if (act) s_o[p][c] = o;
    __syncthreads();
    if (p == 0) {
        float M = s_m[0];
        for (int q = 1; q < NP; ++q) M = fmaxf(M, s_m[q]);
        float L = 0.0f;
        float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int q = 0; q < NP; ++q) {
            const float sc = dk::fast_exp2(s_m[q] - M);
            L = __builtin_fmaf(s_l[q], sc, L);
            const float4 x = s_o[q][c];
            O.x = __builtin_fmaf(x.x, sc, O.x);
            O.y = __builtin_fmaf(x.y, sc, O.y);
            O.z = __builtin_fmaf(x.z, sc, O.z);
            O.w = __builtin_fmaf(x.w, sc, O.w);
        }
        const long long g0 = row * D + 4 * c;
        float4 r;
        r.x = dk::finish_output(M, L, O.x, a.sinks, a.gate, hq, g0);
        r.y = dk::finish_output(M, L, O.y, a.sinks, a.gate, hq, g0 + 1);
        r.z = dk::finish_output(M, L, O.z, a.sinks, a.gate, hq, g0 + 2);
        r.w = dk::finish_output(M, L, O.w, a.sinks, a.gate, hq, g0 + 3);
        reinterpret_cast<float4*>(a.out + row * D)[c] = r;
    }
}

}  // namespace pk
}  // namespace llmp
