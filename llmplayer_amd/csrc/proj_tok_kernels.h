// Projections of up to 16 tokens at once on the matrix cores (the attention half of a layer for
// K tokens: speculative verification and batched forwards, LLMEngine.forwardBatch at
// LLMEngine.java:1019-1033; the plan in docs/optimization/speculative-decoding.md:120-140 reads
// each weight row once for all K tokens).
//
// One token's projection is a matrix-vector product bound by issue (gemv_kernels.h).  K tokens
// make it a skinny matrix product Y[t][r] = sum_c W[r][c] x_t[c], which runs on
// v_mfma_f32_16x16x32_f16 with the rows as M, the tokens as N (padded to 16) and the columns
// as the reduction:
//
//  - A (weights): the quantised integers exactly (Q4_K nibbles, Q6_K 6-bit values minus 32,
//    Q8_0 int8, Q4_0 nibbles minus 8 are all exact in fp16), the per-block scales applied to
//    the fp32 product of each 32-column group afterwards (Q4_K: d*sc * sum(q x) - dmin*m *
//    sum(x), the tensor classes' per-element values summed per block).  F16 weights are exact;
//    BF16 weights are exact within fp16's normal range; F32 weights are two fp16 parts.
//  - B (inputs): each fp32 input is split into two fp16 parts x = hi + lo, which holds x to
//    ~2^-22 of its magnitude, so every product is fp32-accurate and the result matches the CPU
//    path to the tolerance of a reordered fp32 sum.  fp16 holds magnitudes below 65504, so the
//    launch scales its inputs by 2^-E, E the range exponent of the largest input of its tokens
//    (0 for inputs below 2^15), and its outputs by 2^E (exact scalings; E is uniform, so the
//    factor stays in scalar registers, and with a norm it rides on the staged norm weights).
//
// The pre-attention RMSNorm is folded in: a small first kernel (tok_prep_kernel) computes each
// token's factor r = 1/sqrt(sum(x^2)/cols + eps) and the range exponent of its largest x*w; the
// projection multiplies the raw inputs by the norm weights and its outputs by r after the
// reduction (W (r x*w) = r (W x*w), one rounding apart from the CPU path's (x*r)*w).  Without
// a norm the exponent comes from the same kernel (the raw residual of a layer with no pre-norm)
// or from the layer's V range exponents (the output projection's input, the attention output,
// is a convex combination of V rows).
//
// A workgroup owns 16 rows and all tokens; its 8 waves take 128-column chunks in turn and keep
// the next chunk's weight and input loads in flight while they compute the current one; their
// partial tiles and sums of squares are merged through LDS.  The norm weights are staged in LDS
// once per workgroup (in registers they would double the prefetch buffers and halve occupancy).  Rows of two formats (the Q4_K_M
// mix: Q4_K q and k, Q6_K v) run in one launch, each workgroup on its rows' format.
//
// Layout facts of v_mfma_f32_16x16x32_f16 (as in prefill_kernels.h): lane l holds
// A[l%16][8*(l/16)+j], B[8*(l/16)+j][l%16] (j < 8) and D[4*(l/16)+j][l%16] (j < 4).
#pragma once

#include "gemv_kernels.h"

namespace llmp {
namespace tk {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTok = 16;                 // tokens per launch (the MFMA's N)
constexpr int kWaves = 8;                // waves per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kChunk = 128;              // columns per wave step (4 groups of 32)
constexpr int kGroups = kChunk / 32;

using gk::WPlanes;
using gk::rp;
using gk::ldo;
using gk::h2f;
using gk::bf2f;
using gk::u32x4;

struct TokSeg {
    WPlanes w;
    int rows;              // rows of this segment (a multiple of 16)
    int out_off;           // first row of this segment in the launch
    int fmt;               // launches over two formats: 0 = the first, 1 = the second
    const float* bias;     // [rows] or nullptr
    float* out;            // [K][out_pitch] outputs of this segment (when resid is null)
    long long out_pitch;
};

struct ProjTokArgs {
    TokSeg seg[3];
    int nseg;
    int rows_total;        // sum of the segments' rows (a multiple of 16)
    int cols;              // a multiple of 32
    int K;                 // tokens, 1..16
    const float* x;        // inputs [K][x_pitch] fp32 (16-byte aligned rows)
    long long x_pitch;
    const float* norm_w;   // pre-norm weights [cols] (RMSNorm of each input row), or nullptr
    // Per token t (tok_prep_kernel): tok_sc[2t] = r, the RMSNorm factor applied to the outputs
    // (with norm_w), and tok_sc[2t + 1] = e_t, the range exponent of its largest input (an
    // integer in a float); E = max e_t.  When null, E is the largest V range exponent of
    // in_range ([in_range_n][K, V] ints), or 0 when in_range is null too.
    const float* tok_sc;
    const int* in_range;
    int in_range_n;
    float eps;
    float* resid;          // Wo epilogue: resid[t*resid_pitch + row] += rscale? * value
    long long resid_pitch;
    float rscale;          // Granite residual scale, 0 = off
    // The Q8_1 input of the int8 formats (Q8In<...>, tok_q8_kernel): per 32-column group g and
    // lane l = 16 kq + t, q8b[64 g + l] = the 8 quants of token t at columns 32 g + 8 kq .. +7
    // as fp16, q8d[16 g + t] / q8s[16 g + t] the block's scale and sum.
    const uint4* q8b;
    const float* q8d;
    const float* q8s;
};

// Two fp32 values -> packed fp16, round to nearest even (v_cvt_pk_f16_f32).
__device__ __forceinline__ unsigned pk_f16(float x, float y) {
    return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2_t{x, y}, f16x2_t));
}
__device__ __forceinline__ f16x8_t as_f8(const uint4& u) { return __builtin_bit_cast(f16x8_t, u); }
// Eight values that fp16 holds exactly (small integers) -> one A operand.
__device__ __forceinline__ uint4 f16x8_of(const float (&v)[8]) {
    return make_uint4(pk_f16(v[0], v[1]), pk_f16(v[2], v[3]), pk_f16(v[4], v[5]), pk_f16(v[6], v[7]));
}
// hi = fp16(v), lo = fp16(v - hi).  Each lo half comes from one mixed-precision FMA,
// hi(f16) * -1 + v(f32), which forms the difference exactly and rounds it once to fp16 into
// its half of the register (the bits of rounding the exact fp32 difference, 3 instructions per
// pair instead of 6).
__device__ __forceinline__ void split8(const float (&v)[8], uint4& hi, uint4& lo) {
    unsigned h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        h[e] = pk_f16(v[2 * e], v[2 * e + 1]);
        unsigned r;
        asm("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h[e]), "v"(v[2 * e]));
        asm("v_fma_mixhi_f16 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
            : "+v"(r) : "v"(h[e]), "v"(v[2 * e + 1]));
        l[e] = r;
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// ---- weight formats -------------------------------------------------------------------------
// For a 128-column chunk `ch` of A row `row` (lane m = l%16 of the tile) and k-quad kq = l/16,
// a format loads its raw bytes (Raw), writes the chunk's per-row scale factors to the wave's
// LDS table (row m, its own entries), and for group gi < 4 of the chunk builds its A operands
// (NA of them: the exact fp16 integers or parts); `pairs` names the MFMAs (A part, input part)
// it issues.  With TAB > 0 the products of A part 0 (and part 1, Q6_K) are scaled per group
// from the table, for output rows 4*(l/16)+i.
struct PartPair {
    int a, b;
};

// A format on the Q8_1 input (LLMP_INPUT_Q8_1: the reference GPU's int8 matvecs,
// CudaForwardPass.java:216-226, 1998-2037): the same weight integers as its A operand, the
// token's int8 quants (exact in fp16) as the B operand, one MFMA per A part giving the exact
// integer dot of each 32-value block (16 for the halves formats), scaled as the reference's
// dp4a kernels do: ((d*sc) * d_x) * dot - (dmin*m) * s_x per block (the min term for Q4_K and
// Q5_K), (d_s * d_x) * dot per block or half otherwise.
template <class P>
struct Q8In : P {
    static constexpr bool Q8B = true;
};
template <class F, class = void>
struct IsQ8B {
    static constexpr bool value = false;
};
template <class F>
struct IsQ8B<F, std::void_t<decltype(F::Q8B)>> {
    static constexpr bool value = F::Q8B;
};

// Q4_K: chunk = half a super-block (sub-blocks 4h..4h+3, h = ch%2): nibble bytes 64h + 32p +
// 8kq (p = 0, 1: the two 32-byte runs, low nibbles = sub-block 4h+2p, high = 4h+2p+1) and the
// super-block's 16-byte head.  Table per row: (d*sc_s, dmin*m_s) for the chunk's 4 sub-blocks.
struct PQ4K {
    static constexpr int NA = 1, NPAIR = 2, TAB = 8;
    static constexpr bool MIN = true, HALVES = false;
    static constexpr PartPair pairs[2] = {{0, 0}, {0, 1}};
    struct Raw { uint2 q[2]; u32x4 h; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int) {
        const int sb = ch >> 1, h = ch & 1;
        const unsigned char* qp = rp(w, 0, row);
        r.q[0] = ldo<uint2>(qp, (unsigned)(sb * 128 + 64 * h + 8 * kq));
        r.q[1] = ldo<uint2>(qp, (unsigned)(sb * 128 + 64 * h + 32 + 8 * kq));
        r.h = ldo<u32x4>(rp(w, 1, row), (unsigned)sb * 16u);
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int ch) {
        // sub-block s = 4h + kq of this row
        const int s = 4 * (ch & 1) + kq;
        const float d = h2f((unsigned short)(r.h[0] & 0xFFFF));
        const float dmin = h2f((unsigned short)(r.h[0] >> 16));
        int sc, mn;
        auto byte_of = [&](int i) { return (int)((r.h[i >> 2] >> (8 * (i & 3))) & 0xFF); };
        if (s < 4) {
            sc = byte_of(4 + s) & 63;
            mn = byte_of(8 + s) & 63;
        } else {
            sc = (byte_of(8 + s) & 15) | ((byte_of(s) >> 6) << 4);
            mn = (byte_of(8 + s) >> 4) | ((byte_of(4 + s) >> 6) << 4);
        }
        reinterpret_cast<float2*>(tab + m * TAB)[kq] = make_float2(d * (float)sc, dmin * (float)mn);
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int) {
        const uint2 q = r.q[gi >> 1];
        const int sh = 4 * (gi & 1);
        const unsigned u0 = (q.x >> sh) & 0x0F0F0F0Fu, u1 = (q.y >> sh) & 0x0F0F0F0Fu;
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = (float)((u0 >> (8 * e)) & 0xFF);
            v[4 + e] = (float)((u1 >> (8 * e)) & 0xFF);
        }
        a[0] = f16x8_of(v);
    }
};

// Q6_K: chunk = half h = ch%2 of a super-block (quarters c = 0..3 of 32 columns): ql words at
// 64h + 8kq and 64h + 32 + 8kq, qh word at 32h + 8kq, scales sc[8h .. 8h+7], d.  Group gi =
// quarter c: values (nibble of ql[(c&1)] at 4*(c>>1)) | (qh bits 2c..2c+1) << 4, minus 32.
// Columns 0-15 and 16-31 of a quarter have their own scales, so the A operand goes out twice,
// each time with the other half zeroed.  Table per row: d*sc for the chunk's 8 sub-blocks of
// 16.
struct PQ6K {
    static constexpr int NA = 2, NPAIR = 4, TAB = 8;
    static constexpr bool MIN = false, HALVES = true;
    static constexpr PartPair pairs[4] = {{0, 0}, {0, 1}, {1, 0}, {1, 1}};
    struct Raw { uint2 ql[2]; uint2 qh; uint2 sc; unsigned short d; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int) {
        const int sb = ch >> 1, h = ch & 1;
        const unsigned char* ql = rp(w, 0, row);
        r.ql[0] = ldo<uint2>(ql, (unsigned)(sb * 128 + 64 * h + 8 * kq));
        r.ql[1] = ldo<uint2>(ql, (unsigned)(sb * 128 + 64 * h + 32 + 8 * kq));
        r.qh = ldo<uint2>(rp(w, 1, row), (unsigned)(sb * 64 + 32 * h + 8 * kq));
        r.sc = ldo<uint2>(rp(w, 2, row), (unsigned)(sb * 16 + 8 * h));
        r.d = ldo<unsigned short>(rp(w, 3, row), (unsigned)sb * 2u);
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int) {
        const float d = h2f(r.d);
        const unsigned wv = kq < 2 ? r.sc.x : r.sc.y;
        const int i0 = 2 * (kq & 1);
        const float a0 = d * (float)(signed char)((wv >> (8 * i0)) & 0xFF);
        const float a1 = d * (float)(signed char)((wv >> (8 * (i0 + 1))) & 0xFF);
        reinterpret_cast<float2*>(tab + m * TAB)[kq] = make_float2(a0, a1);
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int kq) {
        const uint2 l = r.ql[gi & 1];
        const int sh = 4 * (gi >> 1);
        const unsigned n0 = (l.x >> sh) & 0x0F0F0F0Fu, n1 = (l.y >> sh) & 0x0F0F0F0Fu;
        const unsigned h0 = ((r.qh.x >> (2 * gi)) & 0x03030303u) << 4;
        const unsigned h1 = ((r.qh.y >> (2 * gi)) & 0x03030303u) << 4;
        const unsigned q0 = n0 | h0, q1 = n1 | h1;
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = (float)((int)((q0 >> (8 * e)) & 0xFF) - 32);
            v[4 + e] = (float)((int)((q1 >> (8 * e)) & 0xFF) - 32);
        }
        const uint4 u = f16x8_of(v);
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
        a[0] = kq < 2 ? u : z;   // columns 0-15: sub-block 2c
        a[1] = kq < 2 ? z : u;   // columns 16-31: sub-block 2c + 1
    }
};

// Q8_0: chunk = 4 blocks of 32: quants at 32b + 8kq, scales d (fp16) of the 4 blocks.
struct PQ8_0 {
    static constexpr int NA = 1, NPAIR = 2, TAB = 4;
    static constexpr bool MIN = false, HALVES = false;
    static constexpr PartPair pairs[2] = {{0, 0}, {0, 1}};
    struct Raw { uint2 q[4]; unsigned short d; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
        const unsigned char* qp = rp(w, 0, row);
#pragma unroll
        for (int b = 0; b < 4; ++b)
            r.q[b] = ldo<uint2>(qp, (unsigned)(ch * 128 + 32 * min(b, ng - 1) + 8 * kq));
        r.d = ldo<unsigned short>(rp(w, 1, row), (unsigned)(ch * 4 + min(kq, ng - 1)) * 2u);
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int) {
        tab[m * TAB + kq] = h2f(r.d);
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int) {
        const uint2 q = r.q[gi];
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = (float)(int)(signed char)((q.x >> (8 * e)) & 0xFF);
            v[4 + e] = (float)(int)(signed char)((q.y >> (8 * e)) & 0xFF);
        }
        a[0] = f16x8_of(v);
    }
};

// Q4_0 (the reference's interleave: element 2i low nibble of byte i, 2i+1 high): chunk = 4
// blocks of 16 bytes; lane kq takes bytes 4kq .. 4kq+3 of a block (elements 8kq .. 8kq+7).
struct PQ4_0 {
    static constexpr int NA = 1, NPAIR = 2, TAB = 4;
    static constexpr bool MIN = false, HALVES = false;
    static constexpr PartPair pairs[2] = {{0, 0}, {0, 1}};
    struct Raw { unsigned q[4]; unsigned short d; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
        const unsigned char* qp = rp(w, 0, row);
#pragma unroll
        for (int b = 0; b < 4; ++b)
            r.q[b] = ldo<unsigned>(qp, (unsigned)(ch * 64 + 16 * min(b, ng - 1) + 4 * kq));
        r.d = ldo<unsigned short>(rp(w, 1, row), (unsigned)(ch * 4 + min(kq, ng - 1)) * 2u);
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int) {
        tab[m * TAB + kq] = h2f(r.d);
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int) {
        const unsigned q = r.q[gi];
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const unsigned b = (q >> (8 * e)) & 0xFF;
            v[2 * e] = (float)((int)(b & 15) - 8);
            v[2 * e + 1] = (float)((int)(b >> 4) - 8);
        }
        a[0] = f16x8_of(v);
    }
};

// Split-nibble 32-blocks (Q5_0, IQ4_NL, MXFP4; gemv_kernels.h): chunk = 4 blocks; lane kq
// takes columns 8kq .. 8kq+7 of each, the low (kq < 2) or high (kq >= 2) nibbles of bytes
// 8(kq%2) .. 8(kq%2)+7.  The nibble pair of those 8 bytes.
__device__ __forceinline__ void split_codes(const uint2& q, int kq, unsigned& c0, unsigned& c1) {
    const int sh = 4 * (kq >> 1);
    c0 = (q.x >> sh) & 0x0F0F0F0Fu;
    c1 = (q.y >> sh) & 0x0F0F0F0Fu;
}
// Eight signed bytes (int8 values, exact in fp16) -> one A operand.
__device__ __forceinline__ uint4 f16x8_of_s8(unsigned c0, unsigned c1) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        v[e] = gk::sbyte_f(c0, e);
        v[4 + e] = gk::sbyte_f(c1, e);
    }
    return f16x8_of(v);
}

// Q5_0: values q - 16 with the fifth bit of element e at bit e of the block's qh word (for
// lane kq: bits 8kq .. 8kq+7, low or high nibbles alike).  Table: d of block kq.
struct PQ5_0 {
    static constexpr int NA = 1, NPAIR = 2, TAB = 4;
    static constexpr bool MIN = false, HALVES = false;
    static constexpr PartPair pairs[2] = {{0, 0}, {0, 1}};
    struct Raw { uint2 q[4]; unsigned qh[4]; unsigned short d; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int blk = ch * 4 + min(b, ng - 1);
            r.q[b] = ldo<uint2>(rp(w, 0, row), (unsigned)(blk * 16 + 8 * (kq & 1)));
            r.qh[b] = ldo<unsigned>(rp(w, 1, row), (unsigned)blk * 4u);
        }
        r.d = ldo<unsigned short>(rp(w, 2, row), (unsigned)(ch * 4 + min(kq, ng - 1)) * 2u);
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int) {
        tab[m * TAB + kq] = h2f(r.d);
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int kq) {
        unsigned c0, c1;
        split_codes(r.q[gi], kq, c0, c1);
        const unsigned h = r.qh[gi] >> (8 * kq);
        c0 = (c0 | (gk::spread4(h & 15u) << 4)) ^ 0x10101010u;          // q ^ 16: 5-bit q - 16
        c1 = (c1 | (gk::spread4((h >> 4) & 15u) << 4)) ^ 0x10101010u;
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = (float)((int)(c0 << (27 - 8 * e)) >> 27);
            v[4 + e] = (float)((int)(c1 << (27 - 8 * e)) >> 27);
        }
        a[0] = f16x8_of(v);
    }
};

// Q5_1: values q (0..31) with the fifth bits as Q5_0's; value q * d + m, so the group's input
// sum carries the min: table (d, -m) of block kq (the MIN path adds f.x * t0 - f.y * gs).
struct PQ5_1 {
    static constexpr int NA = 1, NPAIR = 2, TAB = 8;
    static constexpr bool MIN = true, HALVES = false;
    static constexpr PartPair pairs[2] = {{0, 0}, {0, 1}};
    struct Raw { uint2 q[4]; unsigned qh[4]; unsigned short d, m; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int blk = ch * 4 + min(b, ng - 1);
            r.q[b] = ldo<uint2>(rp(w, 0, row), (unsigned)(blk * 16 + 8 * (kq & 1)));
            r.qh[b] = ldo<unsigned>(rp(w, 1, row), (unsigned)blk * 4u);
        }
        const unsigned bk = (unsigned)(ch * 4 + min(kq, ng - 1)) * 2u;
        r.d = ldo<unsigned short>(rp(w, 2, row), bk);
        r.m = ldo<unsigned short>(rp(w, 3, row), bk);
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int) {
        reinterpret_cast<float2*>(tab + m * TAB)[kq] = make_float2(h2f(r.d), -h2f(r.m));
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int kq) {
        unsigned c0, c1;
        split_codes(r.q[gi], kq, c0, c1);
        const unsigned h = r.qh[gi] >> (8 * kq);
        c0 |= gk::spread4(h & 15u) << 4;
        c1 |= gk::spread4((h >> 4) & 15u) << 4;
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = (float)((c0 >> (8 * e)) & 0xFFu);
            v[4 + e] = (float)((c1 >> (8 * e)) & 0xFFu);
        }
        a[0] = f16x8_of(v);
    }
};

// IQ4_NL: values codebook[code].  Table: d of block kq.
struct PIQ4_NL {
    static constexpr int NA = 1, NPAIR = 2, TAB = 4;
    static constexpr bool MIN = false, HALVES = false;
    static constexpr PartPair pairs[2] = {{0, 0}, {0, 1}};
    struct Raw { uint2 q[4]; unsigned short d; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
#pragma unroll
        for (int b = 0; b < 4; ++b)
            r.q[b] = ldo<uint2>(rp(w, 0, row), (unsigned)((ch * 4 + min(b, ng - 1)) * 16 + 8 * (kq & 1)));
        r.d = ldo<unsigned short>(rp(w, 1, row), (unsigned)(ch * 4 + min(kq, ng - 1)) * 2u);
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int) {
        tab[m * TAB + kq] = h2f(r.d);
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int kq) {
        unsigned c0, c1;
        split_codes(r.q[gi], kq, c0, c1);
        using gk::kIq4;
        a[0] = f16x8_of_s8(gk::lut16(c0, kIq4[0], kIq4[1], kIq4[2], kIq4[3]),
                           gk::lut16(c1, kIq4[0], kIq4[1], kIq4[2], kIq4[3]));
    }
};

// MXFP4: values 2 FP4[code] (integers), table 2^(e - 128) of block kq.
struct PMXFP4 {
    static constexpr int NA = 1, NPAIR = 2, TAB = 4;
    static constexpr bool MIN = false, HALVES = false;
    static constexpr PartPair pairs[2] = {{0, 0}, {0, 1}};
    struct Raw { uint2 q[4]; unsigned char e; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
#pragma unroll
        for (int b = 0; b < 4; ++b)
            r.q[b] = ldo<uint2>(rp(w, 0, row), (unsigned)((ch * 4 + min(b, ng - 1)) * 16 + 8 * (kq & 1)));
        r.e = ldo<unsigned char>(rp(w, 1, row), (unsigned)(ch * 4 + min(kq, ng - 1)));
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int) {
        tab[m * TAB + kq] = gk::e8m0_half(r.e);
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int kq) {
        unsigned c0, c1;
        split_codes(r.q[gi], kq, c0, c1);
        using gk::kFp4x2;
        a[0] = f16x8_of_s8(gk::lut16(c0, kFp4x2[0], kFp4x2[1], kFp4x2[2], kFp4x2[3]),
                           gk::lut16(c1, kFp4x2[0], kFp4x2[1], kFp4x2[2], kFp4x2[3]));
    }
};

// IQ4_XS: chunk = 4 sub-blocks of 32 (their nibbles are consecutive 16-byte runs, split as the
// 32-blocks); values codebook[code], table d * (ls - 32) of sub-block kq.
struct PIQ4_XS {
    static constexpr int NA = 1, NPAIR = 2, TAB = 4;
    static constexpr bool MIN = false, HALVES = false;
    static constexpr PartPair pairs[2] = {{0, 0}, {0, 1}};
    struct Raw { uint2 q[4]; unsigned char sc; unsigned short d; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
#pragma unroll
        for (int b = 0; b < 4; ++b)
            r.q[b] = ldo<uint2>(rp(w, 0, row), (unsigned)((ch * 4 + min(b, ng - 1)) * 16 + 8 * (kq & 1)));
        const int sbk = ch * 4 + min(kq, ng - 1);
        r.sc = ldo<unsigned char>(rp(w, 1, row), (unsigned)sbk);
        r.d = ldo<unsigned short>(rp(w, 2, row), (unsigned)(sbk >> 3) * 2u);
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int) {
        tab[m * TAB + kq] = h2f(r.d) * (float)(int)(signed char)r.sc;
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int kq) {
        unsigned c0, c1;
        split_codes(r.q[gi], kq, c0, c1);
        using gk::kIq4;
        a[0] = f16x8_of_s8(gk::lut16(c0, kIq4[0], kIq4[1], kIq4[2], kIq4[3]),
                           gk::lut16(c1, kIq4[0], kIq4[1], kIq4[2], kIq4[3]));
    }
};

// Q5_K: PQ4K's chunk with the fifth bits: qh bytes 8kq .. 8kq+7 of the super-block, bit 4h + gi
// for group gi (sub-block 4h + gi) of chunk half h.
struct PQ5K {
    static constexpr int NA = 1, NPAIR = 2, TAB = 8;
    static constexpr bool MIN = true, HALVES = false;
    static constexpr PartPair pairs[2] = {{0, 0}, {0, 1}};
    struct Raw { PQ4K::Raw q4; uint2 qh; int h; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
        PQ4K::load(r.q4, w, row, ch, kq, ng);
        r.qh = ldo<uint2>(rp(w, 2, row), (unsigned)((ch >> 1) * 32 + 8 * kq));
        r.h = ch & 1;
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int ch) {
        PQ4K::table(r.q4, tab, m, kq, ch);
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int) {
        const uint2 q = r.q4.q[gi >> 1];
        const int sh = 4 * (gi & 1), hb = 4 * r.h + gi;
        const unsigned u0 = ((q.x >> sh) & 0x0F0F0F0Fu) | (((r.qh.x >> hb) & 0x01010101u) << 4);
        const unsigned u1 = ((q.y >> sh) & 0x0F0F0F0Fu) | (((r.qh.y >> hb) & 0x01010101u) << 4);
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = (float)((u0 >> (8 * e)) & 0xFF);
            v[4 + e] = (float)((u1 >> (8 * e)) & 0xFF);
        }
        a[0] = f16x8_of(v);
    }
};

// Q3_K: chunk = half h = ch%2 of a super-block, group gi = pair p (columns 32p .. 32p+31 of the
// half): lane kq takes w = kq/2, l = 8(kq%2) .. +7, i.e. qs bytes 32h + 8kq .. +7 (bits 2p, 2p+1)
// and hmask bytes 8kq .. +7 (bit 4h + p); values q - 4.  Columns 0-15 and 16-31 of a group are
// sub-blocks 8h + 2p and 8h + 2p + 1, so the A operand goes out twice (as Q6_K's).  Table per
// row: the decoded factors d * (sc - 32) of the chunk's 8 sub-blocks.
struct PQ3K {
    static constexpr int NA = 2, NPAIR = 4, TAB = 8;
    static constexpr bool MIN = false, HALVES = true;
    static constexpr PartPair pairs[4] = {{0, 0}, {0, 1}, {1, 0}, {1, 1}};
    struct Raw { uint2 qs, hm, sc; unsigned short d; int h; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int) {
        const int sb = ch >> 1, h = ch & 1;
        r.qs = ldo<uint2>(rp(w, 0, row), (unsigned)(sb * 64 + 32 * h + 8 * kq));
        r.hm = ldo<uint2>(rp(w, 1, row), (unsigned)(sb * 32 + 8 * kq));
        r.sc = ldo<uint2>(rp(w, 2, row), (unsigned)(sb * 16 + 8 * h));
        r.d = ldo<unsigned short>(rp(w, 3, row), (unsigned)sb * 2u);
        r.h = h;
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int) {
        // entry kq: sub-blocks 8h + 2kq and 8h + 2kq + 1 (bytes 2kq, 2kq + 1 of the 8)
        const float d = h2f(r.d);
        const unsigned wv = kq < 2 ? r.sc.x : r.sc.y;
        const int i0 = 2 * (kq & 1);
        reinterpret_cast<float2*>(tab + m * TAB)[kq] =
            make_float2(d * gk::sbyte_f(wv, i0), d * gk::sbyte_f(wv, i0 + 1));
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int kq) {
        const int hb = 4 * r.h + gi;
        const unsigned q0 = (((r.qs.x >> (2 * gi)) & 0x03030303u) | (((r.hm.x >> hb) & 0x01010101u) << 2)) ^ 0x04040404u;
        const unsigned q1 = (((r.qs.y >> (2 * gi)) & 0x03030303u) | (((r.hm.y >> hb) & 0x01010101u) << 2)) ^ 0x04040404u;
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = (float)((int)(q0 << (29 - 8 * e)) >> 29);
            v[4 + e] = (float)((int)(q1 << (29 - 8 * e)) >> 29);
        }
        const uint4 u = f16x8_of(v);
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
        a[0] = kq < 2 ? u : z;   // columns 0-15: sub-block 8h + 2p
        a[1] = kq < 2 ? z : u;   // columns 16-31: sub-block 8h + 2p + 1
    }
};

// Q2_K (the reference's element order: element j of a super-block at bits 2(j%4) of quant byte
// j/4; gemv_kernels.h): chunk = half h = ch%2 of a super-block, lane kq of group gi takes quant
// bytes 32h + 8gi + 2kq, +1 (columns 8kq .. 8kq+7 of the group).  Each 16-column sub-block has
// its own scale and min, so the A operand goes out twice with the other half zeroed (as Q6_K)
// and the min term takes the input sums of both halves (as Q4_K's per 32).  Table per row:
// (d*sc, dmin*m) of the group's two sub-blocks, for each of the chunk's 4 groups
// (Q2_KFloatTensor.dotQ2KF32: d*sc*sumQ - dmin*m*sumF per sub-block of 16).
struct PQ2_K {
    static constexpr int NA = 2, NPAIR = 4, TAB = 16;
    static constexpr bool MIN = true, HALVES = true;
    static constexpr PartPair pairs[4] = {{0, 0}, {0, 1}, {1, 0}, {1, 1}};
    struct Raw { unsigned q[4]; uint2 sc; unsigned short d, dm; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
        const unsigned sb = (unsigned)(ch >> 1), h = (unsigned)(ch & 1);
#pragma unroll
        for (int gi = 0; gi < 4; ++gi)
            r.q[gi] = ldo<unsigned short>(rp(w, 0, row), sb * 64u + 32u * h + 8u * (unsigned)min(gi, ng - 1) + 2u * (unsigned)kq);
        r.sc = ldo<uint2>(rp(w, 1, row), sb * 16u + 8u * h);
        r.d = ldo<unsigned short>(rp(w, 2, row), sb * 2u);
        r.dm = ldo<unsigned short>(rp(w, 3, row), sb * 2u);
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int) {
        // group kq: sub-blocks 2kq and 2kq + 1 of the chunk (scale bytes 2kq, 2kq + 1)
        const unsigned wv = kq < 2 ? r.sc.x : r.sc.y;
        const unsigned b0 = (wv >> (16 * (kq & 1))) & 0xFFu, b1 = (wv >> (16 * (kq & 1) + 8)) & 0xFFu;
        const float d = h2f(r.d), dm = h2f(r.dm);
        reinterpret_cast<float4*>(tab + m * TAB)[kq] =
            make_float4(d * (float)(b0 & 15u), dm * (float)(b0 >> 4), d * (float)(b1 & 15u), dm * (float)(b1 >> 4));
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int kq) {
        const unsigned q = r.q[gi];
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (float)((q >> (8 * (e >> 2) + 2 * (e & 3))) & 3u);
        const uint4 u = f16x8_of(v);
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
        a[0] = kq < 2 ? u : z;   // columns 0-15: sub-block 2gi
        a[1] = kq < 2 ? z : u;   // columns 16-31: sub-block 2gi + 1
    }
};

// ---- codebook formats (IQ3_XXS, IQ3_S, IQ2_S; planes and values as gemv_kernels.h) ---------
// Lane kq of group gi takes unit u = 16 ch + 4 gi + kq (8 columns): 32-group g = 4 (ch%2) + gi
// of super-block ch/2, 8-weight group l = kq.  A = the signed codebook bytes, exact in fp16
// (at most 62); the group scale multiplies the product afterwards, and scale * byte is exact in
// fp32 (an 11-bit d times at most 5 + 6 bits), so each term equals the reference's weight.
// The workgroup copies the codebook to LDS once (wave_rows), as the single-token kernel does.
template <int BYTES>
__device__ __forceinline__ uint4* codebook_lds() {
    __shared__ uint4 g[BYTES / 16];
    return g;
}
// 8 signed codebook bytes (lo: weights 0-3, hi: 4-7; sign bit j of s negates weight j) as fp16
__device__ __forceinline__ uint4 signed_grid8(unsigned lo, unsigned hi, unsigned s) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float a = gk::byte_f(lo, e), b = gk::byte_f(hi, e);
        v[e] = (s >> e) & 1u ? -a : a;
        v[4 + e] = (s >> (4 + e)) & 1u ? -b : b;
    }
    return f16x8_of(v);
}

// IQ3_XXS: per 32-group the factor d * (0.5 + sc) * 0.5.  Table per row: the chunk's 4.
struct PIQ3_XXS {
    static constexpr int NA = 1, NPAIR = 2, TAB = 4, GRID_BYTES = 256 * 4;
    static constexpr bool MIN = false, HALVES = false;
    static constexpr PartPair pairs[2] = {{0, 0}, {0, 1}};
    static __device__ __forceinline__ const void* grid_src() { return gk::kIq3xxsGrid; }
    struct Raw { unsigned q[4], s[4]; uint2 h; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
            const unsigned u = (unsigned)(16 * ch + 4 * min(gi, ng - 1) + kq);
            r.q[gi] = ldo<unsigned short>(rp(w, 0, row), 2u * u);
            r.s[gi] = ldo<unsigned char>(rp(w, 1, row), u);
        }
        r.h = ldo<uint2>(rp(w, 2, row), (unsigned)(ch >> 1) * 8u);
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int ch) {
        const int g = 4 * (ch & 1) + kq;
        const float d = h2f((unsigned short)(r.h.x & 0xFFFFu));
        tab[m * TAB + kq] = (d * (0.5f + (float)((r.h.y >> (4 * g)) & 15u))) * 0.5f;
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int) {
        const unsigned* g = reinterpret_cast<const unsigned*>(codebook_lds<GRID_BYTES>());
        a[0] = signed_grid8(g[r.q[gi] & 0xFFu], g[r.q[gi] >> 8], r.s[gi]);
    }
};

// IQ3_S: ninth index bits from qh[g/4 + g%2] (the reference's reading); per 32-group the factor
// d * (1 + 2 sc).  Table per row: the chunk's 4.
struct PIQ3_S {
    static constexpr int NA = 1, NPAIR = 2, TAB = 4, GRID_BYTES = 512 * 4;
    static constexpr bool MIN = false, HALVES = false;
    static constexpr PartPair pairs[2] = {{0, 0}, {0, 1}};
    static __device__ __forceinline__ const void* grid_src() { return gk::kIq3sGrid; }
    struct Raw { unsigned q[4], s[4]; uint4 side; int h; };   // side: qh[8], scales[4], d
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
            const unsigned u = (unsigned)(16 * ch + 4 * min(gi, ng - 1) + kq);
            r.q[gi] = ldo<unsigned short>(rp(w, 0, row), 2u * u);
            r.s[gi] = ldo<unsigned char>(rp(w, 1, row), u);
        }
        r.side = ldo<uint4>(rp(w, 2, row), (unsigned)(ch >> 1) * 16u);
        r.h = ch & 1;
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int ch) {
        const int g = 4 * (ch & 1) + kq;
        const float d = h2f((unsigned short)(r.side.w & 0xFFFFu));
        tab[m * TAB + kq] = d * (float)(1 + 2 * (int)((r.side.z >> (4 * g)) & 15u));
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int kq) {
        const unsigned* g = reinterpret_cast<const unsigned*>(codebook_lds<GRID_BYTES>());
        // group g = 4h + gi reads qh[g/4 + g%2] = qh[h + gi%2], a byte of side.x
        const unsigned qh = (r.side.x >> (8 * (r.h + (gi & 1)))) & 0xFFu;
        const unsigned l2 = 2u * (unsigned)kq;
        const unsigned i0 = (r.q[gi] & 0xFFu) | (((qh >> l2) & 1u) << 8);
        const unsigned i1 = (r.q[gi] >> 8) | (((qh >> (l2 + 1u)) & 1u) << 8);
        a[0] = signed_grid8(g[i0], g[i1], r.s[gi]);
    }
};

// IQ2_S: index bits 8-9 from bits 2l..2l+1 of qh[g]; the 16-column halves of a 32-group have
// their own factors d * (0.5 + sc) * 0.25, so the A operand goes out twice with the other half
// zeroed (as Q6_K).  Table per row: the two factors of each of the chunk's 4 groups.
struct PIQ2_S {
    static constexpr int NA = 2, NPAIR = 4, TAB = 8, GRID_BYTES = 1024 * 8;
    static constexpr bool MIN = false, HALVES = true;
    static constexpr PartPair pairs[4] = {{0, 0}, {0, 1}, {1, 0}, {1, 1}};
    static __device__ __forceinline__ const void* grid_src() { return gk::kIq2sGrid; }
    struct Raw { unsigned q[4], s[4]; uint2 sc, qh; unsigned short d; int h; };   // 24-byte stride: 8-byte loads
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
        const unsigned sb = (unsigned)(ch >> 1);
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
            const unsigned u = (unsigned)(16 * ch + 4 * min(gi, ng - 1) + kq);
            r.q[gi] = ldo<unsigned char>(rp(w, 0, row), u);
            r.s[gi] = ldo<unsigned char>(rp(w, 1, row), u);
        }
        r.sc = ldo<uint2>(rp(w, 2, row), sb * 24u);
        r.qh = ldo<uint2>(rp(w, 2, row), sb * 24u + 8u);
        r.d = ldo<unsigned short>(rp(w, 2, row), sb * 24u + 16u);
        r.h = ch & 1;
    }
    static __device__ __forceinline__ void table(const Raw& r, float* tab, int m, int kq, int ch) {
        const int g = 4 * (ch & 1) + kq;
        const unsigned b = ((g < 4 ? r.sc.x : r.sc.y) >> (8 * (g & 3))) & 0xFFu;
        const float d = h2f(r.d);
        reinterpret_cast<float2*>(tab + m * TAB)[kq] =
            make_float2((d * (0.5f + (float)(b & 15u))) * 0.25f, (d * (0.5f + (float)(b >> 4))) * 0.25f);
    }
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int kq) {
        const uint2* g = reinterpret_cast<const uint2*>(codebook_lds<GRID_BYTES>());
        const unsigned qh = ((r.h ? r.qh.y : r.qh.x) >> (8 * gi)) & 0xFFu;   // qh[4h + gi]
        const uint2 e = g[r.q[gi] | (((qh >> (2 * kq)) & 3u) << 8)];
        const uint4 u = signed_grid8(e.x, e.y, r.s[gi]);
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
        a[0] = kq < 2 ? u : z;   // columns 0-15: the low scale nibble
        a[1] = kq < 2 ? z : u;   // columns 16-31: the high one
    }
};

// F16 rows: the 8 weights of a lane are its A operand as they are.
struct PF16 {
    static constexpr int NA = 1, NPAIR = 2, TAB = 0;
    static constexpr bool MIN = false, HALVES = false;
    static constexpr PartPair pairs[2] = {{0, 0}, {0, 1}};
    struct Raw { uint4 w[4]; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
        const unsigned char* p = rp(w, 0, row);
#pragma unroll
        for (int g = 0; g < 4; ++g) r.w[g] = ldo<uint4>(p, (unsigned)(ch * 256 + 64 * min(g, ng - 1) + 16 * kq));
    }
    static __device__ __forceinline__ void table(const Raw&, float*, int, int, int) {}
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int) { a[0] = r.w[gi]; }
};

// BF16 rows: converted to fp16, exact within fp16's normal range (weights below 2^-14 keep
// 2^-24 absolute precision).
struct PBF16 {
    static constexpr int NA = 1, NPAIR = 2, TAB = 0;
    static constexpr bool MIN = false, HALVES = false;
    static constexpr PartPair pairs[2] = {{0, 0}, {0, 1}};
    struct Raw { uint4 w[4]; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
        const unsigned char* p = rp(w, 0, row);
#pragma unroll
        for (int g = 0; g < 4; ++g) r.w[g] = ldo<uint4>(p, (unsigned)(ch * 256 + 64 * min(g, ng - 1) + 16 * kq));
    }
    static __device__ __forceinline__ void table(const Raw&, float*, int, int, int) {}
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int) {
        const unsigned u[4] = {r.w[gi].x, r.w[gi].y, r.w[gi].z, r.w[gi].w};
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = bf2f((unsigned short)(u[e] & 0xFFFF));
            v[2 * e + 1] = bf2f((unsigned short)(u[e] >> 16));
        }
        a[0] = f16x8_of(v);
    }
};

// F32 rows: each weight split into fp16 hi + lo; the pairs (hi, hi), (hi, lo), (lo, hi) (the
// lo*lo product is below 2^-22 of the term).
struct PF32 {
    static constexpr int NA = 2, NPAIR = 3, TAB = 0;
    static constexpr bool MIN = false, HALVES = false;
    static constexpr PartPair pairs[3] = {{0, 0}, {0, 1}, {1, 0}};
    struct Raw { uint4 w[8]; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
        const unsigned char* p = rp(w, 0, row);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const unsigned o = (unsigned)(ch * 512 + 128 * min(g, ng - 1) + 32 * kq);
            r.w[2 * g] = ldo<uint4>(p, o);
            r.w[2 * g + 1] = ldo<uint4>(p, o + 16u);
        }
    }
    static __device__ __forceinline__ void table(const Raw&, float*, int, int, int) {}
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA], int) {
        const uint4 w0 = r.w[2 * gi], w1 = r.w[2 * gi + 1];
        const float v[8] = {__uint_as_float(w0.x), __uint_as_float(w0.y), __uint_as_float(w0.z),
                            __uint_as_float(w0.w), __uint_as_float(w1.x), __uint_as_float(w1.y),
                            __uint_as_float(w1.z), __uint_as_float(w1.w)};
        split8(v, a[0], a[1]);
    }
};

// ---- input range and pre-norm factors -------------------------------------------------------
// The launch's input range exponent E (ProjTokArgs::tok_sc), uniform over the workgroup.
__device__ __forceinline__ int input_exp(const ProjTokArgs& a) {
    int e = 0;
    if (a.tok_sc != nullptr) {
        for (int t = 0; t < a.K; ++t) e = max(e, (int)a.tok_sc[2 * t + 1]);
    } else if (a.in_range != nullptr) {
        for (int h = 0; h < a.in_range_n; ++h) e = max(e, a.in_range[2 * h + 1]);
    }
    return __builtin_amdgcn_readfirstlane(e);
}

// One workgroup per token t: with norm weights w, r = 1/sqrt(sum(x^2)/cols + eps) (the factor
// of RMSNorm.apply, RMSNorm.java:13-22) and e the range exponent (dk::range_exp_of_bits) of
// max |x*w| (the values the projection splits); without, r = 1 and e from max |x|.  Writes
// sc[2t] = r and sc[2t + 1] = e.  x rows and w are 16-byte aligned and cols % 4 == 0
// (launch_tok_prep checks).  One pass: each trip issues all of its float4 loads before any
// arithmetic, so a row of up to 4·4·NTHR values costs one memory round trip (a loop with one
// dependent load per trip waited a full round trip per trip: 9.7 µs for 16 rows of 3072).
constexpr int kPrepThreads = 256;
constexpr int kPrepUnroll = 4;
template <int NTHR>
__global__ __launch_bounds__(NTHR) void tok_prep_kernel(const float* x, long long x_pitch, int cols,
                                                        const float* w, float eps, float* sc) {
    __shared__ float red[NTHR / 64];
    __shared__ unsigned redm[NTHR / 64];
    const int tid = threadIdx.x, t = blockIdx.x;
    const float4* xt = reinterpret_cast<const float4*>(x + (long long)t * x_pitch);
    const float4* w4 = reinterpret_cast<const float4*>(w);
    const int n4 = cols >> 2;
    const bool norm = w != nullptr;
    float ss = 0.0f;
    unsigned mb = 0;
    for (int i0 = tid; i0 < n4; i0 += kPrepUnroll * NTHR) {
        float4 xv[kPrepUnroll], wv[kPrepUnroll];
#pragma unroll
        for (int u = 0; u < kPrepUnroll; ++u) {
            const int i = min(i0 + u * NTHR, n4 - 1);   // clamped; the element is not counted below
            xv[u] = xt[i];
            wv[u] = norm ? w4[i] : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        }
#pragma unroll
        for (int u = 0; u < kPrepUnroll; ++u) {
            if (i0 + u * NTHR < n4) {
                const float4 a = xv[u], b = wv[u];
                ss = __builtin_fmaf(a.x, a.x, ss);
                ss = __builtin_fmaf(a.y, a.y, ss);
                ss = __builtin_fmaf(a.z, a.z, ss);
                ss = __builtin_fmaf(a.w, a.w, ss);
                mb = max(mb, max(max(dk::abs_bits(a.x * b.x), dk::abs_bits(a.y * b.y)),
                                 max(dk::abs_bits(a.z * b.z), dk::abs_bits(a.w * b.w))));
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        ss = ss + __shfl_xor(ss, off);
        mb = max(mb, (unsigned)__shfl_xor((int)mb, off));
    }
    if ((tid & 63) == 0) {
        red[tid >> 6] = ss;
        redm[tid >> 6] = mb;
    }
    __syncthreads();
    if (tid == 0) {
        float tot = red[0];
        unsigned m = redm[0];
#pragma unroll
        for (int k = 1; k < NTHR / 64; ++k) {
            tot = tot + red[k];
            m = max(m, redm[k]);
        }
        float r = 1.0f;
        if (norm) {
            float q = tot / (float)cols;
            q = q + eps;
            r = 1.0f / (float)__builtin_sqrt((double)q);
        }
        sc[2 * t] = r;
        sc[2 * t + 1] = (float)dk::range_exp_of_bits(m);
    }
}

// The Q8_1 input of K tokens for the int8 formats (Q8In<...>), one workgroup per token slot
// t < kTok.  Token t < n_tokens: with norm weights w, the staged RMSNorm of the single-token
// projection kernel bit for bit (thread i sums the squares of chunks i, i + NTHR, ... with fmaf,
// each wave's partials by row_group_sum, the waves' in order; r = 1/(float)sqrt((double)(sum/cols
// + eps)); (x*r)*w per value), or x as it is without; then gk::put_q8 per block of 32 into LDS
// (the single-token kernel's quantiser); then the quants as fp16 into q8b in the B-operand
// layout, the block scales and sums into q8d and q8s.  Slots t >= n_tokens get zeros.  With sc,
// also sc[2t] = r and sc[2t + 1] = the range exponent of max|x*w| (for the fp32-input rows of a
// launch pairing an int8 format with Q6_K).  cols % 32 == 0, cols <= kMaxGemvCols.
template <int NTHR>
__global__ __launch_bounds__(NTHR) void tok_q8_kernel(const float* x, long long x_pitch, int cols,
                                                      const float* w, float eps, int n_tokens,
                                                      uint4* q8b, float* q8d, float* q8s, float* sc) {
    static_assert(NTHR == 256, "the single-token kernel's staging: 4 waves of partial sums");
    extern __shared__ unsigned char s_q[];             // the quants, cols bytes
    __shared__ float s_d[gk::kMaxGemvCols / 32], s_s[gk::kMaxGemvCols / 32];
    __shared__ float red[NTHR / 64];
    __shared__ unsigned redm[NTHR / 64];
    const int tid = threadIdx.x, t = blockIdx.x, lane = tid & 63;
    const int n4 = cols >> 2, ng = cols >> 5;
    if (t >= n_tokens) {
        for (int i = tid; i < 4 * ng; i += NTHR) q8b[64 * (i >> 2) + 16 * (i & 3) + t] = make_uint4(0u, 0u, 0u, 0u);
        for (int g = tid; g < ng; g += NTHR) {
            q8d[16 * g + t] = 0.0f;
            q8s[16 * g + t] = 0.0f;
        }
        return;
    }
    const float4* xt = reinterpret_cast<const float4*>(x + (long long)t * x_pitch);
    const float4* w4 = reinterpret_cast<const float4*>(w);
    const bool norm = w != nullptr;
    float ss = 0.0f;
    unsigned mb = 0;
    for (int c = tid; c < n4; c += NTHR) {
        const float4 v = xt[c];
        ss = __builtin_fmaf(v.x, v.x, ss);
        ss = __builtin_fmaf(v.y, v.y, ss);
        ss = __builtin_fmaf(v.z, v.z, ss);
        ss = __builtin_fmaf(v.w, v.w, ss);
        const float4 b = norm ? w4[c] : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        mb = max(mb, max(max(dk::abs_bits(v.x * b.x), dk::abs_bits(v.y * b.y)),
                         max(dk::abs_bits(v.z * b.z), dk::abs_bits(v.w * b.w))));
    }
    ss = dk::row_group_sum<64>(ss);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mb = max(mb, (unsigned)__shfl_xor((int)mb, off));
    if (lane == 0) {
        red[tid >> 6] = ss;
        redm[tid >> 6] = mb;
    }
    __syncthreads();
    float r = 1.0f;
    if (norm) {
        float tot = red[0];
#pragma unroll
        for (int k = 1; k < NTHR / 64; ++k) tot = tot + red[k];
        float q = tot / (float)cols;
        q = q + eps;
        r = 1.0f / (float)__builtin_sqrt((double)q);
    }
    if (sc != nullptr && tid == 0) {
        unsigned m = redm[0];
#pragma unroll
        for (int k = 1; k < NTHR / 64; ++k) m = max(m, redm[k]);
        sc[2 * t] = r;
        sc[2 * t + 1] = (float)dk::range_exp_of_bits(m);
    }
    // quantise: the 8 lanes of a block call put_q8 together (cols % 32 == 0)
    for (int c = tid; c < n4; c += NTHR) {
        const float4 v = xt[c];
        gk::put_q8(c, norm ? gk::scale4(v, r, w4[c]) : v, s_q, s_d, s_s);
    }
    __syncthreads();
    // item i = 4 g + kq: the 8 quants at 32 g + 8 kq as fp16
    for (int i = tid; i < 4 * ng; i += NTHR) {
        const uint2 qb = *reinterpret_cast<const uint2*>(s_q + 8 * i);
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = (float)(int)(signed char)((qb.x >> (8 * e)) & 0xFFu);
            v[4 + e] = (float)(int)(signed char)((qb.y >> (8 * e)) & 0xFFu);
        }
        q8b[64 * (i >> 2) + 16 * (i & 3) + t] = f16x8_of(v);
    }
    for (int g = tid; g < ng; g += NTHR) {
        q8d[16 * g + t] = s_d[g];
        q8s[16 * g + t] = s_s[g];
    }
}

// ---- the projection kernel ------------------------------------------------------------------
__device__ __forceinline__ const TokSeg& tok_seg(const ProjTokArgs& a, int row_g) {
    const bool in1 = a.nseg > 1 && row_g >= a.seg[1].out_off;
    const bool in2 = a.nseg > 2 && row_g >= a.seg[2].out_off;
    return in2 ? a.seg[2] : (in1 ? a.seg[1] : a.seg[0]);
}

// One wave's loads for one chunk: the raw weight bytes, and for each group the lane's 8 inputs
// of token l%16 (columns 8*(l/16) .. +7 of the group) with their norm weights.
template <class F, bool Q8 = IsQ8B<F>::value>
struct ChunkRegs {
    typename F::Raw raw;
    float4 x[kGroups][2];
};
template <class F>
struct ChunkRegs<F, true> {   // the Q8_1 input: the quants as fp16, the block scales and sums
    typename F::Raw raw;
    uint4 b[kGroups];
    float dx[kGroups], sx[kGroups];
};

template <class F, bool NORM>
__device__ __forceinline__ void chunk_issue(ChunkRegs<F>& c, const ProjTokArgs& a, const WPlanes& w,
                                            int row, int ch, int ngroups, int lane, bool tok_live) {
    const int kq = lane >> 4, t = lane & 15;
    const int g0 = ch * kGroups;
    const int ng = min(kGroups, ngroups - g0);
    F::load(c.raw, w, row, ch, kq, ng);
    if constexpr (IsQ8B<F>::value) {   // token slots past K hold zeros (tok_q8_kernel)
#pragma unroll
        for (int gi = 0; gi < kGroups; ++gi) {
            const int g = g0 + min(gi, ng - 1);
            c.b[gi] = a.q8b[64 * g + lane];
            c.dx[gi] = a.q8d[16 * g + t];
            c.sx[gi] = a.q8s[16 * g + t];
        }
    } else {
        // lanes of tokens past K load token K-1's row (no branch between the loads)
        const float* xt = a.x + (long long)(tok_live ? t : a.K - 1) * a.x_pitch;
#pragma unroll
        for (int gi = 0; gi < kGroups; ++gi) {
            const int col = 32 * (g0 + min(gi, ng - 1)) + 8 * kq;
            const float4* xp = reinterpret_cast<const float4*>(xt + col);
            c.x[gi][0] = xp[0];
            c.x[gi][1] = xp[1];
        }
    }
}

template <class F, bool NORM>
__device__ __forceinline__ void chunk_consume(const ChunkRegs<F>& c, f32x4_t& acc, float fin, float* tab,
                                              const float* s_nw, int ch, int ngroups, int lane) {
    const int m = lane & 15, kq = lane >> 4;
    const int ng = min(kGroups, ngroups - ch * kGroups);
    if constexpr (F::TAB > 0) {
        F::table(c.raw, tab, m, kq, ch);
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the table is written
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int gi = 0; gi < kGroups; ++gi) {
        if (gi >= ng) break;   // uniform: a partial last chunk
        if constexpr (IsQ8B<F>::value) {
            static_assert(F::TAB > 0 && !(F::MIN && F::HALVES), "int8 formats carry a scale table");
            uint4 af[F::NA];
            F::afrag(c.raw, gi, af, kq);
            const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
            const f32x4_t t0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f8(af[0]), as_f8(c.b[gi]), z, 0, 0, 0);
            f32x4_t t1 = z;
            if constexpr (F::HALVES)
                t1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f8(af[1]), as_f8(c.b[gi]), z, 0, 0, 0);
            const float dx = c.dx[gi], sx = c.sx[gi];
#pragma unroll
            for (int i = 0; i < 4; ++i) {   // output rows 4*kq + i, token lane%16
                const float* tr = tab + (4 * kq + i) * F::TAB;
                if constexpr (F::MIN) {            // Q4_K, Q5_K: (d*sc, dmin*m) of block gi
                    const float2 f = reinterpret_cast<const float2*>(tr)[gi];
                    acc[i] = acc[i] + ((f.x * dx) * t0[i] - f.y * sx);
                } else if constexpr (F::HALVES) {  // Q3_K: d*(sc - 32) of the two halves
                    const float2 f = reinterpret_cast<const float2*>(tr)[gi];
                    acc[i] = acc[i] + ((f.x * dx) * t0[i] + (f.y * dx) * t1[i]);
                } else {                           // Q8_0, Q5_0, IQ4_NL, IQ4_XS: the block's scale
                    acc[i] = acc[i] + (tr[gi] * dx) * t0[i];
                }
            }
            continue;
        } else {
        // lanes of tokens past K hold token K-1's inputs: finite, and their outputs are never
        // stored.  Inputs times 2^-E: with the norm, the staged weights carry the factor.
        const float xv[8] = {c.x[gi][0].x, c.x[gi][0].y, c.x[gi][0].z, c.x[gi][0].w,
                             c.x[gi][1].x, c.x[gi][1].y, c.x[gi][1].z, c.x[gi][1].w};
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = NORM ? xv[e] : xv[e] * fin;
        if constexpr (NORM) {   // the norm weights of these 8 columns, from LDS
            const float4* wp = reinterpret_cast<const float4*>(s_nw + 32 * (ch * kGroups + gi) + 8 * kq);
            const float4 w0 = wp[0], w1 = wp[1];
            const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = v[e] * wv[e];
        }
        float gs = 0.0f, gs_hi = 0.0f;   // the group's input sum for token l%16 (the min term);
                                          // per 16-column half (Q2_K): gs the first, gs_hi the second
        if constexpr (F::MIN) {
            gs = v[0];
#pragma unroll
            for (int e = 1; e < 8; ++e) gs = gs + v[e];
            gs = dk::lane_step<16, false>(gs);   // the k-quad pairs (lanes l ^ 16): half sums
            if constexpr (F::HALVES) {
                // lanes 0-31 hold the first half's sum, 32-63 the second's: both to every lane
                const unsigned u = __builtin_bit_cast(unsigned, gs);
                const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
                gs = __builtin_bit_cast(float, (unsigned)p[0]);
                gs_hi = __builtin_bit_cast(float, (unsigned)p[1]);
            } else {
                gs = dk::lane_step<32, false>(gs);   // the group's 4 k-quads
            }
        }
        uint4 b[2];
        split8(v, b[0], b[1]);
        uint4 af[F::NA];
        F::afrag(c.raw, gi, af, kq);
        if constexpr (F::TAB == 0) {
#pragma unroll
            for (int k = 0; k < F::NPAIR; ++k)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f8(af[F::pairs[k].a]), as_f8(b[F::pairs[k].b]),
                                                             acc, 0, 0, 0);
        } else {
            f32x4_t t0 = {0.f, 0.f, 0.f, 0.f}, t1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < F::NPAIR; ++k) {
                if (F::pairs[k].a == 0)
                    t0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f8(af[0]), as_f8(b[F::pairs[k].b]), t0, 0, 0, 0);
                else
                    t1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f8(af[F::NA - 1]), as_f8(b[F::pairs[k].b]),
                                                                t1, 0, 0, 0);
            }
            // output rows 4*kq + i of the tile (the D layout)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float* tr = tab + (4 * kq + i) * F::TAB;
                if constexpr (F::MIN && F::HALVES) {   // Q2_K: (d*sc, dmin*m) of both halves
                    const float4 f = reinterpret_cast<const float4*>(tr)[gi];
                    acc[i] = acc[i] + ((f.x * t0[i] - f.y * gs) + (f.z * t1[i] - f.w * gs_hi));
                } else if constexpr (F::MIN) {    // Q4_K: (d*sc, dmin*m) of sub-block gi
                    const float2 f = reinterpret_cast<const float2*>(tr)[gi];
                    acc[i] = acc[i] + (f.x * t0[i] - f.y * gs);
                } else if constexpr (F::HALVES) {  // Q6_K: d*sc of the two halves
                    const float2 f = reinterpret_cast<const float2*>(tr)[gi];
                    acc[i] = acc[i] + (f.x * t0[i] + f.y * t1[i]);
                } else {                           // Q8_0 / Q4_0: d of block gi
                    acc[i] = acc[i] + tr[gi] * t0[i];
                }
            }
        }
        }
    }
    if constexpr (F::TAB > 0) __builtin_amdgcn_wave_barrier();   // table reads before its rewrite
}

// The wave's share of its workgroup's rows: chunks wave, wave + kWaves, ... (n of them), in
// pairs with one exit and no branch between loads: every refill is issued, the last pair's
// clamped to the wave's last chunk (a repeat of loads already in the caches).  A conditional
// refill made the wait-count pass merge the two paths, and each chunk then waited for the next
// chunk's loads.
template <class F, bool NORM>
__device__ __forceinline__ void wave_rows(const ProjTokArgs& a, const WPlanes& w, int row, int wave,
                                          int lane, f32x4_t& acc, float fin, float* tab, float* s_nw) {
    const int ngroups = a.cols >> 5;
    const int nchunks = (ngroups + kGroups - 1) / kGroups;
    const int n = wave < nchunks ? (nchunks - wave + kWaves - 1) / kWaves : 0;
    const bool tok_live = (lane & 15) < a.K;
    auto chunk = [&](int i) { return wave + min(i, n - 1) * kWaves; };
    ChunkRegs<F> ca, cb;
    if (n > 0) chunk_issue<F, NORM>(ca, a, w, row, chunk(0), ngroups, lane, tok_live);
    constexpr int GRID = gk::FmtGrid<F>::BYTES;   // codebook formats: the codebook to LDS
    constexpr bool STAGE_NW = NORM && !IsQ8B<F>::value;   // the Q8_1 input is normalised already
    if constexpr (STAGE_NW || GRID > 0) {
        if constexpr (STAGE_NW) {   // the norm weights times 2^-E to LDS once per workgroup, behind
                                // the first loads ((x * w) * 2^-E = x * (w * 2^-E), exactly)
            const float4* src = reinterpret_cast<const float4*>(a.norm_w);
            for (int c4 = wave * 64 + lane; c4 < (a.cols >> 2); c4 += kThreads) {
                const float4 wv = src[c4];
                reinterpret_cast<float4*>(s_nw)[c4] =
                    make_float4(wv.x * fin, wv.y * fin, wv.z * fin, wv.w * fin);
            }
        }
        if constexpr (GRID > 0) {
            const uint4* src = static_cast<const uint4*>(gk::FmtGrid<F>::src());
            for (int i = wave * 64 + lane; i < GRID / 16; i += kThreads) codebook_lds<GRID>()[i] = src[i];
        }
        __syncthreads();
    }
    if (n == 0) return;
    int i = 0;
    for (; i + 1 < n; i += 2) {
        chunk_issue<F, NORM>(cb, a, w, row, chunk(i + 1), ngroups, lane, tok_live);
        chunk_consume<F, NORM>(ca, acc, fin, tab, s_nw, chunk(i), ngroups, lane);
        chunk_issue<F, NORM>(ca, a, w, row, chunk(i + 2), ngroups, lane, tok_live);
        chunk_consume<F, NORM>(cb, acc, fin, tab, s_nw, chunk(i + 1), ngroups, lane);
    }
    if (n & 1) chunk_consume<F, NORM>(ca, acc, fin, tab, s_nw, chunk(n - 1), ngroups, lane);
}

template <class F1, class F2>
constexpr int tab_floats() { return F1::TAB > F2::TAB ? (F1::TAB > 0 ? F1::TAB : 1) : (F2::TAB > 0 ? F2::TAB : 1); }

// Workgroup b: rows 16b .. 16b+15 (one segment, one format: segment sizes are multiples of 16),
// all K tokens.
// Waves per SIMD the kernel is compiled for: 4 (two workgroups per CU, so 256 CUs take 512
// row tiles in one round), 3 for F32 rows (their raw chunk is twice as large) and IQ2_S rows
// (14 registers of raw bytes per chunk and two A operands: 4 waves spill with the norm).
template <class F1, class F2>
constexpr int waves_per_eu() {
    return std::is_same<F1, PF32>::value || std::is_same<F1, PIQ2_S>::value ? 3 : 4;
}

template <class F1, class F2, bool NORM>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(waves_per_eu<F1, F2>())))
void proj_tok_kernel(ProjTokArgs a) {
    extern __shared__ float s_nw[];   // NORM: the pre-norm weights [cols], times 2^-E
    __shared__ float s_tab[kWaves][16 * tab_floats<F1, F2>()];
    __shared__ f32x4_t s_red[kWaves][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = blockIdx.x * 16;
    const TokSeg& sg = tok_seg(a, row0);
    const int row = row0 - sg.out_off + (lane & 15);   // this lane's A row within its segment
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    // The launch's input range factor 2^-E and output factor 2^E (scalar registers).
    const int E = input_exp(a);
    const float fin = __uint_as_float((unsigned)(127 - E) << 23);
    if (std::is_same<F1, F2>::value || sg.fmt == 0)
        wave_rows<F1, NORM>(a, sg.w, row, wave, lane, acc, fin, s_tab[wave], s_nw);
    else
        wave_rows<F2, NORM>(a, sg.w, row, wave, lane, acc, fin, s_tab[wave], s_nw);

    s_red[wave][lane] = acc;
    __syncthreads();
    // 256 outputs (16 rows x 16 tokens); thread o < 256 sums the waves' partials for (lane o%64,
    // element o/64).
    if (tid < 256) {
        const int ln = tid & 63, i = tid >> 6;
        const int tt = ln & 15, rr = 4 * (ln >> 4) + i;   // token, tile row
        float v = s_red[0][ln][i];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) v = v + s_red[w][ln][i];
        // rows on the Q8_1 input carry its scales already (no 2^-E, normalised before quantising)
        const bool first = std::is_same<F1, F2>::value || sg.fmt == 0;
        const bool q8_rows = first ? IsQ8B<F1>::value : IsQ8B<F2>::value;
        if (tt < a.K) {
            if (!q8_rows) {
                v = v * __uint_as_float((unsigned)(127 + E) << 23);   // the inputs were scaled by 2^-E
                if constexpr (NORM) v = v * a.tok_sc[2 * tt];         // RMSNorm.apply's factor r
            }
            const int r = row0 - sg.out_off + rr;
            if (sg.bias != nullptr) v = v + sg.bias[r];
            if (a.resid != nullptr) {
                if (a.rscale > 0.0f) v = v * a.rscale;
                float* x = a.resid + (long long)tt * a.resid_pitch + row0 + rr;
                *x = *x + v;
            } else {
                sg.out[(long long)tt * sg.out_pitch + r] = v;
            }
        }
    }
}

}  // namespace tk
}  // namespace llmp
