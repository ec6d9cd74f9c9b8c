// Projections of up to 16 tokens at once on the matrix cores (the attention half of a layer for
// K tokens: speculative verification and batched forwards, LLMEngine.forwardBatch at
// LLMEngine.java:1019-1033; the plan in docs/optimization/speculative-decoding.md:120-140 reads
// each weight row once for all K tokens).
//
// One token's projection is a matrix-vector product bound by issue (gemv_kernels.h).  K tokens
// make it a skinny matrix product Y[t][r] = sum_c W[r][c] x_t[c], which runs on
// v_mfma_f32_16x16x32_bf16 with the rows as M, the tokens as N (padded to 16) and the columns
// as the reduction:
//
//  - A (weights): the quantised integers exactly (Q4_K nibbles, Q6_K 6-bit values, Q8_0 int8,
//    Q4_0 nibbles minus 8 are all exact in bf16), the per-block scales applied to the fp32
//    product of each 32-column group afterwards (Q4_K: d*sc * sum(q x) - dmin*m * sum(x), the
//    tensor classes' per-element values summed per block).  BF16 weights are exact; F16 weights
//    are two exact bf16 parts, F32 weights three.
//  - B (inputs): each fp32 input is split into three bf16 parts x = hi + mid + lo, which is
//    exact (8 + 8 + 8 significand bits), so every product is exact and only the fp32
//    accumulation rounds; the result matches the CPU path to the tolerance of a reordered
//    fp32 sum.
//
// A staging launch (proj_stage_kernel, one workgroup per token) applies the pre-attention
// RMSNorm exactly as the single-token kernel does and writes the parts in the B-operand lane
// order, plus each 32-column group's sum (the Q4_K min term).  The projection launch
// (proj_tok_kernel) gives each workgroup 16 rows and all tokens; its 8 waves split the
// columns in 128-column chunks and their partial tiles are summed through LDS.  A wave keeps
// the next chunk's weight and input loads in flight while it computes the current one.
//
// Layout facts of v_mfma_f32_16x16x32_bf16 (as in prefill_kernels.h): lane l holds
// A[l%16][8*(l/16)+j], B[8*(l/16)+j][l%16] (j < 8) and D[4*(l/16)+j][l%16] (j < 4).
#pragma once

#include "gemv_kernels.h"

namespace llmp {
namespace tk {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTok = 16;                 // tokens per launch (the MFMA's N)
constexpr int kWaves = 8;                // waves per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kChunk = 128;              // columns per wave step (4 groups of 32)
constexpr int kGroups = kChunk / 32;
constexpr int kXParts = 3;               // bf16 parts of each input value

using gk::WPlanes;
using gk::rp;
using gk::ldo;
using gk::h2f;
using gk::u32x4;

struct TokSeg {
    WPlanes w;
    int rows;              // rows of this segment (a multiple of 16)
    int out_off;           // first row of this segment in the launch
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
    const uint4* xb;       // staged input parts [cols/32][kXParts][64] (16 bytes each)
    const float* xsum;     // [cols/32][16] per-group input sums (Q4_K)
    float* resid;          // Wo epilogue: resid[t*resid_pitch + row] += rscale? * value
    long long resid_pitch;
    float rscale;          // Granite residual scale, 0 = off
};

// Two fp32 values -> packed bf16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ unsigned pk_bf16(float x, float y) {
    return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2_t{x, y}, bf16x2_t));
}
__device__ __forceinline__ float bf_lo(unsigned p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf_hi(unsigned p) { return __uint_as_float(p & 0xFFFF0000u); }
__device__ __forceinline__ bf16x8_t as_bf8(const uint4& u) { return __builtin_bit_cast(bf16x8_t, u); }
__device__ __forceinline__ uint4 bf8_of(const float (&v)[8]) {
    return make_uint4(pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3]), pk_bf16(v[4], v[5]), pk_bf16(v[6], v[7]));
}

// ---- staging ------------------------------------------------------------------------------
// One workgroup per token t: xs = (x*r)*w with r = 1/(float)sqrt(sum(x^2)/cols + eps) summed
// as gemv_kernel sums it (norm_w null: xs = x), then for each 32-column group g and k-quad kq
// the 8 values of columns 32g + 8kq .. +7 split into hi/mid/lo bf16, stored at lane kq*16 + t
// of the group's three B fragments, and the group's sum ((s0 + s1) + (s2 + s3) over the
// quads' sequential sums).
constexpr int kStageThreads = 256;
template <int NTHR>
__global__ __launch_bounds__(NTHR) void proj_stage_kernel(const float* x, long long x_pitch,
                                                          const float* norm_w, float eps, int cols,
                                                          uint4* xb, float* xsum) {
    constexpr int kStageThreads = NTHR;
    __shared__ float red[kStageThreads / 64];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float* xt = x + (long long)t * x_pitch;
    const float4* x4 = reinterpret_cast<const float4*>(xt);
    const int n4 = cols >> 2;
    float r = 1.0f;
    if (norm_w != nullptr) {
        float ss = 0.0f;
        for (int c = tid; c < n4; c += kStageThreads) {
            const float4 v = x4[c];
            ss = __builtin_fmaf(v.x, v.x, ss);
            ss = __builtin_fmaf(v.y, v.y, ss);
            ss = __builtin_fmaf(v.z, v.z, ss);
            ss = __builtin_fmaf(v.w, v.w, ss);
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss = ss + __shfl_xor(ss, off);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float tot = red[0];
#pragma unroll
        for (int w = 1; w < kStageThreads / 64; ++w) tot = tot + red[w];
        float v = tot / (float)cols;
        v = v + eps;
        r = 1.0f / (float)__builtin_sqrt((double)v);
    }
    const int ngroups = cols >> 5;
    // item (g, kq) = 4g + kq: the 4 quads of a group sit in 4 consecutive lanes
    for (int base = 0; base < ngroups * 4; base += kStageThreads) {
        const int it = base + tid;
        const bool ok = it < ngroups * 4;
        const int itc = ok ? it : ngroups * 4 - 1;
        const int g = itc >> 2, kq = itc & 3;
        const int c0 = 32 * g + 8 * kq;
        float v[8];
        const float4 a = x4[c0 >> 2], b = x4[(c0 >> 2) + 1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        if (norm_w != nullptr) {
            const float4 wa = reinterpret_cast<const float4*>(norm_w)[c0 >> 2];
            const float4 wb = reinterpret_cast<const float4*>(norm_w)[(c0 >> 2) + 1];
            const float w8[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (v[e] * r) * w8[e];
        }
        float s = v[0];
#pragma unroll
        for (int e = 1; e < 8; ++e) s = s + v[e];
        const float s1 = __shfl_xor(s, 1);
        const float s01 = (kq & 1) ? s1 + s : s + s1;         // (s0 + s1) or (s2 + s3)
        const float s23 = __shfl_xor(s01, 2);
        const float gsum = (kq & 2) ? s23 + s01 : s01 + s23;  // (s0 + s1) + (s2 + s3)
        float hi[8], mid[8], lo[8];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const unsigned h = pk_bf16(v[e], v[e + 1]);
            const float r0 = v[e] - bf_lo(h), r1 = v[e + 1] - bf_hi(h);
            const unsigned m = pk_bf16(r0, r1);
            const float q0 = r0 - bf_lo(m), q1 = r1 - bf_hi(m);
            hi[e] = v[e]; hi[e + 1] = v[e + 1];
            mid[e] = r0; mid[e + 1] = r1;
            lo[e] = q0; lo[e + 1] = q1;
        }
        if (ok) {
            uint4* dst = xb + (long long)g * kXParts * 64 + kq * 16 + t;
            dst[0] = bf8_of(hi);
            dst[64] = bf8_of(mid);
            dst[128] = bf8_of(lo);
            if (kq == 0) xsum[g * kTok + t] = gsum;
        }
    }
}

// ---- weight formats -------------------------------------------------------------------------
// For a 128-column chunk `ch` of A row `row` (lane m = l%16 of the tile) and k-quad kq = l/16,
// a format loads its raw bytes (Raw), writes the chunk's per-row scale factors to the wave's
// LDS table (rows m, its own entries), and for group gi < 4 of the chunk builds its A operands
// (NA of them: the exact bf16 integers or parts) and names the MFMA pairs (A part, B part) it
// needs.  post() folds the group's fp32 products into the output accumulator for output rows
// 4*(l/16)+i, with the table entries of those rows.
struct PartPair {
    int a, b;
};

// Q4_K: chunk = half a super-block (sub-blocks 4h..4h+3, h = ch%2): nibble bytes 64h + 32p +
// 8kq (p = 0, 1: the two 32-byte runs, low nibbles = sub-block 4h+2p, high = 4h+2p+1) and the
// super-block's 16-byte head.  Table per row: (d*sc_s, dmin*m_s) for the chunk's 4 sub-blocks.
struct PQ4K {
    static constexpr int NA = 1, NPAIR = 3, TAB = 8;
    static constexpr bool MIN = true;
    static constexpr PartPair pairs[3] = {{0, 0}, {0, 1}, {0, 2}};
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
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA]) {
        const uint2 q = r.q[gi >> 1];
        const int sh = 4 * (gi & 1);
        const unsigned u0 = (q.x >> sh) & 0x0F0F0F0Fu, u1 = (q.y >> sh) & 0x0F0F0F0Fu;
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = (float)((u0 >> (8 * e)) & 0xFF);
            v[4 + e] = (float)((u1 >> (8 * e)) & 0xFF);
        }
        a[0] = bf8_of(v);
    }
};

// Q6_K: chunk = half h = ch%2 of a super-block (quarters c = 0..3 of 32 columns): ql words at
// 64h + 8kq and 64h + 32 + 8kq, qh word at 32h + 8kq, scales sc[8h .. 8h+7], d.  Group gi =
// quarter c: values (nibble of ql[(c&1)] at 4*(c>>1)) | (qh bits 2c..2c+1) << 4, minus 32.
// Columns 0-15 and 16-31 of a quarter have their own scales, so the A operand goes out twice,
// each time with the other half masked to zero.  Table per row: d*sc for the chunk's 8
// sub-blocks of 16.
struct PQ6K {
    static constexpr int NA = 2, NPAIR = 6, TAB = 8;
    static constexpr bool MIN = false;
    static constexpr PartPair pairs[6] = {{0, 0}, {0, 1}, {0, 2}, {1, 0}, {1, 1}, {1, 2}};
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
        const uint4 u = bf8_of(v);
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
        a[0] = kq < 2 ? u : z;   // columns 0-15: sub-block 2c
        a[1] = kq < 2 ? z : u;   // columns 16-31: sub-block 2c + 1
    }
};

// Q8_0: chunk = 4 blocks of 32: quants at 32b + 8kq, scales d (fp16) of the 4 blocks.
struct PQ8_0 {
    static constexpr int NA = 1, NPAIR = 3, TAB = 4;
    static constexpr bool MIN = false;
    static constexpr PartPair pairs[3] = {{0, 0}, {0, 1}, {0, 2}};
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
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA]) {
        const uint2 q = r.q[gi];
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = (float)(int)(signed char)((q.x >> (8 * e)) & 0xFF);
            v[4 + e] = (float)(int)(signed char)((q.y >> (8 * e)) & 0xFF);
        }
        a[0] = bf8_of(v);
    }
};

// Q4_0 (the reference's interleave: element 2i low nibble of byte i, 2i+1 high): chunk = 4
// blocks of 16 bytes; lane kq takes bytes 4kq .. 4kq+3 of a block (elements 8kq .. 8kq+7).
struct PQ4_0 {
    static constexpr int NA = 1, NPAIR = 3, TAB = 4;
    static constexpr bool MIN = false;
    static constexpr PartPair pairs[3] = {{0, 0}, {0, 1}, {0, 2}};
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
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA]) {
        const unsigned q = r.q[gi];
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const unsigned b = (q >> (8 * e)) & 0xFF;
            v[2 * e] = (float)((int)(b & 15) - 8);
            v[2 * e + 1] = (float)((int)(b >> 4) - 8);
        }
        a[0] = bf8_of(v);
    }
};

// BF16 rows: the 8 weights of a lane are its A operand as they are.
struct PBF16 {
    static constexpr int NA = 1, NPAIR = 3, TAB = 0;
    static constexpr bool MIN = false;
    static constexpr PartPair pairs[3] = {{0, 0}, {0, 1}, {0, 2}};
    struct Raw { uint4 w[4]; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
        const unsigned char* p = rp(w, 0, row);
#pragma unroll
        for (int g = 0; g < 4; ++g) r.w[g] = ldo<uint4>(p, (unsigned)(ch * 256 + 64 * min(g, ng - 1) + 16 * kq));
    }
    static __device__ __forceinline__ void table(const Raw&, float*, int, int, int) {}
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA]) { a[0] = r.w[gi]; }
};

// F16 rows: each weight is hi + lo exactly (an fp16 significand has 11 bits).  Pairs whose
// magnitude is at least 2^-16 of the product: hi*(hi, mid, lo), lo*(hi, mid).
struct PF16 {
    static constexpr int NA = 2, NPAIR = 5, TAB = 0;
    static constexpr bool MIN = false;
    static constexpr PartPair pairs[5] = {{0, 0}, {0, 1}, {0, 2}, {1, 0}, {1, 1}};
    struct Raw { uint4 w[4]; };
    static __device__ __forceinline__ void load(Raw& r, const WPlanes& w, int row, int ch, int kq, int ng) {
        const unsigned char* p = rp(w, 0, row);
#pragma unroll
        for (int g = 0; g < 4; ++g) r.w[g] = ldo<uint4>(p, (unsigned)(ch * 256 + 64 * min(g, ng - 1) + 16 * kq));
    }
    static __device__ __forceinline__ void table(const Raw&, float*, int, int, int) {}
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA]) {
        const unsigned u[4] = {r.w[gi].x, r.w[gi].y, r.w[gi].z, r.w[gi].w};
        float v[8], l[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = h2f((unsigned short)(u[e] & 0xFFFF));
            v[2 * e + 1] = h2f((unsigned short)(u[e] >> 16));
        }
        const uint4 h = bf8_of(v);
        const unsigned hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            l[2 * e] = v[2 * e] - bf_lo(hw[e]);
            l[2 * e + 1] = v[2 * e + 1] - bf_hi(hw[e]);
        }
        a[0] = h;
        a[1] = bf8_of(l);
    }
};

// F32 rows: each weight is hi + mid + lo exactly; pairs of magnitude >= 2^-16: (hi, *),
// (mid, hi), (mid, mid), (lo, hi).
struct PF32 {
    static constexpr int NA = 3, NPAIR = 6, TAB = 0;
    static constexpr bool MIN = false;
    static constexpr PartPair pairs[6] = {{0, 0}, {0, 1}, {0, 2}, {1, 0}, {1, 1}, {2, 0}};
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
    static __device__ __forceinline__ void afrag(const Raw& r, int gi, uint4 (&a)[NA]) {
        const uint4 w0 = r.w[2 * gi], w1 = r.w[2 * gi + 1];
        const float v[8] = {__uint_as_float(w0.x), __uint_as_float(w0.y), __uint_as_float(w0.z),
                            __uint_as_float(w0.w), __uint_as_float(w1.x), __uint_as_float(w1.y),
                            __uint_as_float(w1.z), __uint_as_float(w1.w)};
        float r1[8], r2[8];
        const uint4 h = bf8_of(v);
        const unsigned hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            r1[2 * e] = v[2 * e] - bf_lo(hw[e]);
            r1[2 * e + 1] = v[2 * e + 1] - bf_hi(hw[e]);
        }
        const uint4 m = bf8_of(r1);
        const unsigned mw[4] = {m.x, m.y, m.z, m.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            r2[2 * e] = r1[2 * e] - bf_lo(mw[e]);
            r2[2 * e + 1] = r1[2 * e + 1] - bf_hi(mw[e]);
        }
        a[0] = h;
        a[1] = m;
        a[2] = bf8_of(r2);
    }
};

// Formats whose A builder needs the lane's k-quad (Q6_K's masked halves).
template <class F>
__device__ __forceinline__ void afrag_of(const typename F::Raw& r, int gi, uint4 (&a)[F::NA], int kq) {
    if constexpr (std::is_same<F, PQ6K>::value) F::afrag(r, gi, a, kq);
    else F::afrag(r, gi, a);
}

// ---- the projection kernel ------------------------------------------------------------------
__device__ __forceinline__ const TokSeg& tok_seg(const ProjTokArgs& a, int row_g) {
    const bool in1 = a.nseg > 1 && row_g >= a.seg[1].out_off;
    const bool in2 = a.nseg > 2 && row_g >= a.seg[2].out_off;
    return in2 ? a.seg[2] : (in1 ? a.seg[1] : a.seg[0]);
}

// One wave's inputs for one chunk: the raw weight bytes and the B fragments of its groups.
template <class F>
struct ChunkRegs {
    typename F::Raw raw;
    uint4 b[kGroups][kXParts];
    float xs[kGroups];   // group input sums of token l%16 (Q4_K)
};

template <class F>
__device__ __forceinline__ void chunk_issue(ChunkRegs<F>& c, const ProjTokArgs& a, const WPlanes& w,
                                            int row, int ch, int ngroups, int lane, bool tok_live) {
    const int kq = lane >> 4, t = lane & 15;
    const int g0 = ch * kGroups;
    const int ng = min(kGroups, ngroups - g0);
    F::load(c.raw, w, row, ch, kq, ng);
#pragma unroll
    for (int gi = 0; gi < kGroups; ++gi) {
        const int g = g0 + min(gi, ng - 1);
#pragma unroll
        for (int p = 0; p < kXParts; ++p)
            c.b[gi][p] = tok_live ? a.xb[((long long)g * kXParts + p) * 64 + lane] : make_uint4(0u, 0u, 0u, 0u);
        if constexpr (F::MIN) c.xs[gi] = tok_live ? a.xsum[g * kTok + t] : 0.0f;
    }
}

template <class F>
__device__ __forceinline__ void chunk_consume(const ChunkRegs<F>& c, f32x4_t& acc, float* tab,
                                              int ch, int ngroups, int lane) {
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
        uint4 af[F::NA];
        afrag_of<F>(c.raw, gi, af, kq);
        if constexpr (F::TAB == 0) {
#pragma unroll
            for (int k = 0; k < F::NPAIR; ++k)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(af[F::pairs[k].a]),
                                                              as_bf8(c.b[gi][F::pairs[k].b]), acc, 0, 0, 0);
        } else {
            f32x4_t t0 = {0.f, 0.f, 0.f, 0.f}, t1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < F::NPAIR; ++k) {
                if (F::pairs[k].a == 0)
                    t0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(af[0]), as_bf8(c.b[gi][F::pairs[k].b]),
                                                                 t0, 0, 0, 0);
                else
                    t1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(af[F::NA - 1]),
                                                                 as_bf8(c.b[gi][F::pairs[k].b]), t1, 0, 0, 0);
            }
            // output rows 4*kq + i of the tile (the D layout)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float* tr = tab + (4 * kq + i) * F::TAB;
                if constexpr (F::MIN) {          // Q4_K: (d*sc, dmin*m) of sub-block gi
                    const float2 f = reinterpret_cast<const float2*>(tr)[gi];
                    acc[i] = acc[i] + (f.x * t0[i] - f.y * c.xs[gi]);
                } else if constexpr (F::NA == 2) {   // Q6_K: d*sc of the two halves
                    const float2 f = reinterpret_cast<const float2*>(tr)[gi];
                    acc[i] = acc[i] + (f.x * t0[i] + f.y * t1[i]);
                } else {                          // Q8_0 / Q4_0: d of block gi
                    acc[i] = acc[i] + tr[gi] * t0[i];
                }
            }
        }
    }
    if constexpr (F::TAB > 0) __builtin_amdgcn_wave_barrier();   // table reads before its rewrite
}

// Workgroup b: rows 16b .. 16b+15 (one segment: segment sizes are multiples of 16), all K
// tokens; wave w takes the chunks w, w + kWaves, ... and keeps the next one's loads in flight.
template <class F>
__global__ __launch_bounds__(kThreads) void proj_tok_kernel(ProjTokArgs a) {
    __shared__ float s_tab[kWaves][16 * (F::TAB > 0 ? F::TAB : 1)];
    __shared__ f32x4_t s_red[kWaves][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = blockIdx.x * 16;
    const TokSeg& sg = tok_seg(a, row0);
    const int m = lane & 15, t = lane & 15, dq = lane >> 4;
    const int row = row0 - sg.out_off + m;   // this lane's A row within its segment
    const bool tok_live = t < a.K;
    const int ngroups = a.cols >> 5;
    const int nchunks = (ngroups + kGroups - 1) / kGroups;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    float* tab = s_tab[wave];

    ChunkRegs<F> ca, cb;
    int ch = wave;
    if (ch < nchunks) chunk_issue<F>(ca, a, sg.w, row, ch, ngroups, lane, tok_live);
    // pairs of chunks with one exit, so the prefetch is never drained at a join
    while (ch < nchunks) {
        const int ch2 = ch + kWaves;
        if (ch2 < nchunks) chunk_issue<F>(cb, a, sg.w, row, ch2, ngroups, lane, tok_live);
        chunk_consume<F>(ca, acc, tab, ch, ngroups, lane);
        if (ch2 >= nchunks) break;
        const int ch3 = ch2 + kWaves;
        if (ch3 < nchunks) chunk_issue<F>(ca, a, sg.w, row, ch3, ngroups, lane, tok_live);
        chunk_consume<F>(cb, acc, tab, ch2, ngroups, lane);
        ch = ch3;
    }

    s_red[wave][lane] = acc;
    __syncthreads();
    // 256 outputs (16 rows x 16 tokens); thread o < 256 sums the waves' partials for (lane o%64,
    // element o/64).
    if (tid < 256) {
        const int ln = tid & 63, i = tid >> 6;
        float v = s_red[0][ln][i];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) v = v + s_red[w][ln][i];
        const int tt = ln & 15, rr = 4 * (ln >> 4) + i;   // token, tile row
        if (tt < a.K) {
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
    (void)dq;
}

}  // namespace tk
}  // namespace llmp
