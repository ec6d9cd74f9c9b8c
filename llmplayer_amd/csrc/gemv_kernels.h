// Matrix-vector products over GGUF-format projection weights (the attention half's Q/K/V and
// output projections, Attention.java:76-110, 232-238; reference GPU: the matmul_* kernels
// launched from CudaForwardPass.forwardAttentionPart, CudaForwardPass.java:1498-1515, 1572).
//
// Decode is one token: y = W x is bound by the weight bytes read from HBM.  The host repacks
// each GGUF tensor at upload into per-row planes so that every lane reads 16-byte aligned
// chunks (see the plane list of each format below); x (fp32, at most 16384 values) is staged
// once per workgroup in LDS, with the pre-attention RMSNorm applied while staging.  A wave
// takes a row; lane j takes the row's units j, j+64, ... (a unit is 4 to 16 weights); the 64
// partial sums are reduced in registers (DPP and permlane steps).  Dequantised weights
// equal the reference tensor classes' values; the dot's summation order differs from the CPU
// path's, so projections match it to a tolerance, not bit for bit.
#pragma once

#include <type_traits>

#include "decode_kernels.h"
#include "iq_grids.h"

namespace llmp {
namespace gk {

// GGMLType ids (GGMLType.java:4-35) of the formats with a kernel here.
constexpr int kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14, kBF16 = 30;
constexpr int kQ5_0 = 6, kQ3_K = 11, kQ5_K = 13, kIQ4_NL = 20, kIQ4_XS = 23, kMXFP4 = 39;
constexpr int kQ5_1 = 7, kQ2_K = 10, kIQ3_XXS = 18, kIQ3_S = 21, kIQ2_S = 22;

// One weight matrix on the device: up to four planes, each [rows][pitch bytes].
struct WPlanes {
    const unsigned char* p[4];
    long long pitch[4];
};

struct GemvSeg {
    WPlanes w;
    int rows;              // rows of this segment
    int out_off;           // first output row of this segment
    const float* bias;     // [rows] added to the outputs, or nullptr
    int fmt;               // launches over two formats: 0 = the first, 1 = the second
};

constexpr int kGemvThreads = 256;
constexpr int kMaxGemvCols = 16384;

struct GemvArgs {
    GemvSeg seg[3];        // same format; rows [out_off, out_off + rows) of the output
    int nseg;
    int rows_total;
    int cols;
    const float* x;        // [cols]
    const float* norm_w;   // pre-norm weights [cols] (SimdVectorOps.rmsnorm of x), or nullptr
    float eps;
    float* out;            // [rows_total], when resid is null
    float* resid;          // Wo epilogue: resid[row] += rscale? * value (TransformerBlock residual)
    float rscale;          // Granite residual scale, 0 = off
};

__device__ __forceinline__ float h2f(unsigned short h) {   // exact, like Float16.toFloat
    return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ float bf2f(unsigned short b) {
    return __builtin_bit_cast(float, (unsigned)b << 16);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Row base of plane k (wave-uniform) plus a 32-bit unsigned byte offset: the loads address a
// scalar base register plus one vector register.
__device__ __forceinline__ const unsigned char* rp(const WPlanes& w, int k, int row) {
    return w.p[k] + (long long)row * w.pitch[k];
}
template <class T>
__device__ __forceinline__ T ldo(const unsigned char* base, unsigned off) {
    return *reinterpret_cast<const T*>(base + off);
}

// ---- formats ---------------------------------------------------------------------------------
// A lane unit is a few bytes of one row's quants: consecutive lanes take consecutive units, so
// a wave's weight loads are contiguous, and the x values a unit needs are 16-byte chunks that
// consecutive lanes read from consecutive LDS addresses (no bank conflicts).
//
// Each format gives UNIT (weights per unit), MAXU (unit rounds a lane may hold in registers),
// XSUM (the dot uses the sums of the input's 4-value chunks), TAB (floats per super-block of
// the row's decoded scale table, 0 = none), Row + load_row + build_tab (the lanes of a wave
// load the row's per-super-block fields - lane i those of super-block i - and write the table
// to LDS, once per row), Raw + load (one unit's quant bytes) and dot (lane j's share of the
// row's dot product with the staged input for unit ub + j, ub a multiple of 64 and the same
// for the whole wave: the index arithmetic splits into a scalar and a per-lane part).  The dots compute in the reference tensor classes'
// per-element values (dequantised weight times x); their summation order is this kernel's own.
struct Staged {
    const float* xs;            // the input (RMS-normalised when the launch asks for it), cols floats
    const float* xsum;          // [cols/4]: (x0 + x1) + (x2 + x3) of each 4-value chunk (XSUM formats)
    const float* tab;           // this row's scale table (TAB formats)
    const unsigned char* xq;    // Q8IN formats: the input's Q8_1 quants [cols] (int8)
    const float* xd;            //   their block scales [cols/32]
    const float* xss;           //   and block sums [cols/32]
    const void* grid;           // codebook formats: the format's codebook, copied to LDS
};

// A format's codebook (IQ3_XXS, IQ3_S, IQ2_S): GRID_BYTES and grid_src(), its table in device
// memory, which each workgroup copies to LDS.  BYTES = 0 for the other formats.
template <class F, class = void>
struct FmtGrid {
    static constexpr int BYTES = 0;
    static __device__ __forceinline__ const void* src() { return nullptr; }
};
template <class F>
struct FmtGrid<F, std::void_t<decltype(F::GRID_BYTES)>> {
    static constexpr int BYTES = F::GRID_BYTES;
    static __device__ __forceinline__ const void* src() { return F::grid_src(); }
};

__device__ __forceinline__ const float4& x4(const float* xs, int i) {
    return *reinterpret_cast<const float4*>(xs + i);
}
__device__ __forceinline__ float dot4(float a, float b, float c, float d, const float4& x) {
    return __builtin_fmaf(d, x.w, __builtin_fmaf(c, x.z, __builtin_fmaf(b, x.y, a * x.x)));
}
// the four bytes of v as floats (v_cvt_f32_ubyte0..3)
__device__ __forceinline__ float byte_f(unsigned v, int t) { return (float)((v >> (8 * t)) & 0xFFu); }

struct NoRow {};

// F32: plane 0 = [rows][cols] fp32.  Unit u: weights 4u .. 4u+3 (one 16-byte load).
struct FmtF32 {
    static constexpr int UNIT = 4, MAXU = 8, TAB = 0;
    static constexpr bool XSUM = false, Q8IN = false;
    using Row = NoRow;
    static __device__ __forceinline__ Row load_row(const WPlanes&, int, int, int) { return Row{}; }
    static __device__ __forceinline__ void build_tab(const Row&, float*, int, int) {}
    struct Raw { float4 w; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ldo<float4>(rp(w, 0, row), (unsigned)u * 16u)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        return dot4(r.w.x, r.w.y, r.w.z, r.w.w, x4(st.xs, 4 * ub + 4 * j));
    }
};

// F16 / BF16: plane 0 = [rows][cols] 16-bit.  Unit u: weights 4u .. 4u+3 (one 8-byte load).
template <bool BF>
struct FmtHalf {
    static constexpr int UNIT = 4, MAXU = 8, TAB = 0;
    static constexpr bool XSUM = false, Q8IN = false;
    using Row = NoRow;
    static __device__ __forceinline__ Row load_row(const WPlanes&, int, int, int) { return Row{}; }
    static __device__ __forceinline__ void build_tab(const Row&, float*, int, int) {}
    struct Raw { uint2 w; };
    static __device__ __forceinline__ float cvt(unsigned short h) { return BF ? bf2f(h) : h2f(h); }
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ldo<uint2>(rp(w, 0, row), (unsigned)u * 8u)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        return dot4(cvt((unsigned short)(r.w.x & 0xFFFF)), cvt((unsigned short)(r.w.x >> 16)),
                    cvt((unsigned short)(r.w.y & 0xFFFF)), cvt((unsigned short)(r.w.y >> 16)),
                    x4(st.xs, 4 * ub + 4 * j));
    }
};

// Q8_0: plane 0 = quants [rows][cols] int8, plane 1 = scales [rows][cols/32] fp16.
// Unit u: quants 4u .. 4u+3 of block u/8: d * sum(q * x).
struct FmtQ8_0 {
    static constexpr int UNIT = 4, MAXU = 8, TAB = 0;
    static constexpr bool XSUM = false, Q8IN = false;
    using Row = NoRow;
    static __device__ __forceinline__ Row load_row(const WPlanes&, int, int, int) { return Row{}; }
    static __device__ __forceinline__ void build_tab(const Row&, float*, int, int) {}
    struct Raw { unsigned q; unsigned short d; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ldo<unsigned>(rp(w, 0, row), (unsigned)u * 4u),
                   ldo<unsigned short>(rp(w, 1, row), ((unsigned)u >> 3) * 2u)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const float s = dot4((float)(signed char)(r.q & 0xFF), (float)(signed char)((r.q >> 8) & 0xFF),
                             (float)(signed char)((r.q >> 16) & 0xFF), (float)(signed char)(r.q >> 24),
                             x4(st.xs, 4 * ub + 4 * j));
        return h2f(r.d) * s;
    }
};

// Q4_0: plane 0 = nibbles [rows][cols/2] (byte i: element 2i low, 2i+1 high, as
// Q4_0FloatTensor reads them), plane 1 = scales [rows][cols/32] fp16.
// Unit u: nibble bytes 4u .. 4u+3 = elements 8u .. 8u+7 of block u/4: d * sum((q - 8) x).
struct FmtQ4_0 {
    static constexpr int UNIT = 8, MAXU = 8, TAB = 0;
    static constexpr bool XSUM = false, Q8IN = false;
    using Row = NoRow;
    static __device__ __forceinline__ Row load_row(const WPlanes&, int, int, int) { return Row{}; }
    static __device__ __forceinline__ void build_tab(const Row&, float*, int, int) {}
    struct Raw { unsigned q; unsigned short d; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ldo<unsigned>(rp(w, 0, row), (unsigned)u * 4u),
                   ldo<unsigned short>(rp(w, 1, row), ((unsigned)u >> 2) * 2u)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const unsigned q = r.q;
        auto n = [&](int k) { return (float)((int)((q >> (4 * k)) & 15) - 8); };
        const int i = 8 * ub + 8 * j;
        const float s = dot4(n(0), n(1), n(2), n(3), x4(st.xs, i)) +
                        dot4(n(4), n(5), n(6), n(7), x4(st.xs, i + 4));
        return h2f(r.d) * s;
    }
};

// Q4_K: plane 0 = the 128 nibble bytes of each super-block in the GGUF order (byte 32g + l:
// element 64g + l low, 64g + 32 + l high), plane 1 = the 16-byte head of each super-block
// (d, dmin fp16, 12 bytes of 6-bit scales and mins).  Unit u: nibble bytes 4u .. 4u+3 =
// super-block sb = u/32, group g = (u%32)/8, l = 4(u%8) .. +3: elements 64g + l (sub-block
// 2g) and 64g + 32 + l (sub-block 2g + 1); value d*sc*q - dmin*m (Q4_KFloatTensor.dot), summed
// as d*sc * sum(q x) - dmin*m * sum(x).  Table: per super-block, per sub-block s the pair
// (d*sc_s, dmin*m_s), so a unit's four factors are one 16-byte read.
struct FmtQ4_K {
    static constexpr int UNIT = 8, MAXU = 8, TAB = 16;
    static constexpr bool XSUM = true, Q8IN = false;
    struct Row { u32x4 h; };
    static __device__ __forceinline__ Row load_row(const WPlanes& w, int row, int j, int units) {
        return head(w, row, j, units >> 5);
    }
    static __device__ __forceinline__ Row head(const WPlanes& w, int row, int j, int ns) {
        return Row{ldo<u32x4>(rp(w, 1, row), (unsigned)min(j, ns - 1) * 16u)};
    }
    static __device__ __forceinline__ int byte_of(const u32x4& v, int i) {
        return (int)((v[i >> 2] >> (8 * (i & 3))) & 0xFF);
    }
    static __device__ __forceinline__ void build_tab(const Row& r, float* tab, int j, int units) {
        build_tab_ns(r, tab, j, units >> 5);
    }
    static __device__ __forceinline__ void build_tab_ns(const Row& r, float* tab, int j, int ns) {
        if (j >= ns) return;
        const float d = h2f((unsigned short)(r.h[0] & 0xFFFF));
        const float dmin = h2f((unsigned short)(r.h[0] >> 16));
        float v[16];
#pragma unroll
        for (int s = 0; s < 8; ++s) {   // bytes 4..15 of the head are the 12 scale bytes
            int sc, mn;
            if (s < 4) {
                sc = byte_of(r.h, 4 + s) & 63;
                mn = byte_of(r.h, 8 + s) & 63;
            } else {
                sc = (byte_of(r.h, 8 + s) & 15) | ((byte_of(r.h, s) >> 6) << 4);
                mn = (byte_of(r.h, 8 + s) >> 4) | ((byte_of(r.h, 4 + s) >> 6) << 4);
            }
            v[2 * s] = d * (float)sc;
            v[2 * s + 1] = dmin * (float)mn;
        }
        float4* t = reinterpret_cast<float4*>(tab + j * TAB);
#pragma unroll
        for (int g = 0; g < 4; ++g) t[g] = float4{v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]};
    }
    struct Raw { unsigned q; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ldo<unsigned>(rp(w, 0, row), (unsigned)u * 4u)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        // u = ub + j: super-block ub/32 + j/32, g = (j/8)%4, l = 4(j%8)
        const int g = (j >> 3) & 3;
        const int i0 = 8 * ub + (j >> 5) * 256 + 64 * g + 4 * (j & 7), i1 = i0 + 32;
        const float4& x0 = x4(st.xs, i0);
        const float4& x1 = x4(st.xs, i1);
        // (d*sc, dmin*m) of sub-blocks 2g, 2g+1
        const float4 f = x4(st.tab, (ub >> 5) * TAB + (j >> 5) * TAB + 4 * g);
        unsigned lo = r.q & 0x0F0F0F0Fu, hi = (r.q >> 4) & 0x0F0F0F0Fu;
        // opaque to the optimiser: it would narrow the byte extracts to 4-bit fields, which
        // lose the one-instruction byte conversions (v_cvt_f32_ubyte0..3)
        asm("" : "+v"(lo), "+v"(hi));
        const float p0 = dot4(byte_f(lo, 0), byte_f(lo, 1), byte_f(lo, 2), byte_f(lo, 3), x0);
        const float p1 = dot4(byte_f(hi, 0), byte_f(hi, 1), byte_f(hi, 2), byte_f(hi, 3), x1);
        return (f.x * p0 - f.y * st.xsum[i0 >> 2]) + (f.z * p1 - f.w * st.xsum[i1 >> 2]);
    }
};

// Q6_K: plane 0 = ql (128 bytes per super-block), plane 1 = qh (64), plane 2 = scales (16
// int8), plane 3 = d (fp16), each in the GGUF order.  Unit u: super-block sb = u/16, half
// h = (u%16)/8, l = 4(u%8) .. +3 for the four quarters c: elements 128h + 32c + l, from the ql
// words at 64h + l and 64h + 32 + l and the qh word at 32h + l, scales sc[8h + l/16 + 2c]
// (Q6_KFloatTensor.dot's values d*sc*(q - 32)).  Table: per super-block the 16 products
// d*sc[8h + i + 2c] at (2h + i)*4 + c, so a unit's four factors are one 16-byte read.  The
// 6-bit values are assembled four at a time: byte t of (low nibbles | high bits << 4) ^ 0x20
// is q - 32 in 6-bit two's complement, sign-extended by a bit-field extract.
struct FmtQ6_K {
    static constexpr int UNIT = 16, MAXU = 4, TAB = 16;
    static constexpr bool XSUM = false, Q8IN = false;
    struct Row { u32x4 sc; unsigned short d; };
    static __device__ __forceinline__ Row load_row(const WPlanes& w, int row, int j, int units) {
        const unsigned sb = (unsigned)min(j, (units >> 4) - 1);
        return Row{ldo<u32x4>(rp(w, 2, row), sb * 16u), ldo<unsigned short>(rp(w, 3, row), sb * 2u)};
    }
    static __device__ __forceinline__ void build_tab(const Row& r, float* tab, int j, int units) {
        if (j >= (units >> 4)) return;
        const float d = h2f(r.d);
        float v[16];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int k = 8 * h + i + 2 * c;
                    v[(2 * h + i) * 4 + c] = d * (float)(signed char)((r.sc[k >> 2] >> (8 * (k & 3))) & 0xFF);
                }
        float4* t = reinterpret_cast<float4*>(tab + j * TAB);
#pragma unroll
        for (int g = 0; g < 4; ++g) t[g] = float4{v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]};
    }
    struct Raw { unsigned l0, l1, qh; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        const unsigned sb = (unsigned)u >> 4, h = ((unsigned)u >> 3) & 1u, l = 4u * ((unsigned)u & 7u);
        const unsigned char* ql = rp(w, 0, row);
        const unsigned qo = sb * 128u + 64u * h + l;
        return Raw{ldo<unsigned>(ql, qo), ldo<unsigned>(ql, qo + 32u),
                   ldo<unsigned>(rp(w, 1, row), sb * 64u + 32u * h + l)};
    }
    // the signed 6-bit field at bits 8t .. 8t+5 of v (shift left, then arithmetic shift right;
    // the bit-field-extract builtin's result was converted as unsigned by this compiler)
    static __device__ __forceinline__ float sx6(unsigned v, int t) {
        return (float)((int)(v << (26 - 8 * t)) >> 26);
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        // u = ub + j: super-block ub/16 + j/16, h = (j/8)%2, l = 4(j%8), i = l/16
        const int h = (j >> 3) & 1, l = 4 * (j & 7), i = (j & 7) >> 2;
        const int sb = (ub >> 4) + (j >> 4);
        const float4 f = x4(st.tab, sb * TAB + (2 * h + i) * 4);
        const float ds[4] = {f.x, f.y, f.z, f.w};
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const unsigned lo = (c & 1) ? r.l1 : r.l0;
            const unsigned nib = (c >> 1) ? (lo >> 4) & 0x0F0F0F0Fu : lo & 0x0F0F0F0Fu;
            const unsigned q = (nib | (((r.qh >> (2 * c)) & 0x03030303u) << 4)) ^ 0x20202020u;
            s = s + ds[c] * dot4(sx6(q, 0), sx6(q, 1), sx6(q, 2), sx6(q, 3),
                                 x4(st.xs, sb * 256 + 128 * h + 32 * c + l));
        }
        return s;
    }
};

// ---- split-nibble formats ----------------------------------------------------------------------
// Q5_0, IQ4_NL and MXFP4 blocks of 32, and each 32-weight sub-block of IQ4_XS, keep their codes
// split: byte i of the block's 16 holds element i in its low nibble and element 16 + i in its
// high nibble (the order of Q5_0FloatTensor, IQ4_NLFloatTensor, MXFP4FloatTensor and
// IQ4_XSFloatTensor.dot).  Unit u: nibble bytes 4u .. 4u+3 of the row = bytes i0 .. i0+3 of
// block u/4 (i0 = 4(u%4)), elements i0 .. i0+3 and 16+i0 .. 16+i0+3.
__device__ __forceinline__ int split_x(int ub, int j) { return 8 * ub + 32 * (j >> 2) + 4 * (j & 3); }

// Bit k (k < 4) of v moved to bit 0 of byte k (the four shifted copies land on distinct bits).
__device__ __forceinline__ unsigned spread4(unsigned v) { return (v * 0x00204081u) & 0x01010101u; }

// Four table bytes at once: byte k of the result is entry c_k (0..15) of the 16-byte table t,
// c_k = byte k of `codes`.  Two byte permutes pick from entries 0-7 and 8-15, bit 3 selects.
__device__ __forceinline__ unsigned lut16(unsigned codes, unsigned t0, unsigned t1, unsigned t2, unsigned t3) {
    const unsigned sel = codes & 0x07070707u;
    const unsigned a = __builtin_amdgcn_perm(t1, t0, sel);
    const unsigned b = __builtin_amdgcn_perm(t3, t2, sel);
    const unsigned m = ((codes >> 3) & 0x01010101u) * 0xFFu;
    return (a & ~m) | (b & m);
}
// byte t of v as a signed integer, in float
__device__ __forceinline__ float sbyte_f(unsigned v, int t) { return (float)((int)(v << (24 - 8 * t)) >> 24); }

// The IQ4_NL codebook (IQ4_NLFloatTensor.KVALUES_IQ4NL) as int8, four entries per word.
constexpr unsigned pack4(int a, int b, int c, int d) {
    return (unsigned)(a & 0xFF) | ((unsigned)(b & 0xFF) << 8) | ((unsigned)(c & 0xFF) << 16) |
           ((unsigned)(d & 0xFF) << 24);
}
constexpr unsigned kIq4[4] = {pack4(-127, -104, -83, -65), pack4(-49, -35, -22, -10), pack4(1, 13, 25, 38),
                              pack4(53, 69, 89, 113)};
// Twice MXFP4FloatTensor.FP4_TABLE (integers: 0, 1, 2, 3, 4, 6, 8, 12 and their negatives);
// the block scale carries the factor 1/2.
constexpr unsigned kFp4x2[4] = {pack4(0, 1, 2, 3), pack4(4, 6, 8, 12), pack4(0, -1, -2, -3),
                                pack4(-4, -6, -8, -12)};

// The dot of a split-nibble unit whose 8 values are the signed bytes of lo (elements i0..i0+3)
// and hi (16+i0..), with the staged input.
__device__ __forceinline__ float split_dot_s8(unsigned lo, unsigned hi, const Staged& st, int ub, int j) {
    const int xi = split_x(ub, j);
    return dot4(sbyte_f(lo, 0), sbyte_f(lo, 1), sbyte_f(lo, 2), sbyte_f(lo, 3), x4(st.xs, xi)) +
           dot4(sbyte_f(hi, 0), sbyte_f(hi, 1), sbyte_f(hi, 2), sbyte_f(hi, 3), x4(st.xs, xi + 16));
}

// Q5_0: plane 0 = nibbles [rows][cols/2], plane 1 = the fifth bits of each block (uint32, bit i
// = element i) [rows][cols/32], plane 2 = scales [rows][cols/32] fp16.  Values (q - 16) * d
// (Q5_0FloatTensor.getFloat), summed as d * sum((q - 16) x).
struct FmtQ5_0 {
    static constexpr int UNIT = 8, MAXU = 8, TAB = 0;
    static constexpr bool XSUM = false, Q8IN = false;
    using Row = NoRow;
    static __device__ __forceinline__ Row load_row(const WPlanes&, int, int, int) { return Row{}; }
    static __device__ __forceinline__ void build_tab(const Row&, float*, int, int) {}
    struct Raw { unsigned q, qh; unsigned short d; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ldo<unsigned>(rp(w, 0, row), (unsigned)u * 4u),
                   ldo<unsigned>(rp(w, 1, row), ((unsigned)u >> 2) * 4u),
                   ldo<unsigned short>(rp(w, 2, row), ((unsigned)u >> 2) * 2u)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const unsigned h = r.qh >> (4 * (j & 3));
        // q ^ 16 as a 5-bit two's complement number is q - 16: flip bit 4, then sign-extend
        const unsigned lo = ((r.q & 0x0F0F0F0Fu) | (spread4(h & 15u) << 4)) ^ 0x10101010u;
        const unsigned hi = (((r.q >> 4) & 0x0F0F0F0Fu) | (spread4((h >> 16) & 15u) << 4)) ^ 0x10101010u;
        auto s5 = [](unsigned v, int t) { return (float)((int)(v << (27 - 8 * t)) >> 27); };
        const int xi = split_x(ub, j);
        const float s = dot4(s5(lo, 0), s5(lo, 1), s5(lo, 2), s5(lo, 3), x4(st.xs, xi)) +
                        dot4(s5(hi, 0), s5(hi, 1), s5(hi, 2), s5(hi, 3), x4(st.xs, xi + 16));
        return h2f(r.d) * s;
    }
};

// IQ4_NL: plane 0 = nibble codes [rows][cols/2], plane 1 = scales [rows][cols/32] fp16.
// Values d * codebook[code] (IQ4_NLFloatTensor.dot), summed as d * sum(codebook x).
struct FmtIQ4_NL {
    static constexpr int UNIT = 8, MAXU = 8, TAB = 0;
    static constexpr bool XSUM = false, Q8IN = false;
    using Row = NoRow;
    static __device__ __forceinline__ Row load_row(const WPlanes&, int, int, int) { return Row{}; }
    static __device__ __forceinline__ void build_tab(const Row&, float*, int, int) {}
    struct Raw { unsigned q; unsigned short d; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ldo<unsigned>(rp(w, 0, row), (unsigned)u * 4u),
                   ldo<unsigned short>(rp(w, 1, row), ((unsigned)u >> 2) * 2u)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const unsigned lo = lut16(r.q & 0x0F0F0F0Fu, kIq4[0], kIq4[1], kIq4[2], kIq4[3]);
        const unsigned hi = lut16((r.q >> 4) & 0x0F0F0F0Fu, kIq4[0], kIq4[1], kIq4[2], kIq4[3]);
        return h2f(r.d) * split_dot_s8(lo, hi, st, ub, j);
    }
};

// MXFP4: plane 0 = nibble codes [rows][cols/2], plane 1 = E8M0 exponent bytes [rows][cols/32].
// Values FP4[code] * 2^(e - 127), 0 for e = 0 and e = 255 (MXFP4FloatTensor.dot), summed as
// 2^(e - 128) * sum(2 FP4[code] x): both factors are exact, so each product is the same.
__device__ __forceinline__ float e8m0_half(unsigned e) {
    // 2^(e - 128): a normal float for e >= 2, the subnormal 2^-127 for e = 1
    const float v = e >= 2u ? __uint_as_float((e - 1u) << 23) : __uint_as_float(0x00400000u);
    return (e == 0u || e == 255u) ? 0.0f : v;
}
struct FmtMXFP4 {
    static constexpr int UNIT = 8, MAXU = 8, TAB = 0;
    static constexpr bool XSUM = false, Q8IN = false;
    using Row = NoRow;
    static __device__ __forceinline__ Row load_row(const WPlanes&, int, int, int) { return Row{}; }
    static __device__ __forceinline__ void build_tab(const Row&, float*, int, int) {}
    struct Raw { unsigned q; unsigned char e; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ldo<unsigned>(rp(w, 0, row), (unsigned)u * 4u),
                   ldo<unsigned char>(rp(w, 1, row), (unsigned)u >> 2)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const unsigned lo = lut16(r.q & 0x0F0F0F0Fu, kFp4x2[0], kFp4x2[1], kFp4x2[2], kFp4x2[3]);
        const unsigned hi = lut16((r.q >> 4) & 0x0F0F0F0Fu, kFp4x2[0], kFp4x2[1], kFp4x2[2], kFp4x2[3]);
        return e8m0_half(r.e) * split_dot_s8(lo, hi, st, ub, j);
    }
};

// IQ4_XS: plane 0 = nibble codes [rows][cols/2] (sub-block ib of 32 at bytes 16ib .. 16ib+15
// of its super-block, split), plane 1 = the sub-blocks' 6-bit scales decoded at upload to the
// int8 ls - 32 [rows][cols/32], plane 2 = d [rows][cols/256] fp16.  Values
// (d * (ls - 32)) * codebook[code] (IQ4_XSFloatTensor.dot).  Unit u: as the split-nibble
// blocks, sub-block u/4.  Table: per super-block the 8 factors d * (ls - 32).
struct FmtIQ4_XS {
    static constexpr int UNIT = 8, MAXU = 8, TAB = 8;
    static constexpr bool XSUM = false, Q8IN = false;
    struct Row { uint2 sc; unsigned short d; };
    static __device__ __forceinline__ Row load_row(const WPlanes& w, int row, int j, int units) {
        const unsigned sb = (unsigned)min(j, (units >> 5) - 1);
        return Row{ldo<uint2>(rp(w, 1, row), sb * 8u), ldo<unsigned short>(rp(w, 2, row), sb * 2u)};
    }
    static __device__ __forceinline__ void build_tab(const Row& r, float* tab, int j, int units) {
        if (j >= (units >> 5)) return;
        const float d = h2f(r.d);
        float4* t = reinterpret_cast<float4*>(tab + j * TAB);
        t[0] = float4{d * sbyte_f(r.sc.x, 0), d * sbyte_f(r.sc.x, 1), d * sbyte_f(r.sc.x, 2), d * sbyte_f(r.sc.x, 3)};
        t[1] = float4{d * sbyte_f(r.sc.y, 0), d * sbyte_f(r.sc.y, 1), d * sbyte_f(r.sc.y, 2), d * sbyte_f(r.sc.y, 3)};
    }
    struct Raw { unsigned q; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ldo<unsigned>(rp(w, 0, row), (unsigned)u * 4u)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        // u = ub + j: sub-block (ub + j)/4 = 8 * (ub/32) + j/4 of the row's super-blocks
        const float dl = st.tab[(ub >> 2) + (j >> 2)];
        const unsigned lo = lut16(r.q & 0x0F0F0F0Fu, kIq4[0], kIq4[1], kIq4[2], kIq4[3]);
        const unsigned hi = lut16((r.q >> 4) & 0x0F0F0F0Fu, kIq4[0], kIq4[1], kIq4[2], kIq4[3]);
        return dl * split_dot_s8(lo, hi, st, ub, j);
    }
};

// Q5_K: plane 0 = the low nibbles (Q4_K's plane 0 order), plane 1 = the 16-byte head (d, dmin,
// 12 packed scale and min bytes: Q4_K's plane 1), plane 2 = the fifth bits qh (32 bytes per
// super-block: bit 2g + s of byte l = element 64g + 32s + l).  Unit u as Q4_K's; value
// d*sc*q - dmin*m (Q5_KFloatTensor.dot), summed as Q4_K's with the fifth bit or-ed in.
struct FmtQ5_K {
    static constexpr int UNIT = 8, MAXU = 8, TAB = 16;
    static constexpr bool XSUM = true, Q8IN = false;
    using Row = FmtQ4_K::Row;
    static __device__ __forceinline__ Row load_row(const WPlanes& w, int row, int j, int units) {
        return FmtQ4_K::head(w, row, j, units >> 5);
    }
    static __device__ __forceinline__ void build_tab(const Row& r, float* tab, int j, int units) {
        FmtQ4_K::build_tab_ns(r, tab, j, units >> 5);
    }
    struct Raw { unsigned q, qh; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        // qh bytes l .. l+3 of super-block u/32, l = 4(u%8)
        return Raw{ldo<unsigned>(rp(w, 0, row), (unsigned)u * 4u),
                   ldo<unsigned>(rp(w, 2, row), ((unsigned)u >> 5) * 32u + 4u * ((unsigned)u & 7u))};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const int g = (j >> 3) & 3;
        const int i0 = 8 * ub + (j >> 5) * 256 + 64 * g + 4 * (j & 7), i1 = i0 + 32;
        const float4& x0 = x4(st.xs, i0);
        const float4& x1 = x4(st.xs, i1);
        const float4 f = x4(st.tab, (ub >> 5) * TAB + (j >> 5) * TAB + 4 * g);
        unsigned lo = (r.q & 0x0F0F0F0Fu) | (((r.qh >> (2 * g)) & 0x01010101u) << 4);
        unsigned hi = ((r.q >> 4) & 0x0F0F0F0Fu) | (((r.qh >> (2 * g + 1)) & 0x01010101u) << 4);
        asm("" : "+v"(lo), "+v"(hi));   // keep the byte conversions (see FmtQ4_K::dot)
        const float p0 = dot4(byte_f(lo, 0), byte_f(lo, 1), byte_f(lo, 2), byte_f(lo, 3), x0);
        const float p1 = dot4(byte_f(hi, 0), byte_f(hi, 1), byte_f(hi, 2), byte_f(hi, 3), x1);
        return (f.x * p0 - f.y * st.xsum[i0 >> 2]) + (f.z * p1 - f.w * st.xsum[i1 >> 2]);
    }
};

// Q3_K: plane 0 = the 2-bit quants qs (64 bytes per super-block), plane 1 = the high-bit mask
// (32), plane 2 = the 16 sub-block scales decoded at upload to the int8 sc - 32, plane 3 = d
// (fp16).  Element 128h + 32p + 16w + l: bits 2p..2p+1 of qs[32h + 16w + l], bit 4h + p of
// hmask[16w + l], sub-block 8h + 2p + w; value (d * (sc - 32)) * (q - 4)
// (Q3_KFloatTensor.dot).  Unit u: qs bytes 4u .. 4u+3 = super-block sb = u/16, h = (u%16)/8,
// w = (u%8)/4, l = 4(u%4) .. +3, for the four p: 16 weights.  Table: per super-block the 16
// factors d * (sc - 32) at (2h + w)*4 + p, so a unit's four factors are one 16-byte read.
struct FmtQ3_K {
    static constexpr int UNIT = 16, MAXU = 4, TAB = 16;
    static constexpr bool XSUM = false, Q8IN = false;
    struct Row { u32x4 sc; unsigned short d; };
    static __device__ __forceinline__ Row load_row(const WPlanes& w, int row, int j, int units) {
        const unsigned sb = (unsigned)min(j, (units >> 4) - 1);
        return Row{ldo<u32x4>(rp(w, 2, row), sb * 16u), ldo<unsigned short>(rp(w, 3, row), sb * 2u)};
    }
    static __device__ __forceinline__ void build_tab(const Row& r, float* tab, int j, int units) {
        if (j >= (units >> 4)) return;
        const float d = h2f(r.d);
        float v[16];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int w = 0; w < 2; ++w)
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const int k = 8 * h + 2 * p + w;
                    v[(2 * h + w) * 4 + p] = d * sbyte_f(r.sc[k >> 2], k & 3);
                }
        float4* t = reinterpret_cast<float4*>(tab + j * TAB);
#pragma unroll
        for (int g = 0; g < 4; ++g) t[g] = float4{v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]};
    }
    struct Raw { unsigned qs, hm; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        const unsigned sb = (unsigned)u >> 4, wv = ((unsigned)u >> 2) & 1u, l = 4u * ((unsigned)u & 3u);
        return Raw{ldo<unsigned>(rp(w, 0, row), (unsigned)u * 4u),
                   ldo<unsigned>(rp(w, 1, row), sb * 32u + 16u * wv + l)};
    }
    // the signed 3-bit field at bits 8t .. 8t+2 of v
    static __device__ __forceinline__ float sx3(unsigned v, int t) {
        return (float)((int)(v << (29 - 8 * t)) >> 29);
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const int h = (j >> 3) & 1, w = (j >> 2) & 1, l = 4 * (j & 3);
        const int sb = (ub >> 4) + (j >> 4);
        const float4 f = x4(st.tab, sb * TAB + (2 * h + w) * 4);
        const float ds[4] = {f.x, f.y, f.z, f.w};
        float s = 0.0f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            // (q ^ 4) as a 3-bit two's complement number is q - 4
            const unsigned q = (((r.qs >> (2 * p)) & 0x03030303u) | (((r.hm >> (4 * h + p)) & 0x01010101u) << 2)) ^
                               0x04040404u;
            s = s + ds[p] * dot4(sx3(q, 0), sx3(q, 1), sx3(q, 2), sx3(q, 3),
                                 x4(st.xs, sb * 256 + 128 * h + 32 * p + 16 * w + l));
        }
        return s;
    }
};

// Q5_1: plane 0 = nibbles [rows][cols/2], plane 1 = the fifth bits of each block (uint32),
// planes 2 and 3 = d and m [rows][cols/32] fp16.  Values q * d + m (Q5_1FloatTensor.getFloat),
// summed as d * sum(q x) + m * sum(x) (Q5_1FloatTensor.dot: scale * blockSum + min * otherSum).
struct FmtQ5_1 {
    static constexpr int UNIT = 8, MAXU = 8, TAB = 0;
    static constexpr bool XSUM = true, Q8IN = false;
    using Row = NoRow;
    static __device__ __forceinline__ Row load_row(const WPlanes&, int, int, int) { return Row{}; }
    static __device__ __forceinline__ void build_tab(const Row&, float*, int, int) {}
    struct Raw { unsigned q, qh; unsigned short d, m; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        const unsigned b = (unsigned)u >> 2;
        return Raw{ldo<unsigned>(rp(w, 0, row), (unsigned)u * 4u), ldo<unsigned>(rp(w, 1, row), b * 4u),
                   ldo<unsigned short>(rp(w, 2, row), b * 2u), ldo<unsigned short>(rp(w, 3, row), b * 2u)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const unsigned h = r.qh >> (4 * (j & 3));
        unsigned lo = (r.q & 0x0F0F0F0Fu) | (spread4(h & 15u) << 4);
        unsigned hi = ((r.q >> 4) & 0x0F0F0F0Fu) | (spread4((h >> 16) & 15u) << 4);
        asm("" : "+v"(lo), "+v"(hi));   // keep the byte conversions (see FmtQ4_K::dot)
        const int xi = split_x(ub, j);
        const float s = dot4(byte_f(lo, 0), byte_f(lo, 1), byte_f(lo, 2), byte_f(lo, 3), x4(st.xs, xi)) +
                        dot4(byte_f(hi, 0), byte_f(hi, 1), byte_f(hi, 2), byte_f(hi, 3), x4(st.xs, xi + 16));
        return h2f(r.d) * s + h2f(r.m) * (st.xsum[xi >> 2] + st.xsum[(xi + 16) >> 2]);
    }
};

// Q2_K in the reference's layout (Q2_KFloatTensor): element j of a super-block is bits
// 2(j%4) .. +1 of quant byte j/4, sub-block j/16 takes scale byte j/16 (low nibble sc, high
// nibble m).  Plane 0 = the 64 quant bytes [rows][cols/4], plane 1 = the 16 scale bytes
// [rows][cols/16], planes 2 and 3 = d and dmin [rows][cols/256] fp16.  Values d*sc*q - dmin*m,
// summed per sub-block as (d*sc) * sum(q x) - (dmin*m) * sum(x) (Q2_KFloatTensor.dotQ2KF32).
// Unit u = 4 quant bytes = sub-block u (16 consecutive weights).
struct FmtQ2_K {
    static constexpr int UNIT = 16, MAXU = 8, TAB = 0;
    static constexpr bool XSUM = true, Q8IN = false;
    using Row = NoRow;
    static __device__ __forceinline__ Row load_row(const WPlanes&, int, int, int) { return Row{}; }
    static __device__ __forceinline__ void build_tab(const Row&, float*, int, int) {}
    struct Raw { unsigned q; unsigned char sc; unsigned short d, dm; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        const unsigned sb = (unsigned)u >> 4;
        return Raw{ldo<unsigned>(rp(w, 0, row), (unsigned)u * 4u), ldo<unsigned char>(rp(w, 1, row), (unsigned)u),
                   ldo<unsigned short>(rp(w, 2, row), sb * 2u), ldo<unsigned short>(rp(w, 3, row), sb * 2u)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const int i0 = 16 * (ub + j);   // the sub-block's first weight
        const float4 x0 = x4(st.xs, i0), x1 = x4(st.xs, i0 + 4), x2 = x4(st.xs, i0 + 8), x3 = x4(st.xs, i0 + 12);
        // field t of byte b is weight 4b + t: one masked word per t, its bytes the weights
        // t, 4 + t, 8 + t, 12 + t
        const unsigned m0 = r.q & 0x03030303u, m1 = (r.q >> 2) & 0x03030303u;
        const unsigned m2 = (r.q >> 4) & 0x03030303u, m3 = (r.q >> 6) & 0x03030303u;
        const float s = dot4(byte_f(m0, 0), byte_f(m0, 1), byte_f(m0, 2), byte_f(m0, 3), float4{x0.x, x1.x, x2.x, x3.x}) +
                        dot4(byte_f(m1, 0), byte_f(m1, 1), byte_f(m1, 2), byte_f(m1, 3), float4{x0.y, x1.y, x2.y, x3.y}) +
                        dot4(byte_f(m2, 0), byte_f(m2, 1), byte_f(m2, 2), byte_f(m2, 3), float4{x0.z, x1.z, x2.z, x3.z}) +
                        dot4(byte_f(m3, 0), byte_f(m3, 1), byte_f(m3, 2), byte_f(m3, 3), float4{x0.w, x1.w, x2.w, x3.w});
        const float xs = (st.xsum[i0 >> 2] + st.xsum[(i0 >> 2) + 1]) + (st.xsum[(i0 >> 2) + 2] + st.xsum[(i0 >> 2) + 3]);
        return (h2f(r.d) * (float)(r.sc & 15u)) * s - (h2f(r.dm) * (float)(r.sc >> 4)) * xs;
    }
};

// ---- codebook formats (IQ3_XXS, IQ3_S, IQ2_S) ------------------------------------------------
// A unit is one 8-weight group: two 4-weight codebook entries (IQ3_XXS, IQ3_S) or one 8-weight
// entry (IQ2_S), read from the LDS copy of the codebook, and eight sign bits.  Each weight is
// (group scale * codebook byte), negated where its sign bit is set: the value the reference
// classes stage (db * gv * sign; the negation is exact).  Units u = 32 sb + 4 g + l: super-
// block sb, 32-group g, 8-weight group l.

// byte t of the codebook word g times the group scale, its sign from bit t of s
__device__ __forceinline__ float signed_gw(float db, unsigned g, int t, unsigned s) {
    const float w = db * byte_f(g, t);
    return __builtin_bit_cast(float, __builtin_bit_cast(unsigned, w) ^ ((s << (31 - t)) & 0x80000000u));
}
// the 8 weights of unit u (codebook words lo, hi for weights 0-3, 4-7) against x[8u .. 8u+7]
__device__ __forceinline__ float grid_dot8(float db, unsigned lo, unsigned hi, unsigned s, const Staged& st, int xi) {
    const float4 x0 = x4(st.xs, xi), x1 = x4(st.xs, xi + 4);
    return dot4(signed_gw(db, lo, 0, s), signed_gw(db, lo, 1, s), signed_gw(db, lo, 2, s), signed_gw(db, lo, 3, s), x0) +
           dot4(signed_gw(db, hi, 0, s >> 4), signed_gw(db, hi, 1, s >> 4), signed_gw(db, hi, 2, s >> 4),
                signed_gw(db, hi, 3, s >> 4), x1);
}

// IQ3_XXS (IQ3_XXSFloatTensor.dot, super-blocks of 256 in 98 bytes).  Plane 0 = the 64
// codebook-index bytes [rows][cols/4] (unit u: bytes 2u, 2u+1); plane 1 = each unit's 8 sign
// bits, its 7-bit pattern index expanded with the parity bit at upload (KSIGNS_IQ2XS)
// [rows][cols/8]; plane 2 = per super-block 8 bytes: fp16 d, 2 pad bytes, the eight 4-bit
// group scales (group g: nibble g%2 of byte 4 + g/2).  Table: per super-block the 8 factors
// d * (0.5 + sc) * 0.5.
struct FmtIQ3_XXS {
    static constexpr int UNIT = 8, MAXU = 8, TAB = 8, GRID_BYTES = 256 * 4;
    static constexpr bool XSUM = false, Q8IN = false;
    static __device__ __forceinline__ const void* grid_src() { return kIq3xxsGrid; }
    struct Row { uint2 h; };
    static __device__ __forceinline__ Row load_row(const WPlanes& w, int row, int j, int units) {
        const unsigned sb = (unsigned)min(j, (units >> 5) - 1);
        return Row{ldo<uint2>(rp(w, 2, row), sb * 8u)};
    }
    static __device__ __forceinline__ void build_tab(const Row& r, float* tab, int j, int units) {
        if (j >= (units >> 5)) return;
        const float d = h2f((unsigned short)(r.h.x & 0xFFFFu));
        float v[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) v[g] = (d * (0.5f + (float)((r.h.y >> (4 * g)) & 15u))) * 0.5f;
        float4* t = reinterpret_cast<float4*>(tab + j * TAB);
        t[0] = float4{v[0], v[1], v[2], v[3]};
        t[1] = float4{v[4], v[5], v[6], v[7]};
    }
    struct Raw { unsigned q, s; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ldo<unsigned short>(rp(w, 0, row), (unsigned)u * 2u), ldo<unsigned char>(rp(w, 1, row), (unsigned)u)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const unsigned* g = static_cast<const unsigned*>(st.grid);
        const float db = st.tab[(ub >> 2) + (j >> 2)];
        return grid_dot8(db, g[r.q & 0xFFu], g[r.q >> 8], r.s, st, 8 * ub + 8 * j);
    }
};

// IQ3_S (IQ3_SFloatTensor.dot, super-blocks of 256 in 110 bytes).  Plane 0 = the low index
// bytes qs [rows][cols/4] (unit u: bytes 2u, 2u+1); plane 1 = the sign bytes [rows][cols/8]
// (unit u: byte u); plane 2 = per super-block 16 bytes: qh[8], scales[4], fp16 d, 2 pad.
// Index 2l + h of group g has its ninth bit at bit 2l + h of qh[g/4 + g%2] (the reference's
// OFF_QH + ib32/4, +1 for a pair's second group: IQ3_SFloatTensor.java:131, 145 and
// matmul_iq3_s.cu:129, 158; ggml's own dequantiser reads qh[g]).  Table: per super-block the
// 8 factors d * (1 + 2 sc) (exact: an 11-bit significand times at most 31).
struct FmtIQ3_S {
    // three registers per unit: 8 rounds would spill at the kernel's 5 waves per SIMD
    static constexpr int UNIT = 8, MAXU = 6, TAB = 8, GRID_BYTES = 512 * 4;
    static constexpr bool XSUM = false, Q8IN = false;
    static __device__ __forceinline__ const void* grid_src() { return kIq3sGrid; }
    struct Row { uint4 h; };
    static __device__ __forceinline__ Row load_row(const WPlanes& w, int row, int j, int units) {
        const unsigned sb = (unsigned)min(j, (units >> 5) - 1);
        return Row{ldo<uint4>(rp(w, 2, row), sb * 16u)};
    }
    static __device__ __forceinline__ void build_tab(const Row& r, float* tab, int j, int units) {
        if (j >= (units >> 5)) return;
        const float d = h2f((unsigned short)(r.h.w & 0xFFFFu));
        float v[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) v[g] = d * (float)(1 + 2 * (int)((r.h.z >> (4 * g)) & 15u));
        float4* t = reinterpret_cast<float4*>(tab + j * TAB);
        t[0] = float4{v[0], v[1], v[2], v[3]};
        t[1] = float4{v[4], v[5], v[6], v[7]};
    }
    struct Raw { unsigned q, s, h; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        const unsigned g = ((unsigned)u >> 2) & 7u;
        const unsigned hb = ((unsigned)u >> 5) * 16u + (g >> 2) + (g & 1u);
        return Raw{ldo<unsigned short>(rp(w, 0, row), (unsigned)u * 2u), ldo<unsigned char>(rp(w, 1, row), (unsigned)u),
                   ldo<unsigned char>(rp(w, 2, row), hb)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const unsigned* g = static_cast<const unsigned*>(st.grid);
        const unsigned l2 = 2u * ((unsigned)j & 3u);   // ub is a multiple of 64: l = j % 4
        const unsigned i0 = (r.q & 0xFFu) | (((r.h >> l2) & 1u) << 8);
        const unsigned i1 = (r.q >> 8) | (((r.h >> (l2 + 1u)) & 1u) << 8);
        const float db = st.tab[(ub >> 2) + (j >> 2)];
        return grid_dot8(db, g[i0], g[i1], r.s, st, 8 * ub + 8 * j);
    }
};

// IQ2_S (IQ2_SFloatTensor.dot, super-blocks of 256 in 82 bytes).  Plane 0 = the low index
// bytes qs [rows][cols/8] (unit u: byte u); plane 1 = the sign bytes [rows][cols/8]; plane 2 =
// per super-block 24 bytes: scales[8], qh[8], fp16 d, 6 pad.  Unit u's index has bits 8-9 at
// bits 2l..2l+1 of qh[g].  Table: per super-block the 16 factors d * (0.5 + sc) * 0.25 (low
// nibble of scales[g] for groups l = 0, 1 of g, high nibble for l = 2, 3): entry u/2.
struct FmtIQ2_S {
    static constexpr int UNIT = 8, MAXU = 8, TAB = 16, GRID_BYTES = 1024 * 8;
    static constexpr bool XSUM = false, Q8IN = false;
    static __device__ __forceinline__ const void* grid_src() { return kIq2sGrid; }
    struct Row { uint2 sc; unsigned short d; };
    static __device__ __forceinline__ Row load_row(const WPlanes& w, int row, int j, int units) {
        const unsigned sb = (unsigned)min(j, (units >> 5) - 1);
        return Row{ldo<uint2>(rp(w, 2, row), sb * 24u), ldo<unsigned short>(rp(w, 2, row), sb * 24u + 16u)};
    }
    static __device__ __forceinline__ void build_tab(const Row& r, float* tab, int j, int units) {
        if (j >= (units >> 5)) return;
        const float d = h2f(r.d);
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const unsigned w = k < 8 ? r.sc.x : r.sc.y;
            v[k] = (d * (0.5f + (float)((w >> (4 * (k & 7))) & 15u))) * 0.25f;
        }
        float4* t = reinterpret_cast<float4*>(tab + j * TAB);
#pragma unroll
        for (int c = 0; c < 4; ++c) t[c] = float4{v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]};
    }
    struct Raw { unsigned q, s, h; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        const unsigned hb = ((unsigned)u >> 5) * 24u + 8u + (((unsigned)u >> 2) & 7u);
        return Raw{ldo<unsigned char>(rp(w, 0, row), (unsigned)u), ldo<unsigned char>(rp(w, 1, row), (unsigned)u),
                   ldo<unsigned char>(rp(w, 2, row), hb)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const uint2* g = static_cast<const uint2*>(st.grid);
        const unsigned l2 = 2u * ((unsigned)j & 3u);
        const uint2 e = g[r.q | (((r.h >> l2) & 3u) << 8)];
        const float db = st.tab[(ub >> 1) + (j >> 1)];
        return grid_dot8(db, e.x, e.y, r.s, st, 8 * ub + 8 * j);
    }
};

// ---- Q8_1 input: the reference GPU's int8 matvecs -------------------------------------------
// CudaForwardPass runs its Q4_K and Q8_0 projections (and the formats below) on a Q8_1 copy of
// the input by default (CudaForwardPass.java:783-790, 1998-2037; rmsnorm_quantize.cu, quantize_q8.cu,
// matmul_q4_k_dp4a.cu, matmul_q8_0_dp4a.cu): per 32 values d = max|x|/127, quants rint(x*127/
// max|x|) clamped to +-127, s = sum(x); a block's dot is an exact int8 dot product scaled in
// float.  Here the weights keep the planes of FmtQ4_K / FmtQ8_0; a unit is 8 weight bytes,
// and the products are v_dot4c_i32_i8.

// Quantises chunk c (4 values) of the input into the Q8_1 staging.  The 8 chunks of a block
// are held by 8 consecutive lanes (c = tid + 256k), which must all call this together: the
// block's max and sum are butterflies over them (xor 4, 2, 1; the sum of ((x0 + x1) + (x2 +
// x3)) per lane).  One IEEE division per lane: the group's first lane computes max/127 (the
// block scale), the others 127/max (the quantiser's factor), which the first lane takes from
// the second.  The reference's clamp to +-127 is never active: |x| <= max, so |x * RN(127/max)|
// <= 127 (1 + 2^-24), which rounds to at most 127.
__device__ __forceinline__ void put_q8(int c, const float4& v, unsigned char* xq, float* xd, float* xss) {
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    m = fmaxf(m, __shfl_xor(m, 4));
    m = fmaxf(m, __shfl_xor(m, 2));
    m = fmaxf(m, __shfl_xor(m, 1));
    const bool first = (c & 7) == 0;
    const float quo = first ? m / 127.0f : 127.0f / m;
    const float fac = __shfl_xor(quo, 1);
    const float inv = m > 0.0f ? (first ? fac : quo) : 0.0f;
    auto qb = [&](float a) { return (unsigned)((int)__builtin_rintf(a * inv) & 0xFF); };
    reinterpret_cast<unsigned*>(xq)[c] = qb(v.x) | (qb(v.y) << 8) | (qb(v.z) << 16) | (qb(v.w) << 24);
    float s = (v.x + v.y) + (v.z + v.w);
    s = s + __shfl_xor(s, 4);
    s = s + __shfl_xor(s, 2);
    s = s + __shfl_xor(s, 1);
    if (first) {
        xd[c >> 3] = quo;
        xss[c >> 3] = s;
    }
}

__device__ __forceinline__ int dot4_i8(unsigned a, unsigned b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Q4_K on a Q8_1 input (matmul_q4_k_dp4a.cu's arithmetic).  Unit u: nibble bytes 8u .. 8u+7
// = super-block sb = u/16, group g = (u%16)/4, l = 8(u%4) .. +7: elements 64g + l (sub-block
// 2g, low nibbles) and 64g + 32 + l (sub-block 2g + 1).  Per sub-block s the reference adds
// ((d*sc_s)*d_x)*dp - (dmin*m_s)*s_x; the lane at l = 0 adds the min term for its sub-blocks.
struct FmtQ4_KQ8 {
    static constexpr int UNIT = 16, MAXU = 8, TAB = 16;
    static constexpr bool XSUM = false, Q8IN = true;
    using Row = FmtQ4_K::Row;
    static __device__ __forceinline__ Row load_row(const WPlanes& w, int row, int j, int units) {
        return FmtQ4_K::head(w, row, j, units >> 4);
    }
    static __device__ __forceinline__ void build_tab(const Row& r, float* tab, int j, int units) {
        FmtQ4_K::build_tab_ns(r, tab, j, units >> 4);
    }
    struct Raw { uint2 q; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ldo<uint2>(rp(w, 0, row), (unsigned)u * 8u)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const int g = (j >> 2) & 3, sb = (ub >> 4) + (j >> 4);
        const int i0 = sb * 256 + 64 * g + 8 * (j & 3);
        const uint2 xa = *reinterpret_cast<const uint2*>(st.xq + i0);
        const uint2 xb = *reinterpret_cast<const uint2*>(st.xq + i0 + 32);
        const int dp0 = dot4_i8(r.q.y & 0x0F0F0F0Fu, xa.y, dot4_i8(r.q.x & 0x0F0F0F0Fu, xa.x, 0));
        const int dp1 = dot4_i8((r.q.y >> 4) & 0x0F0F0F0Fu, xb.y,
                                dot4_i8((r.q.x >> 4) & 0x0F0F0F0Fu, xb.x, 0));
        const float4 f = x4(st.tab, sb * TAB + 4 * g);   // (d*sc, dmin*m) of sub-blocks 2g, 2g+1
        const int b0 = sb * 8 + 2 * g;
        const float2 dx = *reinterpret_cast<const float2*>(st.xd + b0);
        const float2 sx = *reinterpret_cast<const float2*>(st.xss + b0);
        const float v = (f.x * dx.x) * (float)dp0 + (f.z * dx.y) * (float)dp1;
        const float mt = (f.y * sx.x) + (f.w * sx.y);
        return (j & 3) == 0 ? v - mt : v;
    }
};

// Q8_0 on a Q8_1 input (matmul_q8_0_dp4a.cu's arithmetic: per block (d*d_x)*dp).  Unit u:
// quants 8u .. 8u+7 of block u/4.
struct FmtQ8_0Q8 {
    static constexpr int UNIT = 8, MAXU = 8, TAB = 0;
    static constexpr bool XSUM = false, Q8IN = true;
    using Row = NoRow;
    static __device__ __forceinline__ Row load_row(const WPlanes&, int, int, int) { return Row{}; }
    static __device__ __forceinline__ void build_tab(const Row&, float*, int, int) {}
    struct Raw { uint2 q; unsigned short d; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ldo<uint2>(rp(w, 0, row), (unsigned)u * 8u),
                   ldo<unsigned short>(rp(w, 1, row), ((unsigned)u >> 2) * 2u)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const int i = 8 * ub + 8 * j;
        const uint2 xa = *reinterpret_cast<const uint2*>(st.xq + i);
        const int dp = dot4_i8(r.q.y, xa.y, dot4_i8(r.q.x, xa.x, 0));
        return (h2f(r.d) * st.xd[i >> 5]) * (float)dp;
    }
};

// The other formats CudaForwardPass runs on the Q8_1 input (:1998-2037: Q5_0, Q3_K, Q5_K, IQ4_NL,
// IQ4_XS; matmul_q5_0_dp4a_smem.cu, matmul_q3_k_dp4a.cu, matmul_q5_k_dp4a.cu,
// matmul_iq4_nl_dp4a.cu, matmul_iq4_xs_dp4a_mw.cu): the weights' integer values as int8, an
// exact int8 dot with the input's quants, and the block's factors in the reference's order:
// (scale * d_x) * dp, Q5_K minus (dmin * m) * s_x.  Units and planes are the fp32-input
// formats'; a unit adds its share of a block's dot, so only the float sum's order differs.

// Bytes holding 5-bit (3-bit) two's complement fields, sign-extended to int8 per byte.
__device__ __forceinline__ unsigned sext5x4(unsigned v) { return v | ((v & 0x10101010u) * 0x0Eu); }
__device__ __forceinline__ unsigned sext3x4(unsigned v) { return v | ((v & 0x04040404u) * 0x3Eu); }

struct FmtQ5_0Q8 {
    static constexpr int UNIT = FmtQ5_0::UNIT, MAXU = 8, TAB = 0;
    static constexpr bool XSUM = false, Q8IN = true;
    using Row = NoRow;
    static __device__ __forceinline__ Row load_row(const WPlanes&, int, int, int) { return Row{}; }
    static __device__ __forceinline__ void build_tab(const Row&, float*, int, int) {}
    using Raw = FmtQ5_0::Raw;
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) { return FmtQ5_0::load(w, row, u); }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const unsigned h = r.qh >> (4 * (j & 3));
        const unsigned lo = sext5x4(((r.q & 0x0F0F0F0Fu) | (spread4(h & 15u) << 4)) ^ 0x10101010u);
        const unsigned hi = sext5x4((((r.q >> 4) & 0x0F0F0F0Fu) | (spread4((h >> 16) & 15u) << 4)) ^ 0x10101010u);
        const int xi = split_x(ub, j);
        const int dp = dot4_i8(hi, *reinterpret_cast<const unsigned*>(st.xq + xi + 16),
                               dot4_i8(lo, *reinterpret_cast<const unsigned*>(st.xq + xi), 0));
        return (h2f(r.d) * st.xd[xi >> 5]) * (float)dp;
    }
};

struct FmtIQ4_NLQ8 {
    static constexpr int UNIT = FmtIQ4_NL::UNIT, MAXU = 8, TAB = 0;
    static constexpr bool XSUM = false, Q8IN = true;
    using Row = NoRow;
    static __device__ __forceinline__ Row load_row(const WPlanes&, int, int, int) { return Row{}; }
    static __device__ __forceinline__ void build_tab(const Row&, float*, int, int) {}
    using Raw = FmtIQ4_NL::Raw;
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) { return FmtIQ4_NL::load(w, row, u); }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const unsigned lo = lut16(r.q & 0x0F0F0F0Fu, kIq4[0], kIq4[1], kIq4[2], kIq4[3]);
        const unsigned hi = lut16((r.q >> 4) & 0x0F0F0F0Fu, kIq4[0], kIq4[1], kIq4[2], kIq4[3]);
        const int xi = split_x(ub, j);
        const int dp = dot4_i8(hi, *reinterpret_cast<const unsigned*>(st.xq + xi + 16),
                               dot4_i8(lo, *reinterpret_cast<const unsigned*>(st.xq + xi), 0));
        return (h2f(r.d) * st.xd[xi >> 5]) * (float)dp;
    }
};

struct FmtIQ4_XSQ8 {
    static constexpr int UNIT = FmtIQ4_XS::UNIT, MAXU = 8, TAB = FmtIQ4_XS::TAB;
    static constexpr bool XSUM = false, Q8IN = true;
    using Row = FmtIQ4_XS::Row;
    static __device__ __forceinline__ Row load_row(const WPlanes& w, int row, int j, int units) {
        return FmtIQ4_XS::load_row(w, row, j, units);
    }
    static __device__ __forceinline__ void build_tab(const Row& r, float* tab, int j, int units) {
        FmtIQ4_XS::build_tab(r, tab, j, units);
    }
    using Raw = FmtIQ4_XS::Raw;
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) { return FmtIQ4_XS::load(w, row, u); }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const float dl = st.tab[(ub >> 2) + (j >> 2)];   // d * (ls - 32) of sub-block (ub + j)/4
        const unsigned lo = lut16(r.q & 0x0F0F0F0Fu, kIq4[0], kIq4[1], kIq4[2], kIq4[3]);
        const unsigned hi = lut16((r.q >> 4) & 0x0F0F0F0Fu, kIq4[0], kIq4[1], kIq4[2], kIq4[3]);
        const int xi = split_x(ub, j);
        const int dp = dot4_i8(hi, *reinterpret_cast<const unsigned*>(st.xq + xi + 16),
                               dot4_i8(lo, *reinterpret_cast<const unsigned*>(st.xq + xi), 0));
        return (dl * st.xd[xi >> 5]) * (float)dp;
    }
};

// Q5_K on the Q8_1 input: FmtQ4_KQ8's units (8 nibble bytes: elements 64g + l .. +7 of
// sub-block 2g and 64g + 32 + l .. of sub-block 2g + 1, l = 8(u%4)) with the fifth bits of qh
// bytes l .. l+7 (bit 2g, 2g + 1) or-ed in.
struct FmtQ5_KQ8 {
    // at most 3 rounds in registers: 4 spilled (the fifth-bit words take 2 more VGPRs a unit)
    static constexpr int UNIT = 16, MAXU = 3, TAB = 16;
    static constexpr bool XSUM = false, Q8IN = true;
    using Row = FmtQ4_K::Row;
    static __device__ __forceinline__ Row load_row(const WPlanes& w, int row, int j, int units) {
        return FmtQ4_K::head(w, row, j, units >> 4);
    }
    static __device__ __forceinline__ void build_tab(const Row& r, float* tab, int j, int units) {
        FmtQ4_K::build_tab_ns(r, tab, j, units >> 4);
    }
    struct Raw { uint2 q, qh; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ldo<uint2>(rp(w, 0, row), (unsigned)u * 8u),
                   ldo<uint2>(rp(w, 2, row), ((unsigned)u >> 4) * 32u + 8u * ((unsigned)u & 3u))};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const int g = (j >> 2) & 3, sb = (ub >> 4) + (j >> 4);
        const int i0 = sb * 256 + 64 * g + 8 * (j & 3);
        const uint2 xa = *reinterpret_cast<const uint2*>(st.xq + i0);
        const uint2 xb = *reinterpret_cast<const uint2*>(st.xq + i0 + 32);
        auto q5 = [&](unsigned q, unsigned h, int s) {
            return ((q >> (4 * s)) & 0x0F0F0F0Fu) | (((h >> (2 * g + s)) & 0x01010101u) << 4);
        };
        const int dp0 = dot4_i8(q5(r.q.y, r.qh.y, 0), xa.y, dot4_i8(q5(r.q.x, r.qh.x, 0), xa.x, 0));
        const int dp1 = dot4_i8(q5(r.q.y, r.qh.y, 1), xb.y, dot4_i8(q5(r.q.x, r.qh.x, 1), xb.x, 0));
        const float4 f = x4(st.tab, sb * TAB + 4 * g);   // (d*sc, dmin*m) of sub-blocks 2g, 2g+1
        const int b0 = sb * 8 + 2 * g;
        const float2 dx = *reinterpret_cast<const float2*>(st.xd + b0);
        const float2 sx = *reinterpret_cast<const float2*>(st.xss + b0);
        const float v = (f.x * dx.x) * (float)dp0 + (f.z * dx.y) * (float)dp1;
        const float mt = (f.y * sx.x) + (f.w * sx.y);
        return (j & 3) == 0 ? v - mt : v;
    }
};

// Q3_K on the Q8_1 input: FmtQ3_K's units (the four 2-bit fields of 4 qs bytes: elements
// 128h + 32p + 16w + l .. +3 for p = 0..3), each field (q - 4) as int8; per p the block
// 8sb + 4h + p's factor (d * (sc - 32)) * d_x.
struct FmtQ3_KQ8 {
    static constexpr int UNIT = FmtQ3_K::UNIT, MAXU = 4, TAB = FmtQ3_K::TAB;
    static constexpr bool XSUM = false, Q8IN = true;
    using Row = FmtQ3_K::Row;
    static __device__ __forceinline__ Row load_row(const WPlanes& w, int row, int j, int units) {
        return FmtQ3_K::load_row(w, row, j, units);
    }
    static __device__ __forceinline__ void build_tab(const Row& r, float* tab, int j, int units) {
        FmtQ3_K::build_tab(r, tab, j, units);
    }
    using Raw = FmtQ3_K::Raw;
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) { return FmtQ3_K::load(w, row, u); }
    static __device__ __forceinline__ float dot(const Raw& r, const Staged& st, int ub, int j) {
        const int h = (j >> 3) & 1, w = (j >> 2) & 1, l = 4 * (j & 3);
        const int sb = (ub >> 4) + (j >> 4);
        const float4 f = x4(st.tab, sb * TAB + (2 * h + w) * 4);
        const float ds[4] = {f.x, f.y, f.z, f.w};
        float s = 0.0f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const unsigned q = sext3x4((((r.qs >> (2 * p)) & 0x03030303u) |
                                        (((r.hm >> (4 * h + p)) & 0x01010101u) << 2)) ^ 0x04040404u);
            const int xi = sb * 256 + 128 * h + 32 * p + 16 * w + l;
            const int dp = dot4_i8(q, *reinterpret_cast<const unsigned*>(st.xq + xi), 0);
            s = s + (ds[p] * st.xd[xi >> 5]) * (float)dp;
        }
        return s;
    }
};

// ---- the kernel ------------------------------------------------------------------------------
// One row per wave: kGemvThreads/64 rows per workgroup, row b*(kGemvThreads/64) + w for wave w
// of workgroup b, so the row, its segment and the unit count are wave-uniform (scalar
// registers).  Lane j takes units j, j+64, ...: NK rounds of units are held in registers (the
// host picks NK from the row width).  Every lane issues all of its loads in one straight
// sequence with no branch between them - the input chunks, the norm weights, the row's side
// data, then its NK weight units (unit indices past the row clamped to its last unit, their
// products dropped) - before it waits for any of them, so the weight reads are in flight while
// the input is reduced and staged.  Rows wider than 64*NK units take further batches of NK
// rounds.  Dynamic LDS (GemvLds::bytes): the staged input, its chunk sums (XSUM formats), and
// one scale table per row of the workgroup (TAB formats).
constexpr int kGemvRowsPerGroup = kGemvThreads / 64;
constexpr int kStageChunks = 4;   // float4 chunks of the input per thread held in registers

// Columns rounded up to whole rounds of 64 units: the lanes past a row's last unit in its last
// round read this padding (their products are dropped).  A launch over two formats lays out
// the larger of each region.
template <class F>
__host__ __device__ constexpr int gemv_cols_padded(int cols) {
    return (cols + 64 * F::UNIT - 1) / (64 * F::UNIT) * (64 * F::UNIT);
}
template <class F1, class F2 = F1>
struct GemvLds {
    static constexpr bool F32X = !F1::Q8IN || !F2::Q8IN;   // some format reads the fp32 input
    static constexpr bool Q8X = F1::Q8IN || F2::Q8IN;      // some format reads the Q8_1 input
    static constexpr bool XSUM = F1::XSUM || F2::XSUM;
    static constexpr int TAB = F1::TAB > F2::TAB ? F1::TAB : F2::TAB;
    // the codebook of a codebook format (a launch pairs no two of them)
    static_assert(FmtGrid<F1>::BYTES == 0 || FmtGrid<F2>::BYTES == 0 || std::is_same<F1, F2>::value,
                  "one codebook per launch");
    static constexpr int GRID = FmtGrid<F1>::BYTES > 0 ? FmtGrid<F1>::BYTES : FmtGrid<F2>::BYTES;
    static __device__ __forceinline__ const void* grid_src() {
        return FmtGrid<F1>::BYTES > 0 ? FmtGrid<F1>::src() : FmtGrid<F2>::src();
    }
    static __host__ __device__ constexpr int cols_padded(int cols) {
        return gemv_cols_padded<F1>(cols) > gemv_cols_padded<F2>(cols) ? gemv_cols_padded<F1>(cols)
                                                                        : gemv_cols_padded<F2>(cols);
    }
    // float offsets of the regions: xs | xsum | xq (bytes) | xd | xss | tables
    static __host__ __device__ constexpr int off_xsum(int cp) { return F32X ? cp : 0; }
    static __host__ __device__ constexpr int off_xq(int cp) { return off_xsum(cp) + (XSUM ? cp / 4 : 0); }
    static __host__ __device__ constexpr int off_xd(int cp) { return off_xq(cp) + (Q8X ? cp / 4 : 0); }
    static __host__ __device__ constexpr int off_xss(int cp) { return off_xd(cp) + (Q8X ? cp / 32 : 0); }
    static __host__ __device__ constexpr int off_tab(int cp) { return off_xss(cp) + (Q8X ? cp / 32 : 0); }
    // the codebook after the tables, 16-byte aligned
    static __host__ __device__ constexpr int off_grid(int cp) {
        return (off_tab(cp) + kGemvRowsPerGroup * (cp / 256) * TAB + 3) / 4 * 4;
    }
    static __host__ __device__ constexpr size_t bytes(int cols) {
        const int cp = cols_padded(cols);
        return sizeof(float) * (size_t)off_grid(cp) + (size_t)GRID;
    }
};

__device__ __forceinline__ GemvSeg seg_of(const GemvArgs& a, int row_g) {
    // row_g is wave-uniform: the selects are scalar and the argument block stays in registers
    const bool in1 = a.nseg > 1 && row_g >= a.seg[1].out_off;
    const bool in2 = a.nseg > 2 && row_g >= a.seg[2].out_off;
    return in2 ? a.seg[2] : (in1 ? a.seg[1] : a.seg[0]);
}

__device__ __forceinline__ void store_row(const GemvArgs& a, const GemvSeg& sg, int row_g, int row,
                                          float acc) {
    float v = acc;
    if (sg.bias != nullptr) v = v + sg.bias[row];
    if (a.resid != nullptr) {
        if (a.rscale > 0.0f) v = v * a.rscale;
        a.resid[row_g] = a.resid[row_g] + v;
    } else {
        a.out[row_g] = v;
    }
}

__device__ __forceinline__ float4 scale4(const float4& v, float r, const float4& w) {
    return float4{(v.x * r) * w.x, (v.y * r) * w.y, (v.z * r) * w.z, (v.w * r) * w.w};
}

// Units whose LDS reads the dot loop lets the scheduler hoist together: four, two for Q6_K
// (four LDS chunks per unit).
template <class F>
constexpr int dot_step() { return (F::UNIT == 16 && !F::Q8IN) ? 2 : 4; }
// the largest divisor of NK not above dot_step
template <class F, int NK>
constexpr int dot_step_of() {
    int s = dot_step<F>() < NK ? dot_step<F>() : NK;
    while (NK % s) --s;
    return s;
}

// One row's registers: the lane's share of the row's side data and NK rounds of units.
template <class F, int NK>
struct RowRegs {
    typename F::Row rw;
    typename F::Raw raw[NK];
};

template <class F, int NK>
__device__ __forceinline__ void row_issue(RowRegs<F, NK>& r, const GemvSeg& sg, int row, int j,
                                          int units) {
    r.rw = F::load_row(sg.w, row, j, units);
#pragma unroll
    for (int k = 0; k < NK; ++k) r.raw[k] = F::load(sg.w, row, min(j + 64 * k, units - 1));
}

// The lane's share of the row's dot product: the NK rounds in registers, then further batches.
template <class F, int NK>
__device__ __forceinline__ float row_dot(RowRegs<F, NK>& r, const Staged& st, const GemvSeg& sg,
                                         int row, int j, int units) {
    float acc = 0.0f;
    for (int base = 0;;) {
        // in steps of a few units, the step loop kept rolled: the scheduler would otherwise
        // hoist every unit's LDS reads to the top and run out of registers
        constexpr int STEP = dot_step_of<F, NK>();
#pragma unroll 1
        for (int h = 0; h < NK / STEP; ++h) {
#pragma unroll
            for (int k = 0; k < STEP; ++k) {
                typename F::Raw rk = r.raw[k];
#pragma unroll
                for (int m = 1; m < NK / STEP; ++m)
                    if (h == m) rk = r.raw[m * STEP + k];
                const int ub = base + 64 * (h * STEP + k);
                const float d = F::dot(rk, st, ub, j);
                acc = acc + (ub + j < units ? d : 0.0f);
            }
        }
        base += 64 * NK;
        if (base >= units) break;   // uniform
#pragma unroll
        for (int k = 0; k < NK; ++k) r.raw[k] = F::load(sg.w, row, min(base + j + 64 * k, units - 1));
    }
    return acc;
}

// y = W x over the rows of up to three segments, with the pre-attention RMSNorm of x (norm_w
// set: 1/(float)sqrt(sum(x^2)/cols + eps), then (x*r)*w as SimdVectorOps.rmsnorm forms it)
// applied while x is staged in LDS.  The segments share one format, or two (F1, NK1 for
// GemvSeg::fmt 0 and F2, NK2 for 1: each wave takes its row's path, a uniform branch).
template <class F1, int NK1, class F2 = F1, int NK2 = NK1>
__global__ __launch_bounds__(kGemvThreads) __attribute__((amdgpu_waves_per_eu(5)))
void gemv_kernel(GemvArgs a) {
    using L = GemvLds<F1, F2>;
    constexpr bool TWO = !(std::is_same<F1, F2>::value && NK1 == NK2);
    extern __shared__ float lds[];
    __shared__ float red[kGemvThreads / 64];
    const int tid = threadIdx.x, j = tid & 63, wave = tid >> 6;
    const int row_g = __builtin_amdgcn_readfirstlane(blockIdx.x * kGemvRowsPerGroup + wave);
    const bool live = row_g < a.rows_total;
    const int row_c = live ? row_g : a.rows_total - 1;   // spare waves load a valid row
    const GemvSeg sg = seg_of(a, row_c);
    const int row = row_c - sg.out_off;
    const bool second = TWO && sg.fmt != 0;
    const int units1 = a.cols / F1::UNIT, units2 = a.cols / F2::UNIT;
    const int n4 = a.cols >> 2;
    const int cp = L::cols_padded(a.cols);
    float* xs = lds;
    float* xsum = lds + L::off_xsum(cp);
    unsigned char* xq = reinterpret_cast<unsigned char*>(lds + L::off_xq(cp));
    float* xd = lds + L::off_xd(cp);
    float* xss = lds + L::off_xss(cp);
    float* tab = lds + L::off_tab(cp) + wave * (cp / 256) * L::TAB;
    uint4* grid = reinterpret_cast<uint4*>(lds + L::off_grid(cp));

    // input chunks and norm weights (chunk c = tid + 256k, clamped to the last chunk)
    const bool norm = a.norm_w != nullptr;
    const float4* x4g = reinterpret_cast<const float4*>(a.x);
    const float4* w4g = reinterpret_cast<const float4*>(norm ? a.norm_w : a.x);
    float4 xv[kStageChunks], wv[kStageChunks];
#pragma unroll
    for (int k = 0; k < kStageChunks; ++k) {
        const int c = min(tid + k * kGemvThreads, n4 - 1);
        xv[k] = x4g[c];
        wv[k] = w4g[c];
    }
    // the codebook (codebook formats), 16 bytes per thread per trip, in flight with the input
    constexpr int GRID_TRIPS = (L::GRID / 16 + kGemvThreads - 1) / kGemvThreads;
    uint4 gv[GRID_TRIPS > 0 ? GRID_TRIPS : 1];
#pragma unroll
    for (int k = 0; k < GRID_TRIPS; ++k)
        gv[k] = static_cast<const uint4*>(L::grid_src())[min(tid + k * kGemvThreads, L::GRID / 16 - 1)];
    __builtin_amdgcn_sched_barrier(0);   // keep the input loads ahead of the weight loads
    // the row's side data, then the weight units
    RowRegs<F1, NK1> r1;
    RowRegs<F2, NK2> r2;
    if (!second) row_issue(r1, sg, row, j, units1);
    else row_issue(r2, sg, row, j, units2);

    // sum of squares of x (chunks beyond the registers: a second read, from cache)
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kStageChunks; ++k)
        if (tid + k * kGemvThreads < n4) {
            ss = __builtin_fmaf(xv[k].x, xv[k].x, ss);
            ss = __builtin_fmaf(xv[k].y, xv[k].y, ss);
            ss = __builtin_fmaf(xv[k].z, xv[k].z, ss);
            ss = __builtin_fmaf(xv[k].w, xv[k].w, ss);
        }
    for (int c = tid + kStageChunks * kGemvThreads; c < n4; c += kGemvThreads) {
        const float4 v = x4g[c];
        ss = __builtin_fmaf(v.x, v.x, ss);
        ss = __builtin_fmaf(v.y, v.y, ss);
        ss = __builtin_fmaf(v.z, v.z, ss);
        ss = __builtin_fmaf(v.w, v.w, ss);
    }
    // SimdVectorOps.rmsnorm's scale r from the waves' partial sums (read after a barrier).
    auto rms_factor = [&]() {
        float tot = red[0];
#pragma unroll
        for (int w = 1; w < kGemvThreads / 64; ++w) tot = tot + red[w];
        float v = tot / (float)a.cols;
        v = v + a.eps;
        return 1.0f / (float)__builtin_sqrt((double)v);
    };
    // Without a Q8_1 staging (which quantises the normalised input itself) r multiplies each
    // row's dot product instead: W ((x w) r) = (W (x w)) r, one rounding apart from the CPU
    // path's (x r) w, so staging needs no barrier of its own before the dot's.
    constexpr bool LATE_R = !L::Q8X;
    float r = 1.0f;
    if (norm) {
        ss = dk::row_group_sum<64>(ss);   // pairs at lane distance 1, 2, 4, ..., 32 (DPP, permlane)
        if (j == 0) red[wave] = ss;
        if constexpr (!LATE_R) {
            __syncthreads();
            r = rms_factor();
        }
    }
    float4* xs4 = reinterpret_cast<float4*>(xs);
    auto put = [&](int c, const float4& v) {   // the 8 lanes of a Q8_1 block call together
        if (L::F32X) {
            xs4[c] = v;
            if (L::XSUM) xsum[c] = (v.x + v.y) + (v.z + v.w);
        }
        if (L::Q8X) put_q8(c, v, xq, xd, xss);
    };
#pragma unroll
    for (int k = 0; k < kStageChunks; ++k) {
        const int c = tid + k * kGemvThreads;
        if (c < n4) put(c, norm ? scale4(xv[k], r, wv[k]) : xv[k]);
    }
    for (int c = tid + kStageChunks * kGemvThreads; c < n4; c += kGemvThreads)
        put(c, norm ? scale4(x4g[c], r, w4g[c]) : x4g[c]);
    if (!second) F1::build_tab(r1.rw, tab, j, units1);
    else F2::build_tab(r2.rw, tab, j, units2);
#pragma unroll
    for (int k = 0; k < GRID_TRIPS; ++k)
        if (tid + k * kGemvThreads < L::GRID / 16) grid[tid + k * kGemvThreads] = gv[k];
    __syncthreads();
    if (LATE_R && norm) r = rms_factor();

    const Staged st{xs, xsum, tab, xq, xd, xss, grid};
    float acc = !second ? row_dot(r1, st, sg, row, j, units1) : row_dot(r2, st, sg, row, j, units2);
    acc = dk::row_group_sum<64>(acc);
    if (LATE_R) acc = acc * r;
    if (live && j == 0) store_row(a, sg, row_g, row, acc);
}

// Post-attention norm and residual (Gemma 2/3, OLMo2: TransformerBlock.forward):
// xb = rmsnorm(xb, w); xb *= rscale (Granite, when > 0); x += xb.  One workgroup per token
// (rows dim floats apart).
constexpr int kPostThreads = 1024;
template <int NTHR>
__global__ __launch_bounds__(NTHR) void post_norm_residual_kernel(const float* xb, const float* w,
                                                                  float eps, float rscale, float* x,
                                                                  int dim) {
    constexpr int kPostThreads = NTHR;
    __shared__ float red[kPostThreads / 64];
    const int tid = threadIdx.x;
    xb += (long long)blockIdx.x * dim;
    x += (long long)blockIdx.x * dim;
    float ss = 0.0f;
    for (int i = tid; i < dim; i += kPostThreads) ss = __builtin_fmaf(xb[i], xb[i], ss);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss = ss + __shfl_xor(ss, off);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float tot = red[0];
#pragma unroll
    for (int k = 1; k < kPostThreads / 64; ++k) tot = tot + red[k];
    float v = tot / (float)dim;
    v = v + eps;
    const float r = 1.0f / (float)__builtin_sqrt((double)v);
    for (int i = tid; i < dim; i += kPostThreads) {
        float o = (xb[i] * r) * w[i];
        if (rscale > 0.0f) o = o * rscale;
        x[i] = x[i] + o;
    }
}

}  // namespace gk
}  // namespace llmp
