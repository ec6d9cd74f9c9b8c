// Matrix-vector products over GGUF-format projection weights (the attention half's Q/K/V and
// output projections, Attention.java:76-110, 232-238; reference GPU: the matmul_* kernels
// launched from CudaForwardPass.forwardAttentionPart, CudaForwardPass.java:1498-1515, 1572).
//
// Decode is one token: y = W x is bound by the weight bytes read from HBM.  The host repacks
// each GGUF tensor at upload into per-row planes so that every lane reads 16-byte aligned
// chunks (see the plane list of each format below); x (fp32, at most 16384 values) is staged
// once per workgroup in LDS, with the pre-attention RMSNorm applied while staging.  LPR lanes
// share a row; lane j takes the row's units j, j+LPR, ... (a unit is 8 to 64 weights); the
// LPR partial sums are reduced in registers (DPP and permlane steps).  Dequantised weights
// equal the reference tensor classes' values; the dot's summation order differs from the CPU
// path's, so projections match it to a tolerance, not bit for bit.
#pragma once

#include "decode_kernels.h"

namespace llmp {
namespace gk {

// GGMLType ids (GGMLType.java:4-35) of the formats with a kernel here.
constexpr int kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14, kBF16 = 30;

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
};

constexpr int kGemvThreads = 256;
constexpr int kMaxGemvCols = 16384;

struct GemvArgs {
    GemvSeg seg[3];        // same format; rows [out_off, out_off + rows) of the output
    int nseg;
    int rows_total;
    int cols;
    const float* x;        // [cols]
    const float* norm_w;   // fused pre-norm weights [cols] (SimdVectorOps.rmsnorm), or nullptr
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

__device__ __forceinline__ u32x4 ld16(const unsigned char* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

// ---- formats ---------------------------------------------------------------------------------
// F32: plane 0 = [rows][cols] fp32.  Unit: 8 weights (two 16-byte loads).
struct FmtF32 {
    static constexpr int UNIT = 8;
    struct Raw { u32x4 a, b; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        const unsigned char* p = w.p[0] + row * w.pitch[0] + u * 32;
        return Raw{ld16(p), ld16(p + 16)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* xs, int u) {
        const float* x = xs + u * 8;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) s = __builtin_fmaf(__uint_as_float(r.a[i]), x[i], s);
#pragma unroll
        for (int i = 0; i < 4; ++i) s = __builtin_fmaf(__uint_as_float(r.b[i]), x[4 + i], s);
        return s;
    }
};

// F16 / BF16: plane 0 = [rows][cols] 16-bit.  Unit: 8 weights (one 16-byte load).
template <bool BF>
struct FmtHalf {
    static constexpr int UNIT = 8;
    struct Raw { u32x4 a; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{ld16(w.p[0] + row * w.pitch[0] + u * 16)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* xs, int u) {
        const float* x = xs + u * 8;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const unsigned v = r.a[i];
            const float w0 = BF ? bf2f((unsigned short)(v & 0xFFFF)) : h2f((unsigned short)(v & 0xFFFF));
            const float w1 = BF ? bf2f((unsigned short)(v >> 16)) : h2f((unsigned short)(v >> 16));
            s = __builtin_fmaf(w0, x[2 * i], s);
            s = __builtin_fmaf(w1, x[2 * i + 1], s);
        }
        return s;
    }
};

// Q8_0: plane 0 = quants [rows][cols] int8, plane 1 = scales [rows][cols/32] fp16.
// Unit: one block of 32 (two 16-byte loads and its scale): d * sum(q * x).
struct FmtQ8_0 {
    static constexpr int UNIT = 32;
    struct Raw { u32x4 a, b; unsigned short d; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        const unsigned char* p = w.p[0] + row * w.pitch[0] + u * 32;
        const unsigned short d =
            reinterpret_cast<const unsigned short*>(w.p[1] + row * w.pitch[1])[u];
        return Raw{ld16(p), ld16(p + 16), d};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* xs, int u) {
        const float* x = xs + u * 32;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const unsigned v = i < 4 ? r.a[i] : r.b[i - 4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                s = __builtin_fmaf((float)(signed char)((v >> (8 * k)) & 0xFF), x[4 * i + k], s);
        }
        return h2f(r.d) * s;
    }
};

// Q4_0: plane 0 = nibbles [rows][cols/2] (byte i: element 2i low, 2i+1 high, as
// Q4_0FloatTensor reads them), plane 1 = scales [rows][cols/32] fp16.
// Unit: one block of 32: d * sum((q - 8) * x).
struct FmtQ4_0 {
    static constexpr int UNIT = 32;
    struct Raw { u32x4 a; unsigned short d; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        const unsigned short d =
            reinterpret_cast<const unsigned short*>(w.p[1] + row * w.pitch[1])[u];
        return Raw{ld16(w.p[0] + row * w.pitch[0] + u * 16), d};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* xs, int u) {
        const float* x = xs + u * 32;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const unsigned v = r.a[i];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const unsigned b = (v >> (8 * k)) & 0xFF;
                s = __builtin_fmaf((float)((int)(b & 15) - 8), x[8 * i + 2 * k], s);
                s = __builtin_fmaf((float)((int)(b >> 4) - 8), x[8 * i + 2 * k + 1], s);
            }
        }
        return h2f(r.d) * s;
    }
};

// Q4_K: plane 0 = the 128 nibble bytes of each super-block in the GGUF order (byte 32g + l:
// element 64g + l low, 64g + 32 + l high), plane 1 = the 16-byte head of each super-block
// (d, dmin fp16, 12 bytes of 6-bit scales and mins).  Unit: 16 nibble bytes = elements
// 64g + 16c + i (sub-block 2g) and 64g + 32 + 16c + i (sub-block 2g + 1), i < 16:
// d*sc*sum(q x) - dmin*m*sum(x) per sub-block half (Q4_KFloatTensor.dot's values).
struct FmtQ4_K {
    static constexpr int UNIT = 32;
    struct Raw { u32x4 q, h; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        const int sb = u >> 3;
        return Raw{ld16(w.p[0] + row * w.pitch[0] + u * 16), ld16(w.p[1] + row * w.pitch[1] + sb * 16)};
    }
    static __device__ __forceinline__ int byte_of(const u32x4& v, int i) {
        return (int)((v[i >> 2] >> (8 * (i & 3))) & 0xFF);
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* xs, int u) {
        const int sb = u >> 3, k = u & 7, g = k >> 1, c = k & 1;
        const float d = h2f((unsigned short)(r.h[0] & 0xFFFF));
        const float dmin = h2f((unsigned short)(r.h[0] >> 16));
        // scale/min of sub-blocks s0 = 2g and s1 = 2g + 1 (bytes 4..15 of the head)
        int sc[2], mn[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int s = 2 * g + t;
            if (s < 4) {
                sc[t] = byte_of(r.h, 4 + s) & 63;
                mn[t] = byte_of(r.h, 8 + s) & 63;
            } else {
                sc[t] = (byte_of(r.h, 8 + s) & 15) | ((byte_of(r.h, s) >> 6) << 4);
                mn[t] = (byte_of(r.h, 8 + s) >> 4) | ((byte_of(r.h, 4 + s) >> 6) << 4);
            }
        }
        const float* x0 = xs + sb * 256 + g * 64 + c * 16;
        const float* x1 = x0 + 32;
        float s0 = 0.0f, s1 = 0.0f, t0 = 0.0f, t1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int b = byte_of(r.q, i);
            s0 = __builtin_fmaf((float)(b & 15), x0[i], s0);
            s1 = __builtin_fmaf((float)(b >> 4), x1[i], s1);
            t0 = t0 + x0[i];
            t1 = t1 + x1[i];
        }
        const float ds0 = d * (float)sc[0], dm0 = dmin * (float)mn[0];
        const float ds1 = d * (float)sc[1], dm1 = dmin * (float)mn[1];
        return (ds0 * s0 - dm0 * t0) + (ds1 * s1 - dm1 * t1);
    }
};

// Q6_K: plane 0 = ql (128 bytes per super-block), plane 1 = qh (64), plane 2 = scales (16
// int8), plane 3 = d (fp16), each in the GGUF order.  Unit (h, j) of a super-block: l in
// [16j, 16j + 16) of half h for the four quarters c, i.e. elements 128h + 32c + l, read from
// ql[64h + l], ql[64h + 32 + l], qh[32h + l] (three 16-byte loads) with scales
// sc[8h + j + 2c]: sum over c of d*sc*sum((q - 32) x) (Q6_KFloatTensor.dot's values).
struct FmtQ6_K {
    static constexpr int UNIT = 64;
    struct Raw { u32x4 l0, l1, h; unsigned s01, s23; unsigned short d; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        const int sb = u >> 2, h = (u >> 1) & 1, j = u & 1;
        const unsigned char* ql = w.p[0] + row * w.pitch[0] + sb * 128 + 64 * h + 16 * j;
        const unsigned char* qh = w.p[1] + row * w.pitch[1] + sb * 64 + 32 * h + 16 * j;
        const unsigned char* sc = w.p[2] + row * w.pitch[2] + sb * 16 + 8 * h;
        const unsigned* sw = reinterpret_cast<const unsigned*>(sc);
        const unsigned short d = reinterpret_cast<const unsigned short*>(w.p[3] + row * w.pitch[3])[sb];
        return Raw{ld16(ql), ld16(ql + 32), ld16(qh), sw[0], sw[1], d};
    }
    static __device__ __forceinline__ int byte_of(const u32x4& v, int i) {
        return (int)((v[i >> 2] >> (8 * (i & 3))) & 0xFF);
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* xs, int u) {
        const int sb = u >> 2, h = (u >> 1) & 1, j = u & 1;
        const float d = h2f(r.d);
        // sc[8h + j + 2c], c = 0..3: bytes j, j+2 of the first word and j, j+2 of the second
        const int scv[4] = {(signed char)((r.s01 >> (8 * j)) & 0xFF),
                            (signed char)((r.s01 >> (8 * (j + 2))) & 0xFF),
                            (signed char)((r.s23 >> (8 * j)) & 0xFF),
                            (signed char)((r.s23 >> (8 * (j + 2))) & 0xFF)};
        const float* x = xs + sb * 256 + 128 * h + 16 * j;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int a = byte_of(r.l0, i), b = byte_of(r.l1, i), hb = byte_of(r.h, i);
            const int q0 = (a & 15) | ((hb & 3) << 4);
            const int q1 = (b & 15) | (((hb >> 2) & 3) << 4);
            const int q2 = (a >> 4) | (((hb >> 4) & 3) << 4);
            const int q3 = (b >> 4) | (((hb >> 6) & 3) << 4);
            acc[0] = __builtin_fmaf((float)(q0 - 32), x[i], acc[0]);
            acc[1] = __builtin_fmaf((float)(q1 - 32), x[32 + i], acc[1]);
            acc[2] = __builtin_fmaf((float)(q2 - 32), x[64 + i], acc[2]);
            acc[3] = __builtin_fmaf((float)(q3 - 32), x[96 + i], acc[3]);
        }
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) s = s + (d * (float)scv[c]) * acc[c];
        return s;
    }
};

// ---- the kernel ------------------------------------------------------------------------------
// Workgroup: kGemvThreads threads = kGemvThreads/LPR row groups; row group r of workgroup b
// computes output row b*(kGemvThreads/LPR) + r.  The input is staged in LDS first (fused
// RMSNorm when norm_w is set: 1/(float)sqrt(sum(x^2)/cols + eps), then (x*r)*w as
// SimdVectorOps.rmsnorm forms it).
// Dynamic LDS: cols floats.
template <class F, int LPR>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs a) {
    extern __shared__ float xs[];
    __shared__ float red[kGemvThreads / 64];
    const int tid = threadIdx.x;
    const int cols = a.cols;
    if (a.norm_w != nullptr) {
        float ss = 0.0f;
        for (int i = tid; i < cols; i += kGemvThreads) ss = __builtin_fmaf(a.x[i], a.x[i], ss);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss = ss + __shfl_xor(ss, off);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float tot = red[0];
#pragma unroll
        for (int w = 1; w < kGemvThreads / 64; ++w) tot = tot + red[w];
        float v = tot / (float)cols;
        v = v + a.eps;
        const float r = 1.0f / (float)__builtin_sqrt((double)v);
        for (int i = tid; i < cols; i += kGemvThreads) xs[i] = (a.x[i] * r) * a.norm_w[i];
    } else {
        for (int i = tid; i < cols; i += kGemvThreads) xs[i] = a.x[i];
    }
    __syncthreads();

    constexpr int GROUPS = kGemvThreads / LPR;
    const int grp = tid / LPR, j = tid - grp * LPR;
    const int row_g = blockIdx.x * GROUPS + grp;
    if (row_g >= a.rows_total) return;
    // segment of this row (a uniform select keeps the argument block out of scratch)
    const bool in1 = a.nseg > 1 && row_g >= a.seg[1].out_off;
    const bool in2 = a.nseg > 2 && row_g >= a.seg[2].out_off;
    const GemvSeg sg = in2 ? a.seg[2] : (in1 ? a.seg[1] : a.seg[0]);
    const int row = row_g - sg.out_off;
    const int units = cols / F::UNIT;
    float acc = 0.0f;
    int u = j;
    for (; u + LPR < units; u += 2 * LPR) {   // two units in flight per lane
        const typename F::Raw r0 = F::load(sg.w, row, u);
        const typename F::Raw r1 = F::load(sg.w, row, u + LPR);
        acc = acc + F::dot(r0, xs, u);
        acc = acc + F::dot(r1, xs, u + LPR);
    }
    if (u < units) acc = acc + F::dot(F::load(sg.w, row, u), xs, u);
    acc = dk::row_group_sum<LPR>(acc);
    if (j == 0) {
        float v = acc;
        if (sg.bias != nullptr) v = v + sg.bias[row];
        if (a.resid != nullptr) {
            if (a.rscale > 0.0f) v = v * a.rscale;
            a.resid[row_g] = a.resid[row_g] + v;
        } else {
            a.out[row_g] = v;
        }
    }
}

// Post-attention norm and residual (Gemma 2/3, OLMo2: TransformerBlock.forward):
// xb = rmsnorm(xb, w); xb *= rscale (Granite, when > 0); x += xb.  One workgroup.
constexpr int kPostThreads = 1024;
template <int NTHR>
__global__ __launch_bounds__(NTHR) void post_norm_residual_kernel(const float* xb, const float* w,
                                                                  float eps, float rscale, float* x,
                                                                  int dim) {
    constexpr int kPostThreads = NTHR;
    __shared__ float red[kPostThreads / 64];
    const int tid = threadIdx.x;
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
