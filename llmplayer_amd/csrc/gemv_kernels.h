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

__device__ __forceinline__ u32x4 ld16(const unsigned char* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

// ---- formats ---------------------------------------------------------------------------------
// A lane unit is a few bytes of one row's quants: consecutive lanes take consecutive units, so
// a wave's weight loads are contiguous, and the x values a unit needs are 16-byte chunks that
// consecutive lanes read from consecutive LDS addresses (no bank conflicts).
__device__ __forceinline__ const float4& x4(const float* xs, int i) {
    return *reinterpret_cast<const float4*>(xs + i);
}
__device__ __forceinline__ float dot4(float a, float b, float c, float d, const float4& x) {
    return __builtin_fmaf(d, x.w, __builtin_fmaf(c, x.z, __builtin_fmaf(b, x.y, a * x.x)));
}

// F32: plane 0 = [rows][cols] fp32.  Unit u: weights 4u .. 4u+3 (one 16-byte load).
struct FmtF32 {
    static constexpr int UNIT = 4;
    static constexpr int MAXU = 8;   // units a lane holds in registers
    struct Raw { float4 w; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{*reinterpret_cast<const float4*>(w.p[0] + row * w.pitch[0] + u * 16)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* xs, int u) {
        return dot4(r.w.x, r.w.y, r.w.z, r.w.w, x4(xs, 4 * u));
    }
};

// F16 / BF16: plane 0 = [rows][cols] 16-bit.  Unit u: weights 4u .. 4u+3 (one 8-byte load).
template <bool BF>
struct FmtHalf {
    static constexpr int UNIT = 4;
    static constexpr int MAXU = 16;
    struct Raw { uint2 w; };
    static __device__ __forceinline__ float cvt(unsigned short h) { return BF ? bf2f(h) : h2f(h); }
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{*reinterpret_cast<const uint2*>(w.p[0] + row * w.pitch[0] + u * 8)};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* xs, int u) {
        return dot4(cvt((unsigned short)(r.w.x & 0xFFFF)), cvt((unsigned short)(r.w.x >> 16)),
                    cvt((unsigned short)(r.w.y & 0xFFFF)), cvt((unsigned short)(r.w.y >> 16)),
                    x4(xs, 4 * u));
    }
};

// Q8_0: plane 0 = quants [rows][cols] int8, plane 1 = scales [rows][cols/32] fp16.
// Unit u: quants 4u .. 4u+3 of block u/8: d * sum(q * x).
struct FmtQ8_0 {
    static constexpr int UNIT = 4;
    static constexpr int MAXU = 16;
    struct Raw { unsigned q; unsigned short d; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{*reinterpret_cast<const unsigned*>(w.p[0] + row * w.pitch[0] + u * 4),
                   reinterpret_cast<const unsigned short*>(w.p[1] + row * w.pitch[1])[u >> 3]};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* xs, int u) {
        const float s = dot4((float)(signed char)(r.q & 0xFF), (float)(signed char)((r.q >> 8) & 0xFF),
                             (float)(signed char)((r.q >> 16) & 0xFF), (float)(signed char)(r.q >> 24),
                             x4(xs, 4 * u));
        return h2f(r.d) * s;
    }
};

// Q4_0: plane 0 = nibbles [rows][cols/2] (byte i: element 2i low, 2i+1 high, as
// Q4_0FloatTensor reads them), plane 1 = scales [rows][cols/32] fp16.
// Unit u: nibble bytes 4u .. 4u+3 = elements 8u .. 8u+7 of block u/4: d * sum((q - 8) x).
struct FmtQ4_0 {
    static constexpr int UNIT = 8;
    static constexpr int MAXU = 16;
    struct Raw { unsigned q; unsigned short d; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{*reinterpret_cast<const unsigned*>(w.p[0] + row * w.pitch[0] + u * 4),
                   reinterpret_cast<const unsigned short*>(w.p[1] + row * w.pitch[1])[u >> 2]};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* xs, int u) {
        const unsigned q = r.q;
        auto n = [&](int k) { return (float)((int)((q >> (4 * k)) & 15) - 8); };
        const float s = dot4(n(0), n(1), n(2), n(3), x4(xs, 8 * u)) +
                        dot4(n(4), n(5), n(6), n(7), x4(xs, 8 * u + 4));
        return h2f(r.d) * s;
    }
};

// Q4_K: plane 0 = the 128 nibble bytes of each super-block in the GGUF order (byte 32g + l:
// element 64g + l low, 64g + 32 + l high), plane 1 = the 16-byte head of each super-block
// (d, dmin fp16, 12 bytes of 6-bit scales and mins).  Unit u: nibble bytes 4u .. 4u+3 =
// super-block sb = u/32, group g = (u%32)/8, l = 4(u%8) .. +3: elements 64g + l (sub-block
// 2g) and 64g + 32 + l (sub-block 2g + 1); value d*sc*q - dmin*m (Q4_KFloatTensor.dot).
struct FmtQ4_K {
    static constexpr int UNIT = 8;
    static constexpr int MAXU = 8;
    struct Raw { unsigned q; u32x4 h; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        return Raw{*reinterpret_cast<const unsigned*>(w.p[0] + row * w.pitch[0] + u * 4),
                   ld16(w.p[1] + row * w.pitch[1] + (u >> 5) * 16)};
    }
    static __device__ __forceinline__ int byte_of(const u32x4& v, int i) {
        return (int)((v[i >> 2] >> (8 * (i & 3))) & 0xFF);
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* xs, int u) {
        const int sb = u >> 5, g = (u >> 3) & 3, l = 4 * (u & 7);
        const float d = h2f((unsigned short)(r.h[0] & 0xFFFF));
        const float dmin = h2f((unsigned short)(r.h[0] >> 16));
        int sc[2], mn[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int s = 2 * g + t;   // bytes 4..15 of the head are the 12 scale bytes
            if (s < 4) {
                sc[t] = byte_of(r.h, 4 + s) & 63;
                mn[t] = byte_of(r.h, 8 + s) & 63;
            } else {
                sc[t] = (byte_of(r.h, 8 + s) & 15) | ((byte_of(r.h, s) >> 6) << 4);
                mn[t] = (byte_of(r.h, 8 + s) >> 4) | ((byte_of(r.h, 4 + s) >> 6) << 4);
            }
        }
        const unsigned q = r.q;
        const float4& x0 = x4(xs, sb * 256 + 64 * g + l);
        const float4& x1 = x4(xs, sb * 256 + 64 * g + 32 + l);
        const float s0 = dot4((float)(q & 15), (float)((q >> 8) & 15), (float)((q >> 16) & 15),
                              (float)((q >> 24) & 15), x0);
        const float s1 = dot4((float)((q >> 4) & 15), (float)((q >> 12) & 15), (float)((q >> 20) & 15),
                              (float)(q >> 28), x1);
        const float t0 = (x0.x + x0.y) + (x0.z + x0.w), t1 = (x1.x + x1.y) + (x1.z + x1.w);
        const float ds0 = d * (float)sc[0], dm0 = dmin * (float)mn[0];
        const float ds1 = d * (float)sc[1], dm1 = dmin * (float)mn[1];
        return (ds0 * s0 - dm0 * t0) + (ds1 * s1 - dm1 * t1);
    }
};

// Q6_K: plane 0 = ql (128 bytes per super-block), plane 1 = qh (64), plane 2 = scales (16
// int8), plane 3 = d (fp16), each in the GGUF order.  Unit u: super-block sb = u/16, half
// h = (u%16)/8, l = 4(u%8) .. +3 for the four quarters c: elements 128h + 32c + l, from the ql
// words at 64h + l and 64h + 32 + l and the qh word at 32h + l, scales sc[8h + l/16 + 2c]
// (Q6_KFloatTensor.dot's values d*sc*(q - 32)).
struct FmtQ6_K {
    static constexpr int UNIT = 16;
    static constexpr int MAXU = 8;
    struct Raw { unsigned l0, l1, qh, s01, s23; unsigned short d; };
    static __device__ __forceinline__ Raw load(const WPlanes& w, int row, int u) {
        const int sb = u >> 4, h = (u >> 3) & 1, l = 4 * (u & 7);
        const unsigned char* ql = w.p[0] + row * w.pitch[0] + sb * 128 + 64 * h + l;
        const unsigned* sw =
            reinterpret_cast<const unsigned*>(w.p[2] + row * w.pitch[2] + sb * 16 + 8 * h);
        return Raw{*reinterpret_cast<const unsigned*>(ql), *reinterpret_cast<const unsigned*>(ql + 32),
                   *reinterpret_cast<const unsigned*>(w.p[1] + row * w.pitch[1] + sb * 64 + 32 * h + l),
                   sw[0], sw[1],
                   reinterpret_cast<const unsigned short*>(w.p[3] + row * w.pitch[3])[sb]};
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* xs, int u) {
        const int sb = u >> 4, h = (u >> 3) & 1, l = 4 * (u & 7), j = (u & 7) >> 2;   // j = l/16
        const float d = h2f(r.d);
        // sc[8h + j + 2c]: bytes j, j+2 of the first scale word (c = 0, 1), of the second (c = 2, 3)
        const float ds[4] = {d * (float)(signed char)((r.s01 >> (8 * j)) & 0xFF),
                             d * (float)(signed char)((r.s01 >> (8 * (j + 2))) & 0xFF),
                             d * (float)(signed char)((r.s23 >> (8 * j)) & 0xFF),
                             d * (float)(signed char)((r.s23 >> (8 * (j + 2))) & 0xFF)};
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const unsigned lo = (c & 1) ? r.l1 : r.l0;
            const int nib = (c >> 1) * 4;   // c = 0, 1: low nibbles; c = 2, 3: high nibbles
            float q[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int v = (int)((lo >> (8 * t + nib)) & 15) | (int)(((r.qh >> (8 * t + 2 * c)) & 3) << 4);
                q[t] = (float)(v - 32);
            }
            s = s + ds[c] * dot4(q[0], q[1], q[2], q[3], x4(xs, sb * 256 + 128 * h + 32 * c + l));
        }
        return s;
    }
};

// ---- the kernel ------------------------------------------------------------------------------
// Workgroup: kGemvThreads threads = kGemvThreads/LPR row groups; row group r of workgroup b
// computes output row b*(kGemvThreads/LPR) + r.  Each lane first issues the loads of its
// units (up to F::MAXU, then the rest in a loop), so the weight reads are in flight while the
// input is staged in LDS, RMS-normalised when norm_w is set (1/(float)sqrt(sum(x^2)/cols + eps),
// then (x*r)*w as SimdVectorOps.rmsnorm forms it).  Dynamic LDS: cols floats, 16-byte aligned.
// Dot of one row's lane units with the staged input: the first F::MAXU units come from
// registers loaded at kernel entry, wider rows load the rest in a loop.
template <class F, int LPR>
__device__ __forceinline__ float row_dot(const typename F::Raw (&raw)[F::MAXU], int nu,
                                         const GemvSeg& sg, int row, int j, int units,
                                         const float* xs) {
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < F::MAXU; ++k)
        if (k < nu) acc = acc + F::dot(raw[k], xs, j + k * LPR);
    for (int u = j + F::MAXU * LPR; u < units; u += LPR)
        acc = acc + F::dot(F::load(sg.w, row, u), xs, u);
    return acc;
}

template <class F, int LPR>
__device__ __forceinline__ void row_load(typename F::Raw (&raw)[F::MAXU], int nu, const GemvSeg& sg,
                                         int row, int j) {
#pragma unroll
    for (int k = 0; k < F::MAXU; ++k)
        if (k < nu) raw[k] = F::load(sg.w, row, j + k * LPR);
}

// Input staging: each thread copies float4 chunks c = tid, tid + 256, ... of x into LDS,
// with the loads of up to four chunks in flight together, and sums their squares; with a
// pre-norm, the norm weights of its first four chunks are loaded before the reduction so that
// their latency overlaps it, then each thread scales the chunks it wrote (its own LDS values:
// no barrier needed).  cols is a multiple of 4.  Ends with a barrier.
__device__ __forceinline__ void stage_input(const GemvArgs& a, float* xs, int tid) {
    constexpr int XV = 4;
    const int cols = a.cols, n4 = cols >> 2;
    const float4* x4g = reinterpret_cast<const float4*>(a.x);
    const float4* w4g = reinterpret_cast<const float4*>(a.norm_w);
    float4* xs4 = reinterpret_cast<float4*>(xs);
    float ss = 0.0f;
    for (int base = tid; base < n4; base += XV * kGemvThreads) {
        float4 xv[XV];
#pragma unroll
        for (int k = 0; k < XV; ++k)
            if (base + k * kGemvThreads < n4) xv[k] = x4g[base + k * kGemvThreads];
#pragma unroll
        for (int k = 0; k < XV; ++k)
            if (base + k * kGemvThreads < n4) {
                ss = __builtin_fmaf(xv[k].x, xv[k].x, ss);
                ss = __builtin_fmaf(xv[k].y, xv[k].y, ss);
                ss = __builtin_fmaf(xv[k].z, xv[k].z, ss);
                ss = __builtin_fmaf(xv[k].w, xv[k].w, ss);
                xs4[base + k * kGemvThreads] = xv[k];
            }
    }
    if (w4g != nullptr) {   // pre-attention RMSNorm (SimdVectorOps.rmsnorm's formula)
        float4 wv[XV];
#pragma unroll
        for (int k = 0; k < XV; ++k)
            if (tid + k * kGemvThreads < n4) wv[k] = w4g[tid + k * kGemvThreads];
        __shared__ float red[kGemvThreads / 64];
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
#pragma unroll
        for (int k = 0; k < XV; ++k) {
            const int c = tid + k * kGemvThreads;
            if (c < n4) {
                const float4 xv = xs4[c];
                xs4[c] = float4{(xv.x * r) * wv[k].x, (xv.y * r) * wv[k].y, (xv.z * r) * wv[k].z,
                                (xv.w * r) * wv[k].w};
            }
        }
        for (int c = tid + XV * kGemvThreads; c < n4; c += kGemvThreads) {
            const float4 xv = xs4[c];
            const float4 w = w4g[c];
            xs4[c] = float4{(xv.x * r) * w.x, (xv.y * r) * w.y, (xv.z * r) * w.z, (xv.w * r) * w.w};
        }
    }
    __syncthreads();
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

__device__ __forceinline__ GemvSeg seg_of(const GemvArgs& a, int row_g) {
    // a uniform select keeps the argument block out of scratch
    const bool in1 = a.nseg > 1 && row_g >= a.seg[1].out_off;
    const bool in2 = a.nseg > 2 && row_g >= a.seg[2].out_off;
    return in2 ? a.seg[2] : (in1 ? a.seg[1] : a.seg[0]);
}

// ---- the kernels -----------------------------------------------------------------------------
// Workgroup: kGemvThreads threads = kGemvThreads/LPR row groups; row group r of workgroup b
// computes output row b*(kGemvThreads/LPR) + r.  Each lane first issues the loads of its
// units (up to F::MAXU), so the weight reads are in flight while the input is staged in LDS,
// RMS-normalised when norm_w is set (1/(float)sqrt(sum(x^2)/cols + eps), then (x*r)*w as
// SimdVectorOps.rmsnorm forms it).  Dynamic LDS: cols floats, 16-byte aligned.
template <class F, int LPR>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs a) {
    extern __shared__ float xs[];
    const int tid = threadIdx.x;
    constexpr int GROUPS = kGemvThreads / LPR;
    const int grp = tid / LPR, j = tid - grp * LPR;
    const int row_g = blockIdx.x * GROUPS + grp;
    const bool live = row_g < a.rows_total;
    const GemvSeg sg = seg_of(a, row_g);
    const int row = live ? row_g - sg.out_off : 0;
    const int units = a.cols / F::UNIT;
    const int nu = live ? (units - j + LPR - 1) / LPR : 0;   // units of this lane
    typename F::Raw raw[F::MAXU];
    row_load<F, LPR>(raw, nu, sg, row, j);
    stage_input(a, xs, tid);
    if (!live) return;
    const float acc = dk::row_group_sum<LPR>(row_dot<F, LPR>(raw, nu, sg, row, j, units, xs));
    if (j == 0) store_row(a, sg, row_g, row, acc);
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
