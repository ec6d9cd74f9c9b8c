// Split-K flash-decoding attention for one new token, gfx950 (CDNA4, wave64).
//
// One workgroup = (split j, KV head g): it owns rows [t_start + j*R, ...) of that KV head and
// every query head of the GQA group (Hq/Hkv heads), so each KV byte is read from HBM once per
// layer-call.  The workgroup also does the per-token prep of the reference's separate
// kernels (rmsnorm_per_head, rope_apply, kv_cache_update: CudaForwardPass.java:1529-1564)
// for its own heads, so a layer-call is one split kernel plus one combine kernel (or only the
// split kernel when splits == 1).
//
// Bit-exactness: the appended K row is computed with the CPU path's float step order --
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
#include "llmp_internal.h"

namespace llmp {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr float kLog2e = 1.4426950408889634f;
// Finite "minus infinity" for running maxima, so that exp2(m_old - m_new) never sees
// (-inf) - (-inf).  Masked scores use a true -inf, which exp2 maps to 0.
constexpr float kNegBig = -1.0e30f;

// DPP controls (CDNA3/CDNA4 ISA): quad_perm, row_half_mirror, row_mirror.
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowMirror = 0x140;   // lane i <- lane 15-i within each row of 16
constexpr int kDppRowHalfMirror = 0x141;  // lane i <- lane 7-i within each half row

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over the LPR consecutive lanes that share a row.  Every lane ends with the same value
// (each step adds the same two operands, in either order).
template <int LPR>
__device__ __forceinline__ float row_group_sum(float x) {
    static_assert(LPR == 4 || LPR == 8 || LPR == 16, "rows are shared by 4, 8 or 16 lanes");
    x = x + dpp<kDppQuadXor1>(x);
    x = x + dpp<kDppQuadXor2>(x);
    if constexpr (LPR >= 8) x = x + dpp<kDppRowHalfMirror>(x);
    if constexpr (LPR >= 16) x = x + dpp<kDppRowMirror>(x);
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Elements per lane of a K/V row: 16 keeps the query slice and output slice of a GQA group
// within registers for up to 4 query heads; larger groups use 8 (rows shared by more lanes).
constexpr int pick_epl(int D, int G) { return (G > 4 && D / 8 <= 16) ? 8 : 16; }
// Rows per lane-group per loop trip (loads in flight per lane = 2 * U * EPL floats).
constexpr int pick_unroll(int D, int G) { return (G > 4) ? 1 : 2; }

template <int D, int G, int EPL>
struct Frag {
    static constexpr int LPR = D / EPL;   // lanes per row
    static constexpr int RPW = 64 / LPR;  // rows per wave-wide load
    static constexpr int C4 = EPL / 4;    // 16-byte chunks per lane per row
    // Dimension held by lane j (within its row group) at element e.
    static __device__ __forceinline__ int dim(int j, int e) {
        return (e >> 2) * (LPR * 4) + j * 4 + (e & 3);
    }
};

// Online-softmax update of one row group with U rows: s = (q . K_t) in the log2 domain,
// masked rows get -inf; o and l are rescaled once per call.
template <int D, int G, int EPL, int U>
__device__ __forceinline__ void accumulate_rows(const float (&qr)[G][EPL],
                                                const float4 (&kf)[U][EPL / 4],
                                                const float4 (&vf)[U][EPL / 4],
                                                const bool (&valid)[U], float (&m)[G],
                                                float (&l)[G], float (&o)[G][EPL],
                                                const DecodeArgs& a) {
    using F = Frag<D, G, EPL>;
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
        const float alpha = fast_exp2(m[h] - mx);
        m[h] = mx;
        float lsum = l[h] * alpha;
#pragma unroll
        for (int e = 0; e < EPL; ++e) o[h][e] = o[h][e] * alpha;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float p = fast_exp2(s[u][h] - mx);
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

template <int D, int G, int EPL, int U>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(DecodeArgs a) {
    using F = Frag<D, G, EPL>;
    constexpr int LPR = F::LPR, RPW = F::RPW, C4 = F::C4;
    constexpr int ROWS_WAVE = U * RPW;
    constexpr int ROWS_BLOCK = kWaves * ROWS_WAVE;

    // s_x holds the G query heads followed by the group's K head (post norm and RoPE).
    __shared__ float s_x[(G + 1) * D];
    __shared__ float s_v[D];
    __shared__ float s_acc[(G + 1) * 8];
    __shared__ float s_r[G + 1];
    __shared__ float s_m[kWaves * G];
    __shared__ float s_l[kWaves * G];
    __shared__ float s_o[kWaves * G * D];

    const int tid = threadIdx.x;
    const int split = blockIdx.x;
    const int kvh = blockIdx.y;
    const int h0 = kvh * G;
    const int row_begin = a.t_start + split * a.rows_per_split;
    const int row_end = min(row_begin + a.rows_per_split, a.pos + 1);
    const bool has_pos = (row_end == a.pos + 1);
    const int cache_end = has_pos ? a.pos : row_end;
    const int nh = G + (has_pos ? 1 : 0);

    // 1. Stage the raw projections of this group (and k, v if this split owns row `pos`).
    for (int i = tid; i < G * D; i += kThreads) s_x[i] = a.q[h0 * D + i];
    if (has_pos) {
        for (int i = tid; i < D; i += kThreads) {
            s_x[G * D + i] = a.k[kvh * D + i];
            s_v[i] = a.v[kvh * D + i];
        }
    }
    __syncthreads();

    // 2. Per-head QK-norm (Attention.applyPerHeadNorm, Attention.java:384-394).
    if (a.qnw != nullptr) {
        if (tid < nh * 8) {
            const int hh = tid >> 3, ln = tid & 7;
            const float* xh = s_x + hh * D;
            float acc = 0.0f;
#pragma unroll
            for (int i = ln; i < D; i += 8) acc = __builtin_fmaf(xh[i], xh[i], acc);
            s_acc[tid] = acc;
        }
        __syncthreads();
        if (tid < nh) {
            const float* ac = s_acc + tid * 8;
            float ss = ac[0];
#pragma unroll
            for (int ln = 1; ln < 8; ++ln) ss = ss + ac[ln];
            float t = ss / (float)D;
            t = t + a.eps;
            const float r = (float)__builtin_sqrt((double)t);
            s_r[tid] = 1.0f / r;
        }
        __syncthreads();
        for (int i = tid; i < nh * D; i += kThreads) {
            const int hh = i / D;
            const float* w = (hh < G) ? a.qnw : a.knw;
            const float xs = s_x[i] * s_r[hh];
            s_x[i] = xs * w[i - hh * D];
        }
        __syncthreads();
    }

    // 3. RoPE (RoPE.apply / ropeNeox), pairs (2i,2i+1) or (i, i+R/2).
    if (a.cos_row != nullptr) {
        const int half = a.half_rope;
        for (int idx = tid; idx < nh * half; idx += kThreads) {
            const int hh = idx / half, i = idx - hh * half;
            float* xh = s_x + hh * D;
            const int i0 = (a.rope_type == 0) ? 2 * i : i;
            const int i1 = (a.rope_type == 0) ? 2 * i + 1 : half + i;
            const float c = a.cos_row[i], sn = a.sin_row[i];
            const float v0 = xh[i0], v1 = xh[i1];
            const float t0 = v0 * c, t1 = v1 * sn, t2 = v0 * sn, t3 = v1 * c;
            xh[i0] = t0 - t1;
            xh[i1] = t2 + t3;
        }
        __syncthreads();
    }

    float* kplane = a.kc + (long long)kvh * a.head_stride;
    float* vplane = a.vc + (long long)kvh * a.head_stride;

    // 4. Append row `pos` (KVCache.storeK / storeV): exact copies of the prepared rows.
    if (has_pos) {
        for (int i = tid; i < D; i += kThreads) {
            kplane[(long long)a.pos * D + i] = s_x[G * D + i];
            vplane[(long long)a.pos * D + i] = s_v[i];
        }
    }

    // 5. Query slice of this lane, pre-scaled (log2 domain unless soft-capping).
    const int wave = tid >> 6, lane = tid & 63;
    const int grp = lane / LPR, j = lane - grp * LPR;
    float qr[G][EPL];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < EPL; ++e) qr[h][e] = s_x[h * D + F::dim(j, e)] * a.qk_scale;

    float m[G], l[G], o[G][EPL];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m[h] = kNegBig;
        l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) o[h][e] = 0.0f;
    }

    // 6. Stream the cached rows [row_begin, cache_end).
    for (int base = row_begin + wave * ROWS_WAVE; base < cache_end; base += ROWS_BLOCK) {
        float4 kf[U][C4], vf[U][C4];
        bool valid[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = base + u * RPW + grp;
            valid[u] = t < cache_end;
            const int tt = valid[u] ? t : cache_end - 1;  // in-bounds address for masked rows
            const float4* kp = reinterpret_cast<const float4*>(kplane + (long long)tt * D) + j;
            const float4* vp = reinterpret_cast<const float4*>(vplane + (long long)tt * D) + j;
#pragma unroll
            for (int c = 0; c < C4; ++c) kf[u][c] = kp[c * LPR];
#pragma unroll
            for (int c = 0; c < C4; ++c) vf[u][c] = vp[c * LPR];
        }
        accumulate_rows<D, G, EPL, U>(qr, kf, vf, valid, m, l, o, a);
    }

    // 7. Row `pos` itself comes from LDS (row group 0 of wave 0).
    if (has_pos && wave == 0) {
        float4 kf[1][C4], vf[1][C4];
        bool valid[1] = {grp == 0};
#pragma unroll
        for (int c = 0; c < C4; ++c) {
            const int d0 = c * LPR * 4 + j * 4;
            kf[0][c] = make_float4(s_x[G * D + d0], s_x[G * D + d0 + 1], s_x[G * D + d0 + 2],
                                   s_x[G * D + d0 + 3]);
            vf[0][c] = make_float4(s_v[d0], s_v[d0 + 1], s_v[d0 + 2], s_v[d0 + 3]);
        }
        accumulate_rows<D, G, EPL, 1>(qr, kf, vf, valid, m, l, o, a);
    }

    // 8. Merge the row groups of each wave (lanes j, j+LPR, ...), then the waves via LDS.
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float mw = m[h];
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1) mw = fmaxf(mw, __shfl_xor(mw, off));
        const float sc = fast_exp2(m[h] - mw);
        float lw = l[h] * sc;
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1) lw = lw + __shfl_xor(lw, off);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float x = o[h][e] * sc;
#pragma unroll
            for (int off = LPR; off < 64; off <<= 1) x = x + __shfl_xor(x, off);
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

    for (int idx = tid; idx < G * D; idx += kThreads) {
        const int h = idx / D, d = idx - h * D;
        float M = s_m[h];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w * G + h]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float sc = fast_exp2(s_m[w * G + h] - M);
            L = __builtin_fmaf(s_l[w * G + h], sc, L);
            O = __builtin_fmaf(s_o[(w * G + h) * D + d], sc, O);
        }
        if (a.splits == 1) {
            a.out[(h0 + h) * D + d] = O / L;
        } else {
            const long long slot = ((long long)kvh * a.splits + split) * G + h;
            a.part_o[slot * D + d] = O;
            if (d == 0) {
                a.part_ml[2 * slot] = M;
                a.part_ml[2 * slot + 1] = L;
            }
        }
    }
}

// Log-sum-exp combine of the splits of one query head:
//   M = max_j m_j,  L = sum_j l_j 2^(m_j - M),  out = sum_j o_j 2^(m_j - M) / L.
// With one split this reduces to the online softmax of Attention.java:161-207.
constexpr int kReduceThreads = 256;

__global__ __launch_bounds__(kReduceThreads) void decode_reduce_kernel(DecodeArgs a, int G,
                                                                       int D) {
    __shared__ float s_w[kMaxSplits];
    __shared__ float s_red[kReduceThreads / 64];
    __shared__ float s_part[kReduceThreads];
    const int hq = blockIdx.x;
    const int kvh = hq / G, h = hq - kvh * G;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int S = a.splits;
    const long long slot0 = (long long)kvh * S * G + h;  // slot of split j: slot0 + j*G

    float mx = kNegBig;
    for (int jj = tid; jj < S; jj += kReduceThreads) mx = fmaxf(mx, a.part_ml[2 * (slot0 + jj * G)]);
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (lane == 0) s_red[wave] = mx;
    __syncthreads();
    float M = s_red[0];
    for (int w = 1; w < kReduceThreads / 64; ++w) M = fmaxf(M, s_red[w]);
    __syncthreads();

    float ls = 0.0f;
    for (int jj = tid; jj < S; jj += kReduceThreads) {
        const float w = fast_exp2(a.part_ml[2 * (slot0 + jj * G)] - M);
        s_w[jj] = w;
        ls = __builtin_fmaf(a.part_ml[2 * (slot0 + jj * G) + 1], w, ls);
    }
    for (int off = 32; off > 0; off >>= 1) ls = ls + __shfl_xor(ls, off);
    if (lane == 0) s_red[wave] = ls;
    __syncthreads();
    float L = 0.0f;
    for (int w = 0; w < kReduceThreads / 64; ++w) L = L + s_red[w];
    const float inv_l = 1.0f / L;

    // Threads split (dimension d, split subset p): parts = blockDim / D.
    const int parts = kReduceThreads / D;
    const int d = tid % D, p = tid / D;
    float acc = 0.0f;
    if (p < parts) {
        for (int jj = p; jj < S; jj += parts)
            acc = __builtin_fmaf(s_w[jj], a.part_o[(slot0 + (long long)jj * G) * D + d], acc);
    }
    s_part[tid] = acc;
    __syncthreads();
    if (tid < D) {
        float o = s_part[tid];
        for (int q = 1; q < parts; ++q) o = o + s_part[q * D + tid];
        a.out[hq * D + tid] = o * inv_l;
    }
}

template <int D, int G>
hipError_t launch_dg(const DecodeArgs& a, int n_kv_heads, hipStream_t stream) {
    constexpr int EPL = pick_epl(D, G);
    constexpr int U = pick_unroll(D, G);
    hipLaunchKernelGGL((decode_split_kernel<D, G, EPL, U>), dim3(a.splits, n_kv_heads),
                       dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}

template <int D>
hipError_t launch_d(const DecodeArgs& a, int group, int n_kv_heads, hipStream_t stream) {
    switch (group) {
    case 1: return launch_dg<D, 1>(a, n_kv_heads, stream);
    case 2: return launch_dg<D, 2>(a, n_kv_heads, stream);
    case 3: return launch_dg<D, 3>(a, n_kv_heads, stream);
    case 4: return launch_dg<D, 4>(a, n_kv_heads, stream);
    case 6: return launch_dg<D, 6>(a, n_kv_heads, stream);
    case 8: return launch_dg<D, 8>(a, n_kv_heads, stream);
    default: return hipErrorInvalidValue;
    }
}

__global__ void copy_kernel(float4* __restrict__ dst, const float4* __restrict__ src, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) dst[i] = src[i];
}

}  // namespace

bool decode_shape_supported(int head_dim, int group) {
    const bool d_ok = head_dim == 64 || head_dim == 128 || head_dim == 256;
    const bool g_ok = group == 1 || group == 2 || group == 3 || group == 4 || group == 6 ||
                      group == 8;
    return d_ok && g_ok;
}

hipError_t launch_decode_split(const DecodeArgs& a, int head_dim, int group, int n_kv_heads,
                               hipStream_t stream) {
    switch (head_dim) {
    case 64: return launch_d<64>(a, group, n_kv_heads, stream);
    case 128: return launch_d<128>(a, group, n_kv_heads, stream);
    case 256: return launch_d<256>(a, group, n_kv_heads, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_decode_reduce(const DecodeArgs& a, int head_dim, int group, int n_heads,
                                hipStream_t stream) {
    if (a.splits > kMaxSplits || head_dim > kReduceThreads) return hipErrorInvalidValue;
    hipLaunchKernelGGL(decode_reduce_kernel, dim3(n_heads), dim3(kReduceThreads), 0, stream, a,
                       group, head_dim);
    return hipGetLastError();
}

hipError_t launch_copy(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    const size_t n = bytes / 16;
    if (n == 0) return hipSuccess;
    size_t blocks = (n + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(copy_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<float4*>(dst), static_cast<const float4*>(src), n);
    return hipGetLastError();
}

}  // namespace llmp
