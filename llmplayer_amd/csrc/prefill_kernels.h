// Prefill attention for P prompt tokens at positions pos0..pos0+P-1, gfx950.
//
// The reference has no batched prefill: the prompt runs as P sequential single-token forwards
// (LLMEngine.java:478-480, InferenceEngine.prefill at InferenceEngine.java:374-381), so query i
// attends to rows [start(i), pos0+i] of a cache that already holds rows < pos0+i.  This path
// computes the same result in two launches:
//
//  1. prefill_append_kernel: one workgroup per token widens its bf16 k/v to fp32, applies the
//     exact QK-norm + RoPE of the decode path and writes the K/V rows (bit-identical to P
//     appends by the CPU path).
//  2. prefill_attn_kernel: causal flash attention on MFMA.  A workgroup owns one KV head and
//     16*NB query positions of all G query heads of that KV head; each wave owns 16 positions
//     of one query head.  Per 64-key tile (staged in LDS as bf16 hi/lo, V transposed) a wave
//     computes S^T = K Q^T and O^T += V^T P^T with v_mfma_f32_16x16x32_bf16 and an online
//     softmax in the accumulator layout.
//
// Precision: Q and K are post-RoPE fp32 (not bf16), so each operand is split into
// hi = bf16(x) and lo = bf16(x - hi), and a product uses three MFMAs (hi*hi + hi*lo + lo*hi):
// ~2^-16 relative per term instead of bf16's 2^-9, which keeps the output within 1e-4 of the
// fp32 CPU path.  P V uses the same split for P and for V (cache rows before pos0 may be any
// fp32; rows written from bf16 inputs have lo = 0).
//
// Layout facts of v_mfma_f32_16x16x32_bf16 used here (checked on MI355X): lane i holds
// A[i%16][8*(i/16)+j] and B[8*(i/16)+j][i%16] (j < 8) and D[4*(i/16)+j][i%16] (j < 4).
// S^T's D fragment (lane: query i%16, keys 4*(i/16)+j of a 16-key tile) is fed back as the B
// operand of the P V product without moving data across lanes: the 32 keys of an MFMA step
// are taken in the order {4q..4q+3 of tile 2c, 4q..4q+3 of tile 2c+1} (q = i/16), and V^T's A
// operand is read from LDS in the same key order.
#pragma once

#include "decode_kernels.h"

namespace llmp {
namespace pk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short short8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr float kNegBig = dk::kNegBig;

// Keys per LDS tile: 64, or 32 for head_dim 256 (keeps the bf16 hi/lo tile under 80 KB).
template <int D>
constexpr int tile_keys() { return D >= 256 ? 32 : 64; }

struct PrefillArgs {
    const unsigned short* q;  // bf16 bits [P][Hq*D]
    const unsigned short* k;  // bf16 bits [P][Hkv*D]
    const unsigned short* v;  // bf16 bits [P][Hkv*D]
    float* kc;                // layer K plane [Hkv][max_seq][D]
    float* vc;
    long long head_stride;    // max_seq*D
    const float* cos_t;       // RoPE table [max_seq][half] or nullptr (NoPE)
    const float* sin_t;
    const float* qnw;         // QK-norm weights or nullptr
    const float* knw;
    float* out;               // fp32 [P][Hq*D]
    int pos0, P, Hq, Hkv;
    int half_rope, rope_type;
    int window;               // > 0: attend to the last `window` rows (local layer)
    float eps;
    float qk_scale;           // folded into q: scale*log2(e), or scale when soft-capping
    float softcap, softcap_log2e, inv_softcap;
};

__device__ __forceinline__ float bf16_to_f32(unsigned short b) {
    return __uint_as_float((unsigned)b << 16);
}
// Round-to-nearest-even fp32 -> bf16 (finite inputs).
__device__ __forceinline__ unsigned short f32_to_bf16(float f) {
    unsigned u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (unsigned short)(u >> 16);
}
// x = hi + lo with hi, lo bf16 (x - hi is exact in fp32).
__device__ __forceinline__ void split_bf16(float x, unsigned short& hi, unsigned short& lo) {
    hi = f32_to_bf16(x);
    lo = f32_to_bf16(x - bf16_to_f32(hi));
}

// ---- 1. exact K/V append, one workgroup per token --------------------------------------------
template <int D, int NTHR>
__global__ __launch_bounds__(NTHR) void prefill_append_kernel(PrefillArgs a) {
    extern __shared__ float s_dyn[];
    float* s_k = s_dyn;                    // Hkv*D
    float* s_acc = s_dyn + a.Hkv * D;      // Hkv*8
    float* s_r = s_acc + a.Hkv * 8;        // Hkv
    const int i = blockIdx.x, tid = threadIdx.x;
    const int pos = a.pos0 + i;
    const int kvd = a.Hkv * D;
    for (int e = tid; e < kvd; e += NTHR) s_k[e] = bf16_to_f32(a.k[(long long)i * kvd + e]);
    __syncthreads();
    dk::HeadPrep hp{a.knw, a.knw, a.eps,
                    a.cos_t ? a.cos_t + (long long)pos * a.half_rope : nullptr,
                    a.sin_t ? a.sin_t + (long long)pos * a.half_rope : nullptr, a.half_rope,
                    a.rope_type};
    if (a.qnw == nullptr) hp.qnw = hp.knw = nullptr;
    dk::prep_heads_lds<D, NTHR>(s_k, a.Hkv, 0, s_acc, s_r, hp, tid);
    for (int e = tid; e < kvd; e += NTHR) {
        const int h = e / D, d = e - h * D;
        const long long off = (long long)h * a.head_stride + (long long)pos * D + d;
        a.kc[off] = s_k[e];
        a.vc[off] = bf16_to_f32(a.v[(long long)i * kvd + e]);
    }
}

// ---- 2. MFMA flash attention -------------------------------------------------------------------
// LDS tile: K hi/lo [TK keys][D + 8] bf16 (row padding spreads banks), V^T hi/lo [D][TK + 8].
template <int D>
struct TileLds {
    static constexpr int TK = tile_keys<D>();
    static constexpr int KP = D + 8;   // K row pitch (bf16 elements; 16-byte multiple)
    static constexpr int VP = TK + 8;  // V^T row pitch (8-byte multiple)
    unsigned short kh[TK * KP];
    unsigned short kl[TK * KP];
    unsigned short vh[D * VP];
    unsigned short vl[D * VP];
};

template <int D, int G, int NB>
__global__ __launch_bounds__(G * NB * 64) void prefill_attn_kernel(PrefillArgs a) {
    constexpr int NTHR = G * NB * 64;
    constexpr int KS = D / 32;   // MFMA k-steps over the head dimension
    constexpr int DT = D / 16;   // 16-dim output tiles
    constexpr int TK = TileLds<D>::TK;
    constexpr int NKT = TK / 16;  // 16-key sub-tiles per tile
    constexpr int NC = TK / 32;   // 32-key MFMA steps of P V per tile
    __shared__ TileLds<D> t;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int col = lane & 15, grp = lane >> 4;     // query column, lane group (k / row quad)
    const int kvh = blockIdx.y;
    // Heavy (late) query blocks first: the causal key range grows with the block index.
    const int nblk = gridDim.x;
    const int blk = nblk - 1 - (int)blockIdx.x;
    const int i0 = blk * 16 * NB;                    // first token of the block
    const int sb = wave / G, h = wave - sb * G;      // sub-block, query head within the group
    const int hq = kvh * G + h;
    const int qi = i0 + 16 * sb + col;               // token index of this lane's query
    const bool q_ok = qi < a.P;
    const int qpos = a.pos0 + (q_ok ? qi : a.P - 1);
    const int qstart = a.window > 0 ? max(0, qpos - a.window + 1) : 0;

    // Query fragment: dims 32*s + 8*grp + j of token qi, head hq, fp32 -> norm -> RoPE -> scale.
    float qf[KS][8];
    {
        const unsigned short* qp = a.q + (long long)(q_ok ? qi : a.P - 1) * a.Hq * D + (long long)hq * D;
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int j = 0; j < 8; ++j) qf[s][j] = bf16_to_f32(qp[32 * s + 8 * grp + j]);
        if (a.qnw != nullptr) {
            float ss = 0.0f;
#pragma unroll
            for (int s = 0; s < KS; ++s)
#pragma unroll
                for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(qf[s][j], qf[s][j], ss);
            ss = ss + __shfl_xor(ss, 16);
            ss = ss + __shfl_xor(ss, 32);
            const float r = 1.0f / sqrtf(ss / (float)D + a.eps);
#pragma unroll
            for (int s = 0; s < KS; ++s)
#pragma unroll
                for (int j = 0; j < 8; ++j) qf[s][j] = (qf[s][j] * r) * a.qnw[32 * s + 8 * grp + j];
        }
        if (a.cos_t != nullptr) {
            const float* cr = a.cos_t + (long long)qpos * a.half_rope;
            const float* sr = a.sin_t + (long long)qpos * a.half_rope;
            if (a.rope_type == 0) {
#pragma unroll
                for (int s = 0; s < KS; ++s)
#pragma unroll
                    for (int j = 0; j < 8; j += 2) {
                        const int i = (32 * s + 8 * grp + j) / 2;
                        const bool rot = i < a.half_rope;
                        const float c = cr[rot ? i : 0], sn = sr[rot ? i : 0];
                        const float v0 = qf[s][j], v1 = qf[s][j + 1];
                        const float t0 = v0 * c, t1 = v1 * sn, t2 = v0 * sn, t3 = v1 * c;
                        qf[s][j] = rot ? t0 - t1 : v0;
                        qf[s][j + 1] = rot ? t2 + t3 : v1;
                    }
            } else {  // NEOX with half_rope == D/2: partner dims sit KS/2 k-steps apart
#pragma unroll
                for (int s = 0; s < KS / 2; ++s)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int i = 32 * s + 8 * grp + j;
                        const float c = cr[i], sn = sr[i];
                        const float v0 = qf[s][j], v1 = qf[s + KS / 2][j];
                        const float t0 = v0 * c, t1 = v1 * sn, t2 = v0 * sn, t3 = v1 * c;
                        qf[s][j] = t0 - t1;
                        qf[s + KS / 2][j] = t2 + t3;
                    }
            }
        }
    }
    bf16x8 qh[KS], ql[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        short8 hh, ll;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            unsigned short hi, lo;
            split_bf16(qf[s][j] * a.qk_scale, hi, lo);
            hh[j] = (short)hi;
            ll[j] = (short)lo;
        }
        qh[s] = __builtin_bit_cast(bf16x8, hh);
        ql[s] = __builtin_bit_cast(bf16x8, ll);
    }

    // Key range of the workgroup: up to its last query, from its first query's window start.
    const int last_tok = min(i0 + 16 * NB, a.P) - 1;
    const int kend = a.pos0 + last_tok + 1;
    const int kbeg = a.window > 0 ? max(0, a.pos0 + i0 - a.window + 1) & ~15 : 0;
    const float* kplane = a.kc + (long long)kvh * a.head_stride;
    const float* vplane = a.vc + (long long)kvh * a.head_stride;

    floatx4 o[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) o[d] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m = kNegBig, l = 0.0f;

    for (int t0 = kbeg; t0 < kend; t0 += TK) {
        // Stage the tile: fp32 rows -> bf16 hi/lo; K row-major, V transposed.  Rows past kend
        // (never attended) are clamped to a valid row.
        __syncthreads();
        for (int e = tid; e < TK * D / 4; e += NTHR) {
            const int r = e / (D / 4), c4 = e - r * (D / 4);
            const int row = min(t0 + r, kend - 1);
            const float4 kx = reinterpret_cast<const float4*>(kplane + (long long)row * D)[c4];
            const float4 vx = reinterpret_cast<const float4*>(vplane + (long long)row * D)[c4];
            const float kk[4] = {kx.x, kx.y, kx.z, kx.w};
            const float vv[4] = {vx.x, vx.y, vx.z, vx.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int d = 4 * c4 + u;
                unsigned short hi, lo;
                split_bf16(kk[u], hi, lo);
                t.kh[r * TileLds<D>::KP + d] = hi;
                t.kl[r * TileLds<D>::KP + d] = lo;
                split_bf16(vv[u], hi, lo);
                t.vh[d * TileLds<D>::VP + r] = hi;
                t.vl[d * TileLds<D>::VP + r] = lo;
            }
        }
        __syncthreads();

        // S^T = K Q^T for the 16-key sub-tiles: lane holds keys 4*grp+j of sub-tile kt.
        floatx4 st[NKT];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
            const int krow = kt * 16 + col;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const bf16x8 kh = *reinterpret_cast<const bf16x8*>(
                    &t.kh[krow * TileLds<D>::KP + 32 * s + 8 * grp]);
                const bf16x8 kl = *reinterpret_cast<const bf16x8*>(
                    &t.kl[krow * TileLds<D>::KP + 32 * s + 8 * grp]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qh[s], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, ql[s], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qh[s], acc, 0, 0, 0);
            }
            st[kt] = acc;
        }
        // Mask (causal, window, past kend), soft-cap, tile max.
        float mt = kNegBig;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int key = t0 + kt * 16 + 4 * grp + j;
                float sv = st[kt][j];
                if (a.softcap > 0.0f) sv = a.softcap_log2e * tanhf(sv * a.inv_softcap);
                const bool ok = q_ok && key <= qpos && key >= qstart && key < kend;
                sv = ok ? sv : -__builtin_inff();
                st[kt][j] = sv;
                mt = fmaxf(mt, sv);
            }
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = fmaxf(m, mt);
        const float alpha = dk::fast_exp2(m - mn);
        m = mn;
        l = l * alpha;
#pragma unroll
        for (int d = 0; d < DT; ++d) o[d] = o[d] * alpha;
        // P = exp2(S - m), split for the B operand in the key order described above.
        bf16x8 ph[NC], pl[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            short8 hh, ll;
#pragma unroll
            for (int half = 0; half < 2; ++half)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float p = dk::fast_exp2(st[2 * c + half][j] - mn);
                    l = l + p;
                    unsigned short hi, lo;
                    split_bf16(p, hi, lo);
                    hh[4 * half + j] = (short)hi;
                    ll[4 * half + j] = (short)lo;
                }
            ph[c] = __builtin_bit_cast(bf16x8, hh);
            pl[c] = __builtin_bit_cast(bf16x8, ll);
        }
        // O^T += V^T P^T: A operand = V^T rows (dims), keys {32c+4grp..+3, 32c+16+4grp..+3}.
#pragma unroll
        for (int d = 0; d < DT; ++d) {
            const int dim = d * 16 + col;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int k0 = 32 * c + 4 * grp;   // 4 keys (8 bytes) at k0 and at k0 + 16
                const unsigned short* vhr = &t.vh[dim * TileLds<D>::VP + k0];
                const unsigned short* vlr = &t.vl[dim * TileLds<D>::VP + k0];
                const uint2 h0 = *reinterpret_cast<const uint2*>(vhr);
                const uint2 h1 = *reinterpret_cast<const uint2*>(vhr + 16);
                const uint2 l0 = *reinterpret_cast<const uint2*>(vlr);
                const uint2 l1 = *reinterpret_cast<const uint2*>(vlr + 16);
                const bf16x8 vh = __builtin_bit_cast(bf16x8, make_uint4(h0.x, h0.y, h1.x, h1.y));
                const bf16x8 vl = __builtin_bit_cast(bf16x8, make_uint4(l0.x, l0.y, l1.x, l1.y));
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, ph[c], o[d], 0, 0, 0);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pl[c], o[d], 0, 0, 0);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl, ph[c], o[d], 0, 0, 0);
            }
        }
    }
    // Row sums live in 4 lane groups; o[d] lane holds dims d*16 + 4*grp + j of query col.
    l = l + __shfl_xor(l, 16);
    l = l + __shfl_xor(l, 32);
    if (q_ok) {
        const float inv = 1.0f / l;
        float* op = a.out + (long long)qi * a.Hq * D + (long long)hq * D;
#pragma unroll
        for (int d = 0; d < DT; ++d) {
            float4 r = make_float4(o[d][0] * inv, o[d][1] * inv, o[d][2] * inv, o[d][3] * inv);
            reinterpret_cast<float4*>(op + d * 16 + 4 * grp)[0] = r;
        }
    }
}

}  // namespace pk
}  // namespace llmp
