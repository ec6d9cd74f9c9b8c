// Instantiation and dispatch of the decode kernels (decode_kernels.h) for the shapes the
// library ships: head_dim 64/128/256 (fp32 and Q8_0 caches) with GQA groups 1-8, 512 (fp32: the
// full-attention layers of Gemma 4) with groups 1-8, 96 (fp32: Phi-3) with groups 1-4 and 80
// (fp32: Phi-2) with groups 1-2.  Larger groups (GLM-4's 16 and 24) run as several groups of
// one of these sizes per cached KV head (kernel_group, DecodeArgs::kv_rep).
#include "decode_kernels.h"

namespace llmp {
namespace {

// Per-shape tuning (measured on MI355X at the BASELINE shapes): elements of a K/V row per
// lane (EPL), rows per lane-group per loop trip (U; the loop keeps two trips in registers, the
// one consumed and the one prefetched), non-temporal KV loads.  The number of waves per
// workgroup is chosen per call.
struct Tune {
    int epl, unroll;
    bool nt;
};
constexpr Tune pick(int D, int G) {
    // head_dim 512: 8 elements per lane, so a row spans the whole wave (LPR 64).  head_dim 256
    // (16 elements per lane) and groups above 4 take one row per trip: two trips of two rows
    // would not fit the register file next to the G*EPL query and output values.  head_dim 96
    // and 80 need a power-of-two lane count per row: 12 elements (8 lanes) and 20 (4 lanes);
    // 80's 20 elements per lane take one row per trip.
    if (D == 96) return Tune{12, G > 4 ? 1 : 2, true};
    if (D == 80) return Tune{20, 1, true};
    return Tune{D == 512 ? 8 : ((D == 256 || (G > 4 && D / 8 > 16)) ? 16 : 8),
                (G > 4 || D == 256) ? 1 : 2, true};
}

// The kernel instance for one shape, and the waves per workgroup it runs with.
struct SplitKernel {
    const void* fn;
    int waves;
};

template <int D, int G, int W, bool Q8>
SplitKernel kernel_dgw() {
    constexpr Tune t = pick(D, G);
    // Q8_0 caches with up to 4 query heads per KV head: scores on the int8 matrix cores.  Its
    // K operand loads are 8 bytes per lane (a quarter of a 128-byte row each), so the loads
    // stay temporal: the row's other quarters then hit in L2 (non-temporal loads measured
    // 23.1 against 21.0 us per split launch at the Llama-3.2-3B shape, 32k rows).
    if constexpr (Q8 && G <= 4 && D <= 256) {
        return SplitKernel{reinterpret_cast<const void*>(&dk::decode_q8_mfma_kernel<D, G, W, false>), W};
    } else {
        // Q8_0 rows are read as 16 quants per lane (D/16 lanes per row).
        constexpr int EPL = Q8 ? 16 : t.epl;
        constexpr int UNROLL = Q8 ? 1 : t.unroll;
        return SplitKernel{
            reinterpret_cast<const void*>(&dk::decode_split_kernel<D, G, EPL, UNROLL, W, t.nt, Q8>), W};
    }
}

// 8-wave workgroups except where more than 4 query heads per KV head hold 16 elements per
// lane (head_dim 256, or any Q8_0 cache): that register footprint leaves no room for them.
// head_dim 512 always runs 4 waves (its per-wave LDS partials would pass 128 KB at 8).
// head_dim 64 over an fp32 cache also has 2-wave workgroups, for splits of at most 32 rows
// (one 16-row trip per wave; with 4 waves two of them would sit idle through the merge).
template <int D, int G, bool Q8>
SplitKernel kernel_dg(int waves) {
    if constexpr (((D == 256 || Q8) && G > 4) || D == 512) {
        return kernel_dgw<D, G, 4, Q8>();
    } else {
        if constexpr (D == 64 && !Q8) {
            if (waves == 2) return kernel_dgw<D, G, 2, Q8>();
        }
        return waves == 8 ? kernel_dgw<D, G, 8, Q8>() : kernel_dgw<D, G, 4, Q8>();
    }
}

template <int D, bool Q8>
SplitKernel kernel_d(int group, int waves) {
    switch (group) {
    case 1: return kernel_dg<D, 1, Q8>(waves);
    case 2: return kernel_dg<D, 2, Q8>(waves);
    default: break;
    }
    if constexpr (D == 80) {   // 20 elements per lane: groups beyond 2 would spill
        return SplitKernel{nullptr, 0};
    } else {
        switch (group) {
        case 3: return kernel_dg<D, 3, Q8>(waves);
        case 4: return kernel_dg<D, 4, Q8>(waves);
        default: break;
        }
    }
    if constexpr (D == 80 || D == 96) {   // head sizes of MHA / small-group models
        return SplitKernel{nullptr, 0};
    } else {
        switch (group) {
        case 5: return kernel_dg<D, 5, Q8>(waves);
        case 6: return kernel_dg<D, 6, Q8>(waves);
        case 7: return kernel_dg<D, 7, Q8>(waves);
        case 8: return kernel_dg<D, 8, Q8>(waves);
        default: return SplitKernel{nullptr, 0};
        }
    }
}

template <bool Q8>
SplitKernel kernel_split(int head_dim, int group, int waves) {
    switch (head_dim) {
    case 64: return kernel_d<64, Q8>(group, waves);
    case 128: return kernel_d<128, Q8>(group, waves);
    case 256: return kernel_d<256, Q8>(group, waves);
    case 80: case 96: case 512:   // fp32 caches only
        if constexpr (!Q8) {
            if (head_dim == 80) return kernel_d<80, false>(group, waves);
            if (head_dim == 96) return kernel_d<96, false>(group, waves);
            return kernel_d<512, false>(group, waves);
        }
        return SplitKernel{nullptr, 0};
    default: return SplitKernel{nullptr, 0};
    }
}

SplitKernel resolve_split(int head_dim, int group, int waves, bool q8) {
    if (waves != 2 && waves != 4 && waves != 8) return SplitKernel{nullptr, 0};
    return q8 ? kernel_split<true>(head_dim, group, waves)
              : kernel_split<false>(head_dim, group, waves);
}

__global__ void copy_kernel(float4* __restrict__ dst, const float4* __restrict__ src, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) dst[i] = src[i];
}

}  // namespace

bool decode_shape_supported(int head_dim, int group) { return decode_group_ok(head_dim, group); }

// Measured on MI355X (graph replays, µs per layer-call, combine kernel -> merge in the split
// kernel): C1 pos 511 (16 splits x 2 waves) 8.2 -> 7.2, C3 ctx 32768 (24 x 8) 45.5 -> 45.0,
// but C2 ctx 1024 / 4096 (32 x 4) 8.3 -> 9.1 / 12.4 -> 12.6: with 4-wave workgroups the
// combine kernel stays.
bool decode_fused_merge(int head_dim, int group, int waves, int splits) {
    const int nthr = waves * 64, nc = group * head_dim / 4;
    const int np = nthr >= nc ? nthr / nc : 1;
    return splits > 1 && waves != 4 && (splits + np - 1) / np <= dk::kMergeBatch;
}

int decode_split_waves(int head_dim, int group, int waves, bool q8) {
    return resolve_split(head_dim, group, waves, q8).waves;
}

int decode_split_blocks_per_cu(int head_dim, int group, int waves, bool q8) {
    const SplitKernel k = resolve_split(head_dim, group, waves, q8);
    if (!k.fn) return 0;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k.fn, k.waves * 64, 0) != hipSuccess)
        return 0;
    return n;
}

hipError_t launch_decode_split(const DecodeArgs& a, int head_dim, int group, int n_kv_heads,
                               int waves, bool q8, hipStream_t stream) {
    const SplitKernel k = resolve_split(head_dim, group, waves, q8);
    if (!k.fn) return hipErrorInvalidValue;
    DecodeArgs args = a;
    void* params[] = {&args};
    return hipLaunchKernel(k.fn, dim3(a.splits, n_kv_heads), dim3(k.waves * 64), params, 0, stream);
}

namespace {
// The combine over reduce_column_groups(...) column workgroups per head.
template <int D>
hipError_t launch_reduce_d(const DecodeArgs& a, int group, int n_heads, hipStream_t stream) {
    constexpr int NC = D / 4;
    const int cb = reduce_column_groups(D, a.splits, dk::kReduceThreads, dk::kReduceBatch);
    const dim3 grid(n_heads, cb), block(dk::kReduceThreads);
    switch (cb) {
    case 1: hipLaunchKernelGGL((dk::decode_reduce_kernel<D, 1>), grid, block, 0, stream, a, group); break;
    case 2:
        if constexpr (NC % 2 == 0)
            hipLaunchKernelGGL((dk::decode_reduce_kernel<D, 2>), grid, block, 0, stream, a, group);
        break;
    case 4:
        if constexpr (NC % 4 == 0)
            hipLaunchKernelGGL((dk::decode_reduce_kernel<D, 4>), grid, block, 0, stream, a, group);
        break;
    default:
        if constexpr (NC % 8 == 0)
            hipLaunchKernelGGL((dk::decode_reduce_kernel<D, 8>), grid, block, 0, stream, a, group);
        break;
    }
    return hipGetLastError();
}
}  // namespace

hipError_t launch_decode_reduce(const DecodeArgs& a, int head_dim, int group, int n_heads,
                                hipStream_t stream) {
    if (a.splits > kMaxSplits) return hipErrorInvalidValue;
    switch (head_dim) {
    case 64: return launch_reduce_d<64>(a, group, n_heads, stream);
    case 128: return launch_reduce_d<128>(a, group, n_heads, stream);
    case 256: return launch_reduce_d<256>(a, group, n_heads, stream);
    case 512: return launch_reduce_d<512>(a, group, n_heads, stream);
    case 80: return launch_reduce_d<80>(a, group, n_heads, stream);
    case 96: return launch_reduce_d<96>(a, group, n_heads, stream);
    default: return hipErrorInvalidValue;
    }
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
