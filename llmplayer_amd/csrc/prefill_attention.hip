// Instantiation and dispatch of the prefill kernels (prefill_kernels.h).
#include "prefill_kernels.h"

namespace llmp {
namespace {

constexpr int kAppendThreads = 256;

// Position sub-blocks of 16 per workgroup: about 8 waves (G heads x NB sub-blocks).
constexpr int pick_nb(int G) { return G >= 8 ? 1 : (8 / G > 0 ? 8 / G : 1); }

template <int D, int G>
hipError_t launch_attn_dg(const pk::PrefillArgs& a, hipStream_t stream) {
    constexpr int NB = pick_nb(G);
    const int blocks = (a.P + 16 * NB - 1) / (16 * NB);
    hipLaunchKernelGGL((pk::prefill_attn_kernel<D, G, NB>), dim3(blocks, a.Hkv), dim3(G * NB * 64),
                       0, stream, a);
    return hipGetLastError();
}

template <int D>
hipError_t launch_attn_d(const pk::PrefillArgs& a, int group, hipStream_t stream) {
    switch (group) {
    case 1: return launch_attn_dg<D, 1>(a, stream);
    case 2: return launch_attn_dg<D, 2>(a, stream);
    case 3: return launch_attn_dg<D, 3>(a, stream);
    case 4: return launch_attn_dg<D, 4>(a, stream);
    case 6: return launch_attn_dg<D, 6>(a, stream);
    case 8: return launch_attn_dg<D, 8>(a, stream);
    default: return hipErrorInvalidValue;
    }
}

template <int D>
hipError_t launch_append_d(const pk::PrefillArgs& a, hipStream_t stream) {
    const size_t lds = (size_t)a.Hkv * (D + 9) * sizeof(float);
    hipLaunchKernelGGL((pk::prefill_append_kernel<D, kAppendThreads>), dim3(a.P),
                       dim3(kAppendThreads), lds, stream, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill_append(const pk::PrefillArgs& a, int head_dim, hipStream_t stream) {
    switch (head_dim) {
    case 64: return launch_append_d<64>(a, stream);
    case 128: return launch_append_d<128>(a, stream);
    case 256: return launch_append_d<256>(a, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_prefill_attn(const pk::PrefillArgs& a, int head_dim, int group,
                               hipStream_t stream) {
    switch (head_dim) {
    case 64: return launch_attn_d<64>(a, group, stream);
    case 128: return launch_attn_d<128>(a, group, stream);
    case 256: return launch_attn_d<256>(a, group, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace llmp
