// Instantiation and dispatch of the token-batched projection kernels (proj_tok_kernels.h).
#include "proj_tok_kernels.h"
#include "llmp_internal.h"

namespace llmp {
static_assert(tk::kTok == kTokBatch, "one token count for the kernels and the host");

namespace {

template <class F>
hipError_t launch_f(const tk::ProjTokArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(tk::proj_tok_kernel<F>, dim3(a.rows_total / 16), dim3(tk::kThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace

bool proj_tok_supported(int ggml_type) {
    switch (ggml_type) {
    case gk::kF32: case gk::kF16: case gk::kBF16: case gk::kQ8_0: case gk::kQ4_0: case gk::kQ4_K:
    case gk::kQ6_K:
        return true;
    default:
        return false;
    }
}

size_t proj_tok_stage_bytes(int cols) {
    const size_t ng = (size_t)(cols / 32);
    return ng * tk::kXParts * 64 * 16 + ng * tk::kTok * sizeof(float);
}

hipError_t launch_proj_stage(const float* x, long long x_pitch, const float* norm_w, float eps,
                             int cols, int n_tokens, void* stage, hipStream_t st) {
    if (cols <= 0 || cols % 32 || n_tokens < 1 || n_tokens > tk::kTok) return hipErrorInvalidValue;
    const size_t ng = (size_t)(cols / 32);
    uint4* xb = static_cast<uint4*>(stage);
    float* xsum = reinterpret_cast<float*>(static_cast<char*>(stage) + ng * tk::kXParts * 64 * 16);
    hipLaunchKernelGGL(tk::proj_stage_kernel<tk::kStageThreads>, dim3(n_tokens), dim3(tk::kStageThreads), 0, st, x,
                       x_pitch, norm_w, eps, cols, xb, xsum);
    return hipGetLastError();
}

hipError_t launch_proj_tok(tk::ProjTokArgs a, int ggml_type, const void* stage, hipStream_t st) {
    if (a.cols <= 0 || a.cols % 32 || a.rows_total <= 0 || a.rows_total % 16 || a.K < 1 ||
        a.K > tk::kTok || a.nseg < 1 || a.nseg > 3)
        return hipErrorInvalidValue;
    for (int i = 0; i < a.nseg; ++i)
        if (a.seg[i].rows % 16 || a.seg[i].out_off % 16) return hipErrorInvalidValue;
    if ((ggml_type == gk::kQ4_K || ggml_type == gk::kQ6_K) && a.cols % 256) return hipErrorInvalidValue;
    const size_t ng = (size_t)(a.cols / 32);
    a.xb = static_cast<const uint4*>(stage);
    a.xsum = reinterpret_cast<const float*>(static_cast<const char*>(stage) + ng * tk::kXParts * 64 * 16);
    switch (ggml_type) {
    case gk::kF32: return launch_f<tk::PF32>(a, st);
    case gk::kF16: return launch_f<tk::PF16>(a, st);
    case gk::kBF16: return launch_f<tk::PBF16>(a, st);
    case gk::kQ8_0: return launch_f<tk::PQ8_0>(a, st);
    case gk::kQ4_0: return launch_f<tk::PQ4_0>(a, st);
    case gk::kQ4_K: return launch_f<tk::PQ4K>(a, st);
    case gk::kQ6_K: return launch_f<tk::PQ6K>(a, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace llmp
