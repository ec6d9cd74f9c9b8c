// Instantiation and dispatch of the projection and residual kernels (gemv_kernels.h).
#include "gemv_kernels.h"
#include "llmp_internal.h"

namespace llmp {
namespace {

template <class F>
hipError_t launch_f(const gk::GemvArgs& a, hipStream_t st) {
    // One row per wave: decode projections have a few thousand rows at most, and a workgroup
    // per 4 rows puts every CU to work in a single round of loads.
    const size_t lds = (size_t)a.cols * sizeof(float);
    const int g = gk::kGemvThreads / 64;
    hipLaunchKernelGGL((gk::gemv_kernel<F, 64>), dim3((a.rows_total + g - 1) / g),
                       dim3(gk::kGemvThreads), lds, st, a);
    return hipGetLastError();
}

}  // namespace

int gemv_unit(int ggml_type) {
    switch (ggml_type) {
    case gk::kF32: return gk::FmtF32::UNIT;
    case gk::kF16: return gk::FmtHalf<false>::UNIT;
    case gk::kBF16: return gk::FmtHalf<true>::UNIT;
    case gk::kQ8_0: return gk::FmtQ8_0::UNIT;
    case gk::kQ4_0: return gk::FmtQ4_0::UNIT;
    case gk::kQ4_K: return gk::FmtQ4_K::UNIT;
    case gk::kQ6_K: return gk::FmtQ6_K::UNIT;
    default: return 0;
    }
}

hipError_t launch_gemv(const gk::GemvArgs& a, int ggml_type, hipStream_t st) {
    if (a.cols <= 0 || a.cols > gk::kMaxGemvCols || a.rows_total <= 0 || a.nseg < 1 || a.nseg > 3)
        return hipErrorInvalidValue;
    const int unit = gemv_unit(ggml_type);
    if (unit == 0 || a.cols % unit) return hipErrorInvalidValue;
    switch (ggml_type) {
    case gk::kF32: return launch_f<gk::FmtF32>(a, st);
    case gk::kF16: return launch_f<gk::FmtHalf<false>>(a, st);
    case gk::kBF16: return launch_f<gk::FmtHalf<true>>(a, st);
    case gk::kQ8_0: return launch_f<gk::FmtQ8_0>(a, st);
    case gk::kQ4_0: return launch_f<gk::FmtQ4_0>(a, st);
    case gk::kQ4_K: return launch_f<gk::FmtQ4_K>(a, st);
    case gk::kQ6_K: return launch_f<gk::FmtQ6_K>(a, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_post_norm_residual(const float* xb, const float* w, float eps, float rscale,
                                     float* x, int dim, hipStream_t st) {
    hipLaunchKernelGGL(gk::post_norm_residual_kernel<gk::kPostThreads>, dim3(1), dim3(gk::kPostThreads), 0, st, xb,
                       w, eps, rscale, x, dim);
    return hipGetLastError();
}

}  // namespace llmp
