// Instantiation and dispatch of the projection and residual kernels (gemv_kernels.h).
#include "gemv_kernels.h"
#include "llmp_internal.h"

namespace llmp {
namespace {

template <class F1, int NK1, class F2 = F1, int NK2 = NK1>
hipError_t launch_nk(const gk::GemvArgs& a, hipStream_t st) {
    const size_t lds = gk::GemvLds<F1, F2>::bytes(a.cols);
    const int g = gk::kGemvRowsPerGroup;
    hipLaunchKernelGGL((gk::gemv_kernel<F1, NK1, F2, NK2>), dim3((a.rows_total + g - 1) / g),
                       dim3(gk::kGemvThreads), lds, st, a);
    return hipGetLastError();
}

// One row per wave: decode projections have a few thousand rows at most, and a workgroup per
// 4 rows puts every CU to work in a single round of loads.  NK: the unit rounds a lane holds
// in registers, the row's rounds rounded up to 2, 3, 4, 6 or 8 (at most the format's budget;
// wider rows take several batches).
template <class F>
int nk_for(int cols) {
    const int rounds = (cols / F::UNIT + 63) / 64;
    const int nk = rounds <= 2 ? 2 : rounds <= 3 ? 3 : rounds <= 4 ? 4 : rounds <= 6 ? 6 : 8;
    return nk > F::MAXU ? F::MAXU : nk;
}

// The largest instantiated round count of a format: nk_for never asks for more than MAXU, so
// no instance above it is compiled.
template <class F>
constexpr int nk_cap(int nk) { return nk > F::MAXU ? F::MAXU : nk; }

template <class F>
hipError_t launch_f(const gk::GemvArgs& a, hipStream_t st) {
    switch (nk_for<F>(a.cols)) {
    case 2: return launch_nk<F, 2>(a, st);
    case 3: return launch_nk<F, nk_cap<F>(3)>(a, st);
    case 4: return launch_nk<F, nk_cap<F>(4)>(a, st);
    default:
        if constexpr (F::MAXU >= 8) {
            if (nk_for<F>(a.cols) == 6) return launch_nk<F, 6>(a, st);
            return launch_nk<F, 8>(a, st);
        } else if constexpr (F::MAXU >= 6) {
            return launch_nk<F, 6>(a, st);
        } else {
            return hipErrorInvalidValue;
        }
    }
}

// Q4_K rows (GemvSeg::fmt 0, fp32 or Q8_1 input) and Q6_K rows (fmt 1) in one launch: the
// Q4_K_M mix of the attention projections.
template <class F1, int NK1>
hipError_t launch_q4k_q6k(const gk::GemvArgs& a, hipStream_t st) {
    using F2 = gk::FmtQ6_K;
    switch (nk_for<F2>(a.cols)) {
    case 2: return launch_nk<F1, NK1, F2, 2>(a, st);
    case 3: return launch_nk<F1, NK1, F2, 3>(a, st);
    default: return launch_nk<F1, NK1, F2, 4>(a, st);
    }
}

// Two formats of the K-quant mixes in one launch: F1 rows (GemvSeg::fmt 0) with NK1 rounds,
// F2 rows (fmt 1) with at most 4 (Q3_K_L: Q3_K q and k with Q5_K v; Q5_K_M: Q5_K with Q6_K).
template <class F1, int NK1, class F2>
hipError_t launch_mix2(const gk::GemvArgs& a, hipStream_t st) {
    switch (nk_for<F2>(a.cols)) {
    case 2: return launch_nk<F1, NK1, F2, 2>(a, st);
    case 3: return launch_nk<F1, NK1, F2, nk_cap<F2>(3)>(a, st);
    default: return launch_nk<F1, NK1, F2, nk_cap<F2>(4)>(a, st);
    }
}
template <class F1, class F2>
hipError_t launch_mix(const gk::GemvArgs& a, hipStream_t st) {
    switch (nk_for<F1>(a.cols)) {
    case 2: return launch_mix2<F1, 2, F2>(a, st);
    case 3: return launch_mix2<F1, nk_cap<F1>(3), F2>(a, st);
    default: return launch_mix2<F1, nk_cap<F1>(4), F2>(a, st);
    }
}

// The Q8_1-input Q4_K side holds at most 4 rounds next to Q6_K (more spills registers); its
// rows need 4 rounds up to 4096 columns.
template <class F1>
hipError_t launch_pair_f(const gk::GemvArgs& a, hipStream_t st) {
    switch (nk_for<F1>(a.cols)) {
    case 2: return launch_q4k_q6k<F1, 2>(a, st);
    case 3: return launch_q4k_q6k<F1, 3>(a, st);
    case 4: return launch_q4k_q6k<F1, 4>(a, st);
    default:
        if constexpr (F1::Q8IN) {
            return launch_q4k_q6k<F1, 4>(a, st);
        } else {
            if (nk_for<F1>(a.cols) == 6) return launch_q4k_q6k<F1, 6>(a, st);
            return launch_q4k_q6k<F1, 8>(a, st);
        }
    }
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
    // block formats: the unit divides the block, so the host's whole-block check covers it
    case gk::kQ5_0: return gk::FmtQ5_0::UNIT;
    case gk::kQ3_K: return gk::FmtQ3_K::UNIT;
    case gk::kQ5_K: return gk::FmtQ5_K::UNIT;
    case gk::kIQ4_NL: return gk::FmtIQ4_NL::UNIT;
    case gk::kIQ4_XS: return gk::FmtIQ4_XS::UNIT;
    case gk::kMXFP4: return gk::FmtMXFP4::UNIT;
    case gk::kQ5_1: return gk::FmtQ5_1::UNIT;
    case gk::kQ2_K: return gk::FmtQ2_K::UNIT;
    case gk::kIQ3_XXS: return gk::FmtIQ3_XXS::UNIT;
    case gk::kIQ3_S: return gk::FmtIQ3_S::UNIT;
    case gk::kIQ2_S: return gk::FmtIQ2_S::UNIT;
    default: return 0;
    }
}

bool gemv_pair_supported(int first_type, int second_type) {
    return (first_type == gk::kQ4_K && second_type == gk::kQ6_K) ||
           (first_type == gk::kQ3_K && second_type == gk::kQ5_K) ||
           (first_type == gk::kQ5_K && second_type == gk::kQ6_K);
}

hipError_t launch_gemv_pair(const gk::GemvArgs& a, int first_type, int second_type, bool q8_input,
                            hipStream_t st) {
    if (!gemv_pair_supported(first_type, second_type)) return hipErrorInvalidValue;
    if (a.cols <= 0 || a.cols > gk::kMaxGemvCols || a.cols % 256 || a.rows_total <= 0 ||
        a.nseg < 1 || a.nseg > 3)
        return hipErrorInvalidValue;
    // The Q8_1 mode runs Q3_K, Q5_K and Q4_K on the int8 input; Q6_K stays on the fp32 one
    // (its dp4a kernel is opt-in in the reference, CudaForwardPass.java:2031-2038).
    if (first_type == gk::kQ3_K)
        return q8_input ? launch_mix<gk::FmtQ3_KQ8, gk::FmtQ5_KQ8>(a, st) : launch_mix<gk::FmtQ3_K, gk::FmtQ5_K>(a, st);
    if (first_type == gk::kQ5_K)
        return q8_input ? launch_mix<gk::FmtQ5_KQ8, gk::FmtQ6_K>(a, st) : launch_mix<gk::FmtQ5_K, gk::FmtQ6_K>(a, st);
    return q8_input ? launch_pair_f<gk::FmtQ4_KQ8>(a, st) : launch_pair_f<gk::FmtQ4_K>(a, st);
}

hipError_t launch_gemv(const gk::GemvArgs& a, int ggml_type, bool q8_input, hipStream_t st) {
    if (a.cols <= 0 || a.cols > gk::kMaxGemvCols || a.rows_total <= 0 || a.nseg < 1 || a.nseg > 3)
        return hipErrorInvalidValue;
    const int unit = gemv_unit(ggml_type);
    if (unit == 0 || a.cols % unit) return hipErrorInvalidValue;
    if (q8_input) {   // the formats the reference GPU runs on its Q8_1 input (dp4aType != 0, not Q6_K)
        switch (ggml_type) {
        case gk::kQ4_K: return launch_f<gk::FmtQ4_KQ8>(a, st);
        case gk::kQ8_0: return launch_f<gk::FmtQ8_0Q8>(a, st);
        case gk::kQ5_0: return launch_f<gk::FmtQ5_0Q8>(a, st);
        case gk::kQ3_K: return launch_f<gk::FmtQ3_KQ8>(a, st);
        case gk::kQ5_K: return launch_f<gk::FmtQ5_KQ8>(a, st);
        case gk::kIQ4_NL: return launch_f<gk::FmtIQ4_NLQ8>(a, st);
        case gk::kIQ4_XS: return launch_f<gk::FmtIQ4_XSQ8>(a, st);
        default: break;
        }
    }
    switch (ggml_type) {
    case gk::kF32: return launch_f<gk::FmtF32>(a, st);
    case gk::kF16: return launch_f<gk::FmtHalf<false>>(a, st);
    case gk::kBF16: return launch_f<gk::FmtHalf<true>>(a, st);
    case gk::kQ8_0: return launch_f<gk::FmtQ8_0>(a, st);
    case gk::kQ4_0: return launch_f<gk::FmtQ4_0>(a, st);
    case gk::kQ4_K: return launch_f<gk::FmtQ4_K>(a, st);
    case gk::kQ6_K: return launch_f<gk::FmtQ6_K>(a, st);
    case gk::kQ5_0: return launch_f<gk::FmtQ5_0>(a, st);
    case gk::kQ3_K: return launch_f<gk::FmtQ3_K>(a, st);
    case gk::kQ5_K: return launch_f<gk::FmtQ5_K>(a, st);
    case gk::kIQ4_NL: return launch_f<gk::FmtIQ4_NL>(a, st);
    case gk::kIQ4_XS: return launch_f<gk::FmtIQ4_XS>(a, st);
    case gk::kMXFP4: return launch_f<gk::FmtMXFP4>(a, st);
    case gk::kQ5_1: return launch_f<gk::FmtQ5_1>(a, st);
    case gk::kQ2_K: return launch_f<gk::FmtQ2_K>(a, st);
    case gk::kIQ3_XXS: return launch_f<gk::FmtIQ3_XXS>(a, st);
    case gk::kIQ3_S: return launch_f<gk::FmtIQ3_S>(a, st);
    case gk::kIQ2_S: return launch_f<gk::FmtIQ2_S>(a, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_post_norm_residual(const float* xb, const float* w, float eps, float rscale,
                                     float* x, int dim, int n_tokens, hipStream_t st) {
    if (n_tokens < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gk::post_norm_residual_kernel<gk::kPostThreads>, dim3(n_tokens),
                       dim3(gk::kPostThreads), 0, st, xb, w, eps, rscale, x, dim);
    return hipGetLastError();
}

}  // namespace llmp
