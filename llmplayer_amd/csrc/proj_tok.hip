// Instantiation and dispatch of the token-batched projection kernel (proj_tok_kernels.h).
#include "proj_tok_kernels.h"
#include "llmp_internal.h"

namespace llmp {
static_assert(tk::kTok == kTokBatch, "one token count for the kernels and the host");

namespace {

template <class F1, class F2>
hipError_t launch_ff(const tk::ProjTokArgs& a, hipStream_t st) {
    if (a.norm_w != nullptr)
        hipLaunchKernelGGL((tk::proj_tok_kernel<F1, F2, true>), dim3(a.rows_total / 16), dim3(tk::kThreads),
                           (size_t)a.cols * sizeof(float), st, a);
    else
        hipLaunchKernelGGL((tk::proj_tok_kernel<F1, F2, false>), dim3(a.rows_total / 16), dim3(tk::kThreads),
                           0, st, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_tok_prep(const float* x, long long x_pitch, int cols, const float* norm_w, float eps,
                           float* sc, int n_tokens, hipStream_t st) {
    if (x == nullptr || sc == nullptr || cols <= 0 || (cols & 3) || (x_pitch & 3) || n_tokens < 1 ||
        n_tokens > tk::kTok || (reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(norm_w) & 15))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(tk::tok_prep_kernel<tk::kPrepThreads>, dim3(n_tokens), dim3(tk::kPrepThreads), 0, st, x, x_pitch,
                       cols, norm_w, eps, sc);
    return hipGetLastError();
}

hipError_t launch_tok_q8(const float* x, long long x_pitch, int cols, const float* norm_w, float eps,
                         int n_tokens, void* q8b, float* q8d, float* q8s, float* sc, hipStream_t st) {
    if (x == nullptr || q8b == nullptr || q8d == nullptr || q8s == nullptr || cols <= 0 || (cols & 31) ||
        cols > gk::kMaxGemvCols || (x_pitch & 3) || n_tokens < 1 || n_tokens > tk::kTok ||
        (reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(norm_w) & 15) ||
        (reinterpret_cast<uintptr_t>(q8b) & 15))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(tk::tok_q8_kernel<tk::kPrepThreads>, dim3(tk::kTok), dim3(tk::kPrepThreads), (size_t)cols,
                       st, x, x_pitch, cols, norm_w, eps, n_tokens, static_cast<uint4*>(q8b), q8d, q8s, sc);
    return hipGetLastError();
}

bool proj_tok_q8_routed(int ggml_type) {
    switch (ggml_type) {
    case gk::kQ4_K: case gk::kQ8_0: case gk::kQ5_0: case gk::kQ3_K: case gk::kQ5_K: case gk::kIQ4_NL:
    case gk::kIQ4_XS:
        return true;
    default:
        return false;
    }
}

bool proj_tok_supported(int ggml_type) {
    switch (ggml_type) {
    case gk::kF32: case gk::kF16: case gk::kBF16: case gk::kQ8_0: case gk::kQ4_0: case gk::kQ4_K:
    case gk::kQ6_K: case gk::kQ5_0: case gk::kQ3_K: case gk::kQ5_K: case gk::kIQ4_NL: case gk::kIQ4_XS:
    case gk::kMXFP4: case gk::kQ5_1: case gk::kIQ3_XXS: case gk::kIQ3_S: case gk::kIQ2_S: case gk::kQ2_K:
        return true;
    default:
        return false;
    }
}

bool proj_tok_pair_supported(int first_type, int second_type) {
    return (first_type == gk::kQ4_K && second_type == gk::kQ6_K) ||
           (first_type == gk::kQ3_K && second_type == gk::kQ5_K) ||
           (first_type == gk::kQ5_K && second_type == gk::kQ6_K);
}

namespace {
// The Q8_1-input form of a routed type's launch (one type, or one of the two-format mixes).
hipError_t launch_q8(const tk::ProjTokArgs& a, int first_type, int second_type, hipStream_t st) {
    if (a.q8b == nullptr || a.q8d == nullptr || a.q8s == nullptr) return hipErrorInvalidValue;
    using tk::Q8In;
    if (second_type >= 0) {
        if (first_type == gk::kQ3_K) return launch_ff<Q8In<tk::PQ3K>, Q8In<tk::PQ5K>>(a, st);
        if (first_type == gk::kQ5_K) return launch_ff<Q8In<tk::PQ5K>, tk::PQ6K>(a, st);
        return launch_ff<Q8In<tk::PQ4K>, tk::PQ6K>(a, st);
    }
    switch (first_type) {
    case gk::kQ4_K: return launch_ff<Q8In<tk::PQ4K>, Q8In<tk::PQ4K>>(a, st);
    case gk::kQ8_0: return launch_ff<Q8In<tk::PQ8_0>, Q8In<tk::PQ8_0>>(a, st);
    case gk::kQ5_0: return launch_ff<Q8In<tk::PQ5_0>, Q8In<tk::PQ5_0>>(a, st);
    case gk::kQ3_K: return launch_ff<Q8In<tk::PQ3K>, Q8In<tk::PQ3K>>(a, st);
    case gk::kQ5_K: return launch_ff<Q8In<tk::PQ5K>, Q8In<tk::PQ5K>>(a, st);
    case gk::kIQ4_NL: return launch_ff<Q8In<tk::PIQ4_NL>, Q8In<tk::PIQ4_NL>>(a, st);
    case gk::kIQ4_XS: return launch_ff<Q8In<tk::PIQ4_XS>, Q8In<tk::PIQ4_XS>>(a, st);
    default: return hipErrorInvalidValue;
    }
}
}  // namespace

hipError_t launch_proj_tok(const tk::ProjTokArgs& a, int first_type, int second_type, bool q8, hipStream_t st) {
    if ((a.norm_w != nullptr && a.tok_sc == nullptr) || a.cols <= 0 || a.cols % 32 || a.rows_total <= 0 || a.rows_total % 16 || a.K < 1 ||
        a.K > tk::kTok || a.nseg < 1 || a.nseg > 3 || a.x == nullptr || (a.x_pitch & 3) ||
        (reinterpret_cast<uintptr_t>(a.x) & 15) || (reinterpret_cast<uintptr_t>(a.norm_w) & 15) ||
        a.cols > gk::kMaxGemvCols)
        return hipErrorInvalidValue;
    for (int i = 0; i < a.nseg; ++i)
        if (a.seg[i].rows % 16 || a.seg[i].out_off % 16) return hipErrorInvalidValue;
    // super-block formats need whole super-blocks of 256 columns
    auto superblock = [](int t) {
        return t == gk::kQ4_K || t == gk::kQ6_K || t == gk::kQ3_K || t == gk::kQ5_K || t == gk::kIQ4_XS ||
               t == gk::kIQ3_XXS || t == gk::kIQ3_S || t == gk::kIQ2_S || t == gk::kQ2_K;
    };
    if ((superblock(first_type) || superblock(second_type)) && a.cols % 256) return hipErrorInvalidValue;
    if (second_type >= 0 && !proj_tok_pair_supported(first_type, second_type)) return hipErrorInvalidValue;
    // in the Q8_1 mode a pair's first type is always routed (Q4_K, Q3_K, Q5_K)
    if (q8 && proj_tok_q8_routed(first_type)) return launch_q8(a, first_type, second_type, st);
    if (second_type >= 0) {
        if (first_type == gk::kQ3_K) return launch_ff<tk::PQ3K, tk::PQ5K>(a, st);
        if (first_type == gk::kQ5_K) return launch_ff<tk::PQ5K, tk::PQ6K>(a, st);
        return launch_ff<tk::PQ4K, tk::PQ6K>(a, st);
    }
    switch (first_type) {
    case gk::kF32: return launch_ff<tk::PF32, tk::PF32>(a, st);
    case gk::kF16: return launch_ff<tk::PF16, tk::PF16>(a, st);
    case gk::kBF16: return launch_ff<tk::PBF16, tk::PBF16>(a, st);
    case gk::kQ8_0: return launch_ff<tk::PQ8_0, tk::PQ8_0>(a, st);
    case gk::kQ4_0: return launch_ff<tk::PQ4_0, tk::PQ4_0>(a, st);
    case gk::kQ4_K: return launch_ff<tk::PQ4K, tk::PQ4K>(a, st);
    case gk::kQ6_K: return launch_ff<tk::PQ6K, tk::PQ6K>(a, st);
    case gk::kQ5_0: return launch_ff<tk::PQ5_0, tk::PQ5_0>(a, st);
    case gk::kQ3_K: return launch_ff<tk::PQ3K, tk::PQ3K>(a, st);
    case gk::kQ5_K: return launch_ff<tk::PQ5K, tk::PQ5K>(a, st);
    case gk::kIQ4_NL: return launch_ff<tk::PIQ4_NL, tk::PIQ4_NL>(a, st);
    case gk::kIQ4_XS: return launch_ff<tk::PIQ4_XS, tk::PIQ4_XS>(a, st);
    case gk::kMXFP4: return launch_ff<tk::PMXFP4, tk::PMXFP4>(a, st);
    case gk::kQ5_1: return launch_ff<tk::PQ5_1, tk::PQ5_1>(a, st);
    case gk::kQ2_K: return launch_ff<tk::PQ2_K, tk::PQ2_K>(a, st);
    case gk::kIQ3_XXS: return launch_ff<tk::PIQ3_XXS, tk::PIQ3_XXS>(a, st);
    case gk::kIQ3_S: return launch_ff<tk::PIQ3_S, tk::PIQ3_S>(a, st);
    case gk::kIQ2_S: return launch_ff<tk::PIQ2_S, tk::PIQ2_S>(a, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace llmp
