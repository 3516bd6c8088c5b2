// Linear-layer GEMMs: forward (matmul_nt_v2.comp), dx
// (linear_backward_dx_batched.comp) and dW (linear_backward_dw_batched.comp)
// on MFMA, with fused residual / accumulate epilogues.
#include "gemm.hpp"
#include "ops.hpp"

namespace vkh {

namespace {

inline int es(DType d) { return d == DType::F32 ? 4 : 2; }

template <Lay LA, Lay LB, class Epi>
hipError_t run(Precision pr, Mat a, Mat b, int M, int N, int K, const Epi &epi,
               hipStream_t st) {
    GemmOperand oa{a.p, a.ld, vec_ok(a.p, a.ld, es(a.dt), LA)};
    GemmOperand ob{b.p, b.ld, vec_ok(b.p, b.ld, es(b.dt), LB)};
    GemmShape s{M, N, K};
    if (pr == Precision::FP32) {
        if (a.dt != DType::F32 || b.dt != DType::F32) return hipErrorInvalidValue;
        return gemm_dispatch<false, float, LA, float, LB>(oa, ob, s, epi, st);
    }
    if (a.dt == DType::F32 && b.dt == DType::F32)
        return gemm_dispatch<true, float, LA, float, LB>(oa, ob, s, epi, st);
    if (a.dt == DType::BF16 && b.dt == DType::F32)
        return gemm_dispatch<true, bf16, LA, float, LB>(oa, ob, s, epi, st);
    if (a.dt == DType::F32 && b.dt == DType::BF16)
        return gemm_dispatch<true, float, LA, bf16, LB>(oa, ob, s, epi, st);
    return gemm_dispatch<true, bf16, LA, bf16, LB>(oa, ob, s, epi, st);
}

}  // namespace

hipError_t gemm_nt(Precision pr, Mat x, Mat w, float *y, long ldy, int M, int N, int K,
                   const float *R, long ldr, float alpha, float beta, hipStream_t st) {
    EpiStore e{y, ldy, R, ldr, alpha, beta};
    return run<Lay::K, Lay::K>(pr, x, w, M, N, K, e, st);
}

hipError_t gemm_nn(Precision pr, Mat dy, Mat w, float *dx, long lddx, int M, int N, int K,
                   float alpha, float beta, hipStream_t st) {
    // C[m, k'] = sum_n dy[m, n] W[n, k']: contraction over N; B(k', n) = W[n*ld + k'].
    EpiStore e{dx, lddx, nullptr, 0, alpha, beta};
    return run<Lay::K, Lay::MN>(pr, dy, w, M, K, N, e, st);
}

hipError_t gemm_tn(Precision pr, Mat dy, Mat x, float *dw, long lddw, int M, int N, int K,
                   float alpha, float beta, hipStream_t st) {
    // C[n, k'] = sum_m dy[m, n] x[m, k']: contraction over M; both operands MN-major.
    EpiStore e{dw, lddw, nullptr, 0, alpha, beta};
    return run<Lay::MN, Lay::MN>(pr, dy, x, N, K, M, e, st);
}

hipError_t gemm_nt_bf16out(Mat x, Mat w, bf16 *y, long ldy, int M, int N, int K, float alpha,
                           hipStream_t st) {
    EpiStoreBf16 e{y, ldy, alpha};
    return run<Lay::K, Lay::K>(Precision::BF16, x, w, M, N, K, e, st);
}

}  // namespace vkh
