// wm_prefill_kq.hip -- the K-quant instances of the prefill expert GEMMs
// (wm_pf_gemm.h), in a translation unit of their own so that they build in
// parallel with the rest.
#include <hip/hip_runtime.h>

#include "wm_pf_gemm.h"

namespace wm {

template <int WT, int M> static int launch_down(int nsub, const PfGemm& g, int n_wg, hipStream_t s) {
    return nsub == 4 ? launch_pf_gemm<1, 2, 4, WT, M>(g, n_wg, s) : launch_pf_gemm<1, 2, 2, WT, M>(g, n_wg, s);
}

template <int M> static int launch_kq(int nmat, int nsub, int wt, const PfGemm& g, int n_wg, hipStream_t s) {
    if constexpr (M == 16) {
        // with passes of 16 pairs and H a multiple of 512, Q2_K .. Q4_K run
        // gate and up in alternate stages of two super-blocks per row: runs
        // twice as long per row at the same stage size
        if (nmat == 2 && g.ncol_r % 512 == 0 && g.ncol_s % 512 == 0) {
            switch (wt) {
            case Q2_K: return launch_pf_gemm<1, 1, 2, Q2_K, 16, 2>(g, n_wg, s);
            case Q3_K: return launch_pf_gemm<1, 1, 2, Q3_K, 16, 2>(g, n_wg, s);
            case Q4_K: return launch_pf_gemm<1, 1, 2, Q4_K, 16, 2>(g, n_wg, s);
            default: break;
            }
        }
    }
    if (nmat == 2) {
        // gate and up in one stage (half the stages of alternating them, at
        // a 2-deep ring: faster for these formats); Q6_K's row slots only fit
        // as alternate gate and up stages
        switch (wt) {
        case Q2_K: return launch_pf_gemm<2, 1, 1, Q2_K, M>(g, n_wg, s);
        case Q3_K: return launch_pf_gemm<2, 1, 1, Q3_K, M>(g, n_wg, s);
        case Q4_K: return launch_pf_gemm<2, 1, 1, Q4_K, M>(g, n_wg, s);
        case Q5_K: return launch_pf_gemm<2, 1, 1, Q5_K, M>(g, n_wg, s);
        case Q6_K: return launch_pf_gemm<1, 1, 2, Q6_K, M>(g, n_wg, s);
        default: return (int)hipErrorInvalidValue;
        }
    }
    if (nmat != 1 || (nsub != 2 && nsub != 4)) return (int)hipErrorInvalidValue;
    switch (wt) {
    case Q2_K: return launch_down<Q2_K, M>(nsub, g, n_wg, s);
    case Q3_K: return launch_down<Q3_K, M>(nsub, g, n_wg, s);
    case Q4_K: return launch_down<Q4_K, M>(nsub, g, n_wg, s);
    case Q5_K: return launch_down<Q5_K, M>(nsub, g, n_wg, s);
    case Q6_K: return launch_down<Q6_K, M>(nsub, g, n_wg, s);
    default: return (int)hipErrorInvalidValue;
    }
}

int launch_pf_gemm_kq(int m, int nmat, int nsub, int wt, const PfGemm& g, int n_wg, hipStream_t s) {
    if (m == 16) return launch_kq<16>(nmat, nsub, wt, g, n_wg, s);
    if (m == 32) return launch_kq<32>(nmat, nsub, wt, g, n_wg, s);
    return (int)hipErrorInvalidValue;
}

}  // namespace wm
