// Host-side entry points of the MFMA GEMM engine, shared by the dense, attention and convolution translation units.
#pragma once

#include "om_gemm_core.hpp"

namespace omg {

// Tile shape and K split chosen from the shape and the CU count only (so results never depend on anything else).
struct Choice {
    int bm, bn, splits, k_split, bkt;
    int dma = 0;  // 1: an NT product on the direct-to-LDS kernel even when its tiles take more than one round
};
Choice choose(int m, int n, int k, int batch, int cus);
// A zeroed Params for a single dense product C[m,n] = A[m,k] B[k,n] with the given leading dimensions.
Params dense_params(int m, int n, int k, const float *a, int64_t lda, const float *b, int64_t ldb, float *c,
                    int64_t ldc);
// Launches a dense (optionally batched) product; adds the split-K reduce when the chooser splits K.
// With p.db set on a weight-gradient product (ta, !tb), the bias gradient db (+)= column sums of A is fused into the
// launch when the chosen kernel supports it; *colsum_fused reports whether it was (else p.db was ignored). With p.mse_t
// set, *mse_slots reports the wavefront partials of the fused MSE written to p.mse_part (0: the launch took a kernel
// without that epilogue, and p.mse_t was ignored).
om_status launch_dense(om_ctx *ctx, Params p, bool ta, bool tb, int batch, const char *what,
                       bool *colsum_fused = nullptr, int *mse_slots = nullptr);

}  // namespace omg
