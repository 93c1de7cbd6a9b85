// Prefill-width grouped expert GEMM (q4 G = 128 experts, BF16 activations) on the matrix cores.
#pragma once
#include "qmm.hpp"

namespace sx::gg {

// Tokens from which the grouped entry points take this kernel (the reference switches its grouped path to the WMMA
// tiles at prefill width; at verify width buckets hold a few slots and qmm's one pass over the weights wins).
constexpr int64_t kPrefillMinTokens = 32;

bool eligible(int bits, int64_t G, int64_t K, int act);
// Tokens from which a dense linear takes the MFMA tiles (launch_dense): below, qmm's dense mode is faster. 4096 x
// 4096, qmm against the K-split tiles (gs_kernel): q4 20.2 / 23.0 us at M = 64, 25.2 / 23.1 at 96; q8 23.7 / 29.3 at
// 32, 34.0 / 29.5 at 64.
constexpr int64_t kDenseMinTokens = 96, kDenseMinTokensQ8 = 48;
constexpr int64_t dense_min_tokens(int bits) { return bits == 8 ? kDenseMinTokensQ8 : kDenseMinTokens; }
// Up to this many tokens launch_dense splits K over each block's waves (gs_kernel): four times the blocks, a quarter
// of the steps each. 4096 x 4096, gs_kernel against gg_kernel: q4 23.5 / 51.5 us at M = 256, 45.9 / 52.0 at 512,
// 90.4 / 53.2 at 1024; q8 31.3 / 82.5 at 256, 60.8 / 83.2 at 512, 119.8 / 83.5 at 1024.
constexpr int64_t kDenseSplitMaxTokens = 512;
// The dense linears the tiles take: eligible's q4, and q8 (G = 64, K % 256 == 0, K <= 4096, BF16 x).
bool eligible_dense(int bits, int64_t G, int64_t K, int act);
// A dense linear at prefill width on the same tiles: y [M, w->N] (BF16 or FP32) = x [M, K] (BF16) . deq(w)^T, tile u
// = tokens 64 u .. 64 u + 63 (eligible_dense(bits, G, K, BF16)).
hipError_t launch_dense(const void *x, const sx_qview *w, void *y, int64_t M, int out_act, hipStream_t stream);
// mode: qmm::SWIGLU (h [S, N/2]), qmm::GATHER (y [S, N]), qmm::COMBINE (FP32 partials [S, N]); N = w->N / E.
hipError_t launch(int mode, const void *x, const sx_qview *w, void *y, const int32_t *ws, int64_t M, int64_t A,
                  int64_t E, int out_act, hipStream_t stream);

}  // namespace sx::gg
