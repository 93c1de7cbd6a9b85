// Prefill-width grouped expert GEMM (q4 G = 128 experts, BF16 activations) on the matrix cores.
#pragma once
#include "qmm.hpp"

namespace sx::gg {

// Tokens from which the grouped entry points take this kernel (the reference switches its grouped path to the WMMA
// tiles at prefill width; at verify width buckets hold a few slots and qmm's one pass over the weights wins).
constexpr int64_t kPrefillMinTokens = 32;

bool eligible(int bits, int64_t G, int64_t K, int act);
// Tokens from which a dense linear takes the grouped kernel's tiles (launch_dense): below, its few tiles leave the
// chip idle and qmm's dense mode is faster. 4096 x 4096, qmm against the tiles: q4 37 / 59 us at M = 128, 64 / 59 at
// 255; q8 68 / 91 at 128, 88 / 92 at 192, 115 / 92 at 255.
constexpr int64_t kDenseMinTokens = 256, kDenseMinTokensQ8 = 200;
constexpr int64_t dense_min_tokens(int bits) { return bits == 8 ? kDenseMinTokensQ8 : kDenseMinTokens; }
// The dense linears the tiles take: eligible's q4, and q8 (G = 64, K % 256 == 0, K <= 4096, BF16 x).
bool eligible_dense(int bits, int64_t G, int64_t K, int act);
// A dense linear at prefill width on the same tiles: y [M, w->N] (BF16 or FP32) = x [M, K] (BF16) . deq(w)^T, tile u
// = tokens 64 u .. 64 u + 63 (eligible_dense(bits, G, K, BF16)).
hipError_t launch_dense(const void *x, const sx_qview *w, void *y, int64_t M, int out_act, hipStream_t stream);
// mode: qmm::SWIGLU (h [S, N/2]), qmm::GATHER (y [S, N]), qmm::COMBINE (FP32 partials [S, N]); N = w->N / E.
hipError_t launch(int mode, const void *x, const sx_qview *w, void *y, const int32_t *ws, int64_t M, int64_t A,
                  int64_t E, int out_act, hipStream_t stream);

}  // namespace sx::gg
