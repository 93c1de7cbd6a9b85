// Verify-width MoE FFN (verify_ffn.hip): routing + gate_up + SwiGLU in one launch, down + combine in another.
#pragma once
#include "common.hpp"

namespace sx::vf {

constexpr int kMaxSlots = 64;        // M * A
constexpr int kMaxTokens = 16;       // M: the rows of one MFMA tile
constexpr int kMaxExperts = 1024;    // experts in the weights
constexpr int kMaxSpansGu = 32;      // gate_up K <= 4096
constexpr int kMaxSpansDn = 16;      // down K <= 2048
constexpr int kHsElems = 64 * 1032;  // down: M * A * (K + 8) BF16 rows of h in LDS

struct GateUpParams {
    const uint16_t *x;  // BF16 [M, K]
    int M, A, k, E, Ew;  // tokens, slots a token (k + shared), top-k, routed experts, experts in the weight
    const float *logits;
    int64_t ld;
    const float *shared_logit;  // nullable
    int64_t shared_ld;
    int shared_id;
    const uint8_t *q;
    const uint16_t *scale, *minv;
    int64_t N, K;       // rows an expert (2I: gate | up), K
    int32_t *ids;
    float *coef;
    uint16_t *h;        // BF16 [M * A, I]
    float *h_sums;      // nullable: FP32 [M * A, ceil(I / 16)], each 16-feature run of an h row summed as stored
    uint32_t *router_err, *expert_err;
};

struct DownParams {
    const uint16_t *h;  // BF16 [M * A, K]
    const float *h_sums;  // nullable: gate_up's 16-feature sums of h (else the span sums are taken from h here)
    int M, A, Ew;
    const int32_t *ids;
    const float *coef;
    const uint8_t *q;
    const uint16_t *scale, *minv;
    int64_t N, K;       // rows an expert (d), K (I)
    void *y;            // [M, N] in act
    int act;
    uint32_t *expert_err;
};

hipError_t launch_gate_up(const GateUpParams &p, int cus, hipStream_t stream);
hipError_t launch_down(const DownParams &p, hipStream_t stream);

}  // namespace sx::vf
