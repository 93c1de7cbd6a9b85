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

struct LayerSync;

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
    LayerSync *sync;    // nullable: after a fixed run a block, items from the pool counter of its set epoch & 1
    uint32_t epoch;
    void *plan;         // nullable: block 0 stores its routing (ids, coef, the expert list, slot table) here for down
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
    const void *plan;   // nullable: gate_up's stored routing, taken as is instead of rebuilding it from ids / coef
};

// The one-launch layer's shared state: block b stores the launch's epoch (numbered by the host, never 0) into its
// slot of a phase when its part of the phase is done; the logits are published tagged with the epoch; the gate_up
// work counters alternate between two sets by epoch parity. Zero before the first launch; nothing to reset after one.
constexpr int kMaxBlocks = 1024;
constexpr int kMaxRouterRows = 1040;  // router weight rows: E + 1 <= 1025
constexpr int kQueues = 16;           // counter lines a set (the gate_up pool uses the first)
struct LayerSync {
    uint32_t queues[2][kQueues][32];  // gate_up pool counter ([set][0][0]), 128-byte lines; set epoch & 1 in use (the
                                      // other one is zeroed during the launch for the next)
    uint32_t done_b[kMaxBlocks];  // routing + gate_up + SwiGLU (h, h_sums) done
    uint64_t tagged[kMaxTokens * kMaxRouterRows];  // the router logits as (epoch << 32 | value bits) [M, rows]
};

struct LayerParams {
    GateUpParams gu;    // gu.logits = logits (written by the projection phase); gu.h_sums required
    DownParams dn;      // dn.h = gu.h, dn.h_sums = gu.h_sums; ids / coef unused (the routing stays in LDS)
    const void *wr;     // router weight [rows, K]: FP32 or BF16
    int rows;
    float *logits;      // [M, ld = rows]
    int64_t ld;
    LayerSync *sync;
    uint64_t *tagged;   // = sync->tagged, [M, ld]
    uint32_t epoch;
    uint64_t *trace;    // nullable: per block, s_memrealtime stamps of its phase boundaries (kTraceSlots a block)
};
constexpr int kTraceSlots = 16;

hipError_t launch_gate_up(const GateUpParams &p, int cus, hipStream_t stream);
hipError_t launch_down(const DownParams &p, hipStream_t stream);
hipError_t launch_layer(const LayerParams &p, bool wr_f32, int cus, hipStream_t stream);

}  // namespace sx::vf
