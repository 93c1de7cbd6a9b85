// The reference's operator signatures (strixite kernels/*.hpp, unchanged) on top of libstrixite_amd's C ABI.
//
// A maintainer adds this file to strixite's strix_kernels target in place of kernels/linear.hip, linear_q4.hip,
// linear_q56.hip, linear_q8.hip, linear_wmma.hip, moe_router.hip, moe_grouped.hip, swiglu.hip, logits_topk.hip and
// mtp_pick.hip, and links libstrixite_amd.so; it is
// compiled inside the strixite tree (it includes strixite's own headers), so runtime/qwen4exp.cpp and serve/engine.cpp
// call the gfx950 kernels without a change. Every function forwards to the sx_* entry point that replaces it and turns
// a nonzero status into strix::Error with the library's message (common/check.hpp's exception type).
#include "common/check.hpp"
#include "common/hip_check.hpp"
#include "kernels/linear.hpp"
#include "kernels/linear_q4.hpp"
#include "kernels/linear_q5.hpp"
#include "kernels/linear_q6.hpp"
#include "kernels/linear_q8.hpp"
#include "kernels/linear_wmma.hpp"
#include "kernels/logits_topk.hpp"
#include "kernels/moe_grouped.hpp"
#include "kernels/moe_router.hpp"
#include "kernels/mtp_pick.hpp"
#include "kernels/swiglu.hpp"

#include "strixite_amd.h"

namespace strix::kernels {

namespace {

sx_qview qv(const Q4DeviceView &w) { return {w.q, w.scale, w.minv, w.N, w.K, w.G}; }
sx_qview qv(const Q8DeviceView &w) { return {w.q, w.scale, w.minv, w.N, w.K, w.G}; }
sx_stream st(hipStream_t s) { return reinterpret_cast<sx_stream>(s); }

void ok(int rc, const char *fn) {
    if (rc != SX_OK) STRIX_FAIL(fn, ": ", sx_last_error());
}

static_assert(sizeof(LogitCand) == sizeof(sx_logit_cand), "LogitCand and sx_logit_cand share a layout");
static_assert(sizeof(MtpPick) == sizeof(sx_mtp_pick_t), "MtpPick and sx_mtp_pick_t share a layout");
static_assert(sizeof(EmbeddingError) == sizeof(unsigned long long), "EmbeddingError is one 64-bit word");

}  // namespace

// ---- kernels/linear_q4.hpp ----
void linear_q4(const void *x, const Q4DeviceView &w, void *y, int64_t M, Act act, hipStream_t stream) {
    linear_q4(x, w, y, M, act, act, stream);
}
void linear_q4(const void *x, const Q4DeviceView &w, void *y, int64_t M, Act act, Act out_act, hipStream_t stream) {
    const sx_qview v = qv(w);
    ok(sx_linear_q4(x, &v, y, M, (int)act, (int)out_act, st(stream)), "linear_q4");
}
void linear_q4_experts_gather(const void *x, const Q4DeviceView &w, int64_t E, const int32_t *ids, int64_t M,
                              int64_t A, void *y, Act act, uint32_t *err, hipStream_t stream) {
    const sx_qview v = qv(w);
    ok(sx_linear_q4_experts_gather(x, &v, E, ids, M, A, y, (int)act, err, st(stream)), "linear_q4_experts_gather");
}
void linear_q4_experts_combine(const void *h, const Q4DeviceView &w, int64_t E, const int32_t *ids,
                               const float *coef, int64_t M, int64_t A, void *y, Act act, uint32_t *err,
                               hipStream_t stream) {
    const sx_qview v = qv(w);
    ok(sx_linear_q4_experts_combine(h, &v, E, ids, coef, M, A, y, (int)act, err, st(stream)),
       "linear_q4_experts_combine");
}
void linear_q4_experts_gather_swiglu(const void *x, const Q4DeviceView &w, int64_t E, const int32_t *ids, int64_t M,
                                     int64_t A, void *h, Act act, uint32_t *err, hipStream_t stream) {
    const sx_qview v = qv(w);
    ok(sx_linear_q4_experts_gather_swiglu(x, &v, E, ids, M, A, h, (int)act, err, st(stream)),
       "linear_q4_experts_gather_swiglu");
}
void check_expert_error(const uint32_t *err, const char *what) {
    STRIX_CHECK(err != nullptr, "check_expert_error(", what, "): null err");
    uint32_t e[3];
    STRIX_HIP_CHECK(hipMemcpy(e, err, sizeof(e), hipMemcpyDeviceToHost), "reading expert error word for ", what);
    report_expert_error(e, what);
}
void report_expert_error(const uint32_t e[3], const char *what) { ok(sx_report_expert_error(e, what), what); }

// Q5 / Q6 are not in the served layout (docs/weights.md:17-31); runtime/qweight.hpp only needs the symbols.
void linear_q5_experts_gather(const void *, const Q5DeviceView &, int64_t, const int32_t *, int64_t, int64_t, void *,
                              Act, uint32_t *, hipStream_t) {
    STRIX_FAIL("linear_q5_experts_gather: Q5 weights are not supported on gfx950");
}
void linear_q5_experts_combine(const void *, const Q5DeviceView &, int64_t, const int32_t *, const float *, int64_t,
                               int64_t, void *, Act, uint32_t *, hipStream_t) {
    STRIX_FAIL("linear_q5_experts_combine: Q5 weights are not supported on gfx950");
}
void linear_q5_experts_gather_swiglu(const void *, const Q5DeviceView &, int64_t, const int32_t *, int64_t, int64_t,
                                     void *, Act, uint32_t *, hipStream_t) {
    STRIX_FAIL("linear_q5_experts_gather_swiglu: Q5 weights are not supported on gfx950");
}

// ---- kernels/linear_q5.hpp, linear_q6.hpp ----
void linear_q5(const void *, const Q5DeviceView &, void *, int64_t, Act, hipStream_t) {
    STRIX_FAIL("linear_q5: Q5 weights are not supported on gfx950");
}
void linear_q5(const void *, const Q5DeviceView &, void *, int64_t, Act, Act, hipStream_t) {
    STRIX_FAIL("linear_q5: Q5 weights are not supported on gfx950");
}
void linear_q6(const void *, const Q6DeviceView &, void *, int64_t, Act, hipStream_t) {
    STRIX_FAIL("linear_q6: Q6 weights are not supported on gfx950");
}
void linear_q6(const void *, const Q6DeviceView &, void *, int64_t, Act, Act, hipStream_t) {
    STRIX_FAIL("linear_q6: Q6 weights are not supported on gfx950");
}

// ---- kernels/linear_q8.hpp ----
void linear_q8(const void *x, const Q8DeviceView &w, void *y, int64_t M, Act act, hipStream_t stream) {
    linear_q8(x, w, y, M, act, act, stream);
}
void linear_q8(const void *x, const Q8DeviceView &w, void *y, int64_t M, Act act, Act out_act, hipStream_t stream) {
    const sx_qview v = qv(w);
    ok(sx_linear_q8(x, &v, y, M, (int)act, (int)out_act, st(stream)), "linear_q8");
}

// ---- kernels/linear.hpp: BF16 weights (the router projection, W [E + 1, d]) ----
void linear_bf16w(const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, Act act,
                  hipStream_t stream) {
    linear_bf16w(x, w, y, M, N, K, act, act, stream);
}
void linear_bf16w(const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, Act act, Act out_act,
                  hipStream_t stream) {
    ok(sx_linear_bf16w(x, w, y, M, N, K, (int)act, (int)out_act, st(stream)), "linear_bf16w");
}

// ---- kernels/linear_wmma.hpp: the prefill-width dense linears run the same MFMA kernels (16 rows a weight pass) ----
// With FP32 x these keep x exact (three BF16 planes on the matrix cores), where the reference's wmma contract rounds
// x to BF16 first: the results are the exact path's, within FP32 rounding of the exact product.
void linear_q4_wmma(const void *x, const Q4DeviceView &w, void *y, int64_t M, Act act, Act out_act,
                    hipStream_t stream) {
    linear_q4(x, w, y, M, act, out_act, stream);
}
void linear_q8_wmma(const void *x, const Q8DeviceView &w, void *y, int64_t M, Act act, Act out_act,
                    hipStream_t stream) {
    linear_q8(x, w, y, M, act, out_act, stream);
}
void linear_bf16w_wmma(const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, Act act,
                       Act out_act, hipStream_t stream) {
    ok(sx_linear_bf16w_wmma(x, w, y, M, N, K, (int)act, (int)out_act, st(stream)), "linear_bf16w_wmma");
}
void linear_q5_wmma(const void *, const Q5DeviceView &, void *, int64_t, Act, Act, hipStream_t) {
    STRIX_FAIL("linear_q5_wmma: Q5 weights are not supported on gfx950");
}
void linear_q6_wmma(const void *, const Q6DeviceView &, void *, int64_t, Act, Act, hipStream_t) {
    STRIX_FAIL("linear_q6_wmma: Q6 weights are not supported on gfx950");
}

// ---- kernels/moe_router.hpp ----
void moe_router(const void *logits, int64_t ld, int64_t M, int64_t E, int64_t k, const void *shared_logit,
                int64_t shared_ld, int32_t shared_id, int32_t *ids, float *coef, Act act, uint32_t *err,
                hipStream_t stream) {
    ok(sx_moe_router(logits, ld, M, E, k, shared_logit, shared_ld, shared_id, ids, coef, (int)act, err, st(stream)),
       "moe_router");
}
void check_router_error(const uint32_t *err, const char *what) {
    STRIX_CHECK(err != nullptr, "check_router_error(", what, "): null err");
    uint32_t e[3];
    STRIX_HIP_CHECK(hipMemcpy(e, err, sizeof(e), hipMemcpyDeviceToHost), "reading router error word for ", what);
    report_router_error(e, what);
}
void report_router_error(const uint32_t e[3], const char *what) { ok(sx_report_router_error(e, what), what); }
void moe_shared_add(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                    uint32_t gate_index, Act act, uint32_t *err, hipStream_t stream) {
    ok(sx_moe_shared_add(y, s, gate_logit, gate_ld, M, N, gate_index, (int)act, err, st(stream)), "moe_shared_add");
}
void moe_shared_add_inject(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                           uint32_t gate_index, void *x, const float *w_in, int64_t H, Act act, uint32_t *err,
                           hipStream_t stream) {
    ok(sx_moe_shared_add_inject(y, s, gate_logit, gate_ld, M, N, gate_index, x, w_in, H, (int)act, err, st(stream)),
       "moe_shared_add_inject");
}

// ---- kernels/moe_grouped.hpp ----
size_t moe_route_workspace_bytes(int64_t M, int64_t A, int64_t E) {
    size_t b = 0;
    ok(sx_moe_route_workspace_bytes(M, A, E, &b), "moe_route_workspace_bytes");
    return b;
}
void moe_group_routes(const int32_t *ids, int64_t M, int64_t A, int64_t E, void *ws, size_t ws_bytes, uint32_t *err,
                      hipStream_t stream) {
    ok(sx_moe_group_routes(ids, M, A, E, ws, ws_bytes, err, st(stream)), "moe_group_routes");
}
void linear_q4_experts_gather_grouped(const void *x, const Q4DeviceView &w, int64_t E, const void *ws,
                                      size_t ws_bytes, int64_t M, int64_t A, void *y, Act act, MoeMath math,
                                      hipStream_t stream) {
    const sx_qview v = qv(w);
    ok(sx_linear_q4_experts_gather_grouped(x, &v, E, ws, ws_bytes, M, A, y, (int)act, (int)math, st(stream)),
       "linear_q4_experts_gather_grouped");
}
void linear_q4_experts_combine_grouped(const void *h, const Q4DeviceView &w, int64_t E, const int32_t *ids,
                                       const float *coef, const void *ws, size_t ws_bytes, float *partial, int64_t M,
                                       int64_t A, void *y, Act act, MoeMath math, hipStream_t stream) {
    const sx_qview v = qv(w);
    ok(sx_linear_q4_experts_combine_grouped(h, &v, E, ids, coef, ws, ws_bytes, partial, M, A, y, (int)act, (int)math,
                                            st(stream)),
       "linear_q4_experts_combine_grouped");
}
void linear_q5_experts_gather_grouped(const void *, const Q5DeviceView &, int64_t, const void *, size_t, int64_t,
                                      int64_t, void *, Act, MoeMath, hipStream_t) {
    STRIX_FAIL("linear_q5_experts_gather_grouped: Q5 weights are not supported on gfx950");
}
void linear_q5_experts_combine_grouped(const void *, const Q5DeviceView &, int64_t, const int32_t *, const float *,
                                       const void *, size_t, float *, int64_t, int64_t, void *, Act, MoeMath,
                                       hipStream_t) {
    STRIX_FAIL("linear_q5_experts_combine_grouped: Q5 weights are not supported on gfx950");
}

// ---- kernels/swiglu.hpp ----
void swiglu(const void *gu, void *h, int64_t rows, int64_t I, Act act, hipStream_t stream) {
    ok(sx_swiglu(gu, h, rows, I, (int)act, st(stream)), "swiglu");
}

// ---- kernels/logits_topk.hpp (kLogitCands = 20 candidates a row) ----
size_t logits_topk_workspace_bytes(int64_t rows, int64_t n_valid) {
    size_t b = 0;
    ok(sx_logits_topk_workspace_bytes(rows, n_valid, kLogitCands, &b), "logits_topk_workspace_bytes");
    return b;
}
void logits_topk(const float *logits, int64_t rows, int64_t ld, int64_t n_valid, LogitCand *out, uint32_t *nan,
                 void *workspace, size_t workspace_bytes, hipStream_t stream, const uint32_t *mask,
                 int64_t mask_words) {
    ok(sx_logits_topk(logits, rows, ld, n_valid, kLogitCands, reinterpret_cast<sx_logit_cand *>(out), nan, workspace,
                      workspace_bytes, mask, mask_words, st(stream)),
       "logits_topk");
}

// ---- kernels/mtp_pick.hpp ----
void mtp_pick(const float *logits, int64_t n, const uint32_t *router_err, const uint32_t *expert_err,
              const uint32_t *attn_err, const EmbeddingError *emb_err, MtpPick *out, hipStream_t stream) {
    ok(sx_mtp_pick(logits, n, router_err, expert_err, attn_err, reinterpret_cast<const unsigned long long *>(emb_err),
                   reinterpret_cast<sx_mtp_pick_t *>(out), st(stream)),
       "mtp_pick");
}

}  // namespace strix::kernels
