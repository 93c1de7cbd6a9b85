// C-ABI entry points of the dequantizing GEMMs: dense linear (q4 / q8) and the per-slot and grouped MoE experts.
// Host-side preconditions follow the reference launchers (kernels/linear_q4.hip:353-440, linear_q8.hip:192-223,
// moe_grouped.hip:476-556); the work runs in qmm_impl.hpp.
#include "common.hpp"
#include "gemm_grouped.hpp"
#include "dense_ks.hpp"
#include "qmm.hpp"

namespace sx {
namespace {

using qmm::Params;

constexpr int64_t kMaxN = 0x7fffffff;
constexpr int64_t kMaxK = 1 << 24;
constexpr size_t kLdsBudget = 56 * 1024;  // x staging per block: 2 blocks (8 waves) a CU of the 160 KB

// Checks of a weight view shared by every entry point (linear_q4.hip:353-362).
int check_view(const char *fn, const sx_qview *w, int bits) {
    if (w == nullptr) {
        set_error(cat(fn, ": null weight view"));
        return SX_EINVAL;
    }
    if (!(w->q && w->scale && w->minv)) {
        set_error(cat(fn, ": null weight pointer (q=", (const void *)w->q, ", scale=", w->scale, ", min=", w->minv, ")"));
        return SX_EINVAL;
    }
    if (!(w->G == 32 || w->G == 64 || w->G == 128)) {
        set_error(cat(fn, ": group size ", w->G, " unsupported (32, 64 or 128)"));
        return SX_EINVAL;
    }
    if (!(w->N >= 1 && w->N <= kMaxN)) {
        set_error(cat(fn, ": N = ", w->N, ", expected 1..", kMaxN));
        return SX_EINVAL;
    }
    if (!(w->K >= w->G && w->K <= kMaxK && w->K % w->G == 0)) {
        set_error(cat(fn, ": K = ", w->K, " must be a positive multiple of group size ", w->G, " and <= ", kMaxK));
        return SX_EINVAL;
    }
    if (!aligned(w->q, 16)) {
        set_error(cat(fn, ": code array ", (const void *)w->q, " must be 16-byte aligned for vector loads"));
        return SX_EINVAL;
    }
    return SX_OK;
}

// Activation rows one block stages in LDS: up to `want` (<= 16), as many as fit the budget.
int rows_that_fit(int bits, int nsplit, int64_t K, int64_t G, int want, size_t budget = kLdsBudget) {
    int r = want < 16 ? want : 16;
    while (r > 1 && qmm::lds_bytes(bits, nsplit, K, G, r, 1) > budget) --r;
    return r;
}

// Tiles a block covers: 4 waves x tiles a wave, enough waves for the chip (~8 a CU) but no more than the work.
int tiles_per_chunk(int64_t total_tiles) {
    const int64_t waves = (int64_t)device_cus() * 8;
    int64_t tpw = (total_tiles + waves - 1) / waves;
    tpw = tpw < 1 ? 1 : tpw > 16 ? 16 : tpw;
    return (int)(tpw * qmm::kWaves);
}

int launch_qmm(const char *fn, int mode, int bits, int act_x, int act_y, Params &p, int64_t units, int64_t rows_out,
               int64_t grid_y, hipStream_t stream) {
    const int64_t tiles = (rows_out + qmm::kTile - 1) / qmm::kTile;
    p.tiles_per_chunk = tiles_per_chunk(tiles * units);
    p.nchunks = (int)((tiles + p.tiles_per_chunk - 1) / p.tiles_per_chunk);
    const int64_t gx = units * p.nchunks;
    SX_CHECK(gx >= 1 && gx <= 0x7fffffff && grid_y <= 65535, fn, " grid ", gx, " x ", grid_y, " out of range");
    SX_HIP(qmm::launch(mode, bits, act_x, act_y, p, dim3((unsigned)gx, (unsigned)grid_y), stream), fn);
    return SX_OK;
}

int linear(const char *fn, int bits, const void *x, const sx_qview *w, void *y, int64_t M, int act, int out_act,
           sx_stream stream) {
    SX_CHECK(x != nullptr && y != nullptr, fn, " null pointer (x=", x, ", y=", y, ")");
    if (int rc = check_view(fn, w, bits)) return rc;
    SX_CHECK(M >= 1 && M <= 65535ll * 8, fn, " M (rows of x) = ", M, ", expected 1..", 65535ll * 8);
    SX_CHECK(aligned(x, 16), fn, " x ", x, " must be 16-byte aligned for vector loads");
    SX_CHECK(act == SX_ACT_F32 || act == SX_ACT_BF16, fn, " unsupported activation dtype ", act);
    SX_CHECK(out_act == act || (act == SX_ACT_BF16 && out_act == SX_ACT_F32), fn, " output dtype ", out_act,
             " with input ", act, " unsupported (same dtype, or BF16 -> F32)");
    SX_CHECK(apart(x, M * w->K * act_bytes(act), y, M * w->N * act_bytes(out_act)), fn, " output y [", y, ", +",
             M * w->N * act_bytes(out_act), " B) overlaps input x [", x, ", +", M * w->K * act_bytes(act), " B)");
    if (dks::eligible(bits, w->G, w->N, w->K, M, act, out_act, device_cus())) {  // decode width: K split over a block
        dks::Params d{};
        d.x = x, d.q = w->q, d.scale = w->scale, d.minv = w->minv, d.y = y, d.M = (int)M, d.N = w->N, d.K = w->K;
        SX_HIP(dks::launch(bits, w->G, act, out_act, d, device_cus(), stream_of(stream)), fn);
        return SX_OK;
    }
    if (M >= gg::dense_min_tokens(bits) && gg::eligible_dense(bits, w->G, w->K, act) && aligned(w->scale, 4) &&
        aligned(w->minv, 4)) {  // prefill width: the grouped kernel's MFMA tiles, the tokens as one bucket
        SX_HIP(gg::launch_dense(x, w, y, M, out_act, stream_of(stream)), fn);
        return SX_OK;
    }
    const int nsplit = act == SX_ACT_F32 ? 3 : 1;
    const int rows = rows_that_fit(bits, nsplit, w->K, w->G, (int)(M < 16 ? M : 16));
    SX_CHECK(qmm::lds_bytes(bits, nsplit, w->K, w->G, rows, 1) <= 160 * 1024, fn, " K = ", w->K,
             " too long to stage one activation row in LDS");
    Params p{};
    p.x = x, p.q = w->q, p.scale = w->scale, p.minv = w->minv, p.y = y;
    p.M = M, p.A = 1, p.E = 1, p.N = w->N, p.K = w->K, p.G = (int)w->G, p.max_rows = rows;
    return launch_qmm(fn, qmm::DENSE, bits, act, out_act, p, 1, w->N, (M + rows - 1) / rows, stream_of(stream));
}

int experts_common(const char *fn, const void *x, const sx_qview *w, int64_t E, int64_t M, int64_t A, void *y,
                   int act) {
    SX_CHECK(x != nullptr && y != nullptr, fn, " null pointer (x=", x, ", y=", y, ")");
    if (int rc = check_view(fn, w, 4)) return rc;
    SX_CHECK(E >= 1 && w->N % E == 0, fn, " weight has ", w->N, " rows, not a multiple of E = ", E, " experts");
    SX_CHECK(M >= 1 && M <= 65535, fn, " M (tokens) = ", M, ", expected 1..65535");
    SX_CHECK(A >= 1 && A <= 64 && A <= E, fn, " A (active experts per token) = ", A, ", expected 1..min(64, E=", E, ")");
    SX_CHECK(aligned(x, 16), fn, " input ", x, " must be 16-byte aligned");
    SX_CHECK(act == SX_ACT_F32 || act == SX_ACT_BF16, fn, " unsupported activation dtype ", act);
    return SX_OK;
}

// The route workspace checks of moe_grouped.hip:476-497, plus the header E read back from nothing: the layout is
// recomputed on the host from (M, A, E).
int grouped_common(const char *fn, const void *x, const sx_qview *w, int64_t E, int64_t M, int64_t A, const void *ws,
                   size_t ws_bytes, void *y, int act, int math) {
    if (int rc = experts_common(fn, x, w, E, M, A, y, act)) return rc;
    SX_CHECK(ws != nullptr, fn, " null workspace");
    SX_CHECK(E <= 1023 && M * A <= (1 << 20), fn, " E = ", E, " (<= 1023), M*A = ", M * A, " (<= 2^20)");
    size_t need = 0;
    if (int rc = sx_moe_route_workspace_bytes(M, A, E, &need)) return rc;
    SX_CHECK(ws_bytes >= need, fn, " workspace of ", ws_bytes, " bytes, needs ", need, " for M = ", M, ", A = ", A,
             ", E = ", E);
    SX_CHECK(math == SX_MOE_F32 || math == SX_MOE_WMMA_BF16 || math == SX_MOE_WMMA_F16, fn, " unknown math ", math);
    return SX_OK;
}

}  // namespace
}  // namespace sx

using namespace sx;

extern "C" {

int sx_linear_q4(const void *x, const sx_qview *w, void *y, int64_t M, int act, int out_act, sx_stream stream) {
    return linear("sx_linear_q4", 4, x, w, y, M, act, out_act, stream);
}

int sx_linear_q8(const void *x, const sx_qview *w, void *y, int64_t M, int act, int out_act, sx_stream stream) {
    return linear("sx_linear_q8", 8, x, w, y, M, act, out_act, stream);
}

int sx_mtp_head_pick(const void *x, const sx_qview *w, int bits, float *logits, const uint32_t *router_err,
                     const uint32_t *expert_err, const uint32_t *attn_err, const unsigned long long *emb_err,
                     sx_mtp_pick_t *out, void *workspace, size_t workspace_bytes, sx_stream stream) {
    const char *fn = "sx_mtp_head_pick";
    SX_CHECK(bits == 4 || bits == 8, fn, " bits = ", bits, ", expected 4 or 8");
    SX_CHECK(x && logits && router_err && expert_err && attn_err && emb_err && out && workspace, fn, " null pointer");
    if (int rc = check_view(fn, w, bits)) return rc;
    SX_CHECK(aligned(x, 16), fn, " x ", x, " must be 16-byte aligned for vector loads");
    SX_CHECK(apart(x, w->K * 2, logits, w->N * 4), fn, " logits overlap x");
    SX_CHECK(workspace_bytes >= sizeof(pick::Workspace), fn, " workspace ", workspace_bytes, " bytes, need ",
             sizeof(pick::Workspace));
    SX_CHECK(aligned(workspace, 16), fn, " workspace must be 16-byte aligned");
    const pick::Args pa{static_cast<pick::Workspace *>(workspace), router_err, expert_err, attn_err, emb_err, out};
    const int cus = device_cus();
    if (cus <= pick::kMaxParts && dks::eligible(bits, w->G, w->N, w->K, 1, SX_ACT_BF16, SX_ACT_F32, cus)) {
        dks::Params d{};
        d.x = x, d.q = w->q, d.scale = w->scale, d.minv = w->minv, d.y = logits, d.M = 1, d.N = w->N, d.K = w->K;
        d.pick = pa;
        SX_HIP(dks::launch(bits, w->G, SX_ACT_BF16, SX_ACT_F32, d, cus, stream_of(stream)), fn);
        return SX_OK;
    }
    // other shapes: the GEMV, then the pick over the logits
    if (int rc = linear(fn, bits, x, w, logits, 1, SX_ACT_BF16, SX_ACT_F32, stream)) return rc;
    return sx_mtp_pick_ws(logits, w->N, router_err, expert_err, attn_err, emb_err, out, workspace, workspace_bytes,
                          stream);
}

int sx_linear_q4_experts_gather(const void *x, const sx_qview *w, int64_t E, const int32_t *ids, int64_t M, int64_t A,
                                void *y, int act, uint32_t *err, sx_stream stream) {
    const char *fn = "sx_linear_q4_experts_gather";
    if (int rc = experts_common(fn, x, w, E, M, A, y, act)) return rc;
    SX_CHECK(ids != nullptr && err != nullptr, fn, " null pointer (ids=", (const void *)ids, ", err=", (void *)err, ")");
    const int64_t N = w->N / E, es = act_bytes(act);
    SX_CHECK(apart(x, M * w->K * es, y, M * A * N * es), fn, " output overlaps input");
    Params p{};
    p.x = x, p.q = w->q, p.scale = w->scale, p.minv = w->minv, p.y = y, p.ids = ids, p.err = err;
    p.M = M, p.A = A, p.E = E, p.N = N, p.K = w->K, p.G = (int)w->G, p.max_rows = 1;
    return launch_qmm(fn, qmm::SLOT_GATHER, 4, act, act, p, M * A, N, 1, stream_of(stream));
}

int sx_linear_q4_experts_gather_swiglu(const void *x, const sx_qview *w, int64_t E, const int32_t *ids, int64_t M,
                                       int64_t A, void *h, int act, uint32_t *err, sx_stream stream) {
    const char *fn = "sx_linear_q4_experts_gather_swiglu";
    if (int rc = experts_common(fn, x, w, E, M, A, h, act)) return rc;
    SX_CHECK(ids != nullptr && err != nullptr, fn, " null pointer (ids=", (const void *)ids, ", err=", (void *)err, ")");
    const int64_t N = w->N / E, es = act_bytes(act);
    SX_CHECK(N % 2 == 0, fn, " SwiGLU gather needs an even row count per expert ([gate | up]), got ", N);
    SX_CHECK(apart(x, M * w->K * es, h, M * A * (N / 2) * es), fn, " output overlaps input");
    Params p{};
    p.x = x, p.q = w->q, p.scale = w->scale, p.minv = w->minv, p.y = h, p.ids = ids, p.err = err;
    p.M = M, p.A = A, p.E = E, p.N = N, p.K = w->K, p.G = (int)w->G, p.max_rows = 1;
    return launch_qmm(fn, qmm::SLOT_SWIGLU, 4, act, act, p, M * A, N / 2, 1, stream_of(stream));
}

int sx_linear_q4_experts_combine(const void *h, const sx_qview *w, int64_t E, const int32_t *ids, const float *coef,
                                 int64_t M, int64_t A, void *y, int act, uint32_t *err, sx_stream stream) {
    const char *fn = "sx_linear_q4_experts_combine";
    if (int rc = experts_common(fn, h, w, E, M, A, y, act)) return rc;
    SX_CHECK(ids != nullptr && err != nullptr && coef != nullptr, fn, " null pointer (ids=", (const void *)ids,
             ", coef=", (const void *)coef, ", err=", (void *)err, ")");
    const int64_t N = w->N / E, es = act_bytes(act);
    SX_CHECK(apart(h, M * A * w->K * es, y, M * N * es), fn, " output overlaps input");
    const int nsplit = act == SX_ACT_F32 ? 3 : 1;
    SX_CHECK(qmm::lds_bytes(4, nsplit, w->K, w->G, (int)A, (int)A) <= 96 * 1024, fn, " A x K = ", A, " x ", w->K,
             " activation rows exceed the LDS the per-token combine stages");
    Params p{};
    p.x = h, p.q = w->q, p.scale = w->scale, p.minv = w->minv, p.y = y, p.ids = ids, p.coef = coef, p.err = err;
    p.M = M, p.A = A, p.E = E, p.N = N, p.K = w->K, p.G = (int)w->G, p.max_rows = (int)A;
    return launch_qmm(fn, qmm::SLOT_COMBINE, 4, act, act, p, M, N, 1, stream_of(stream));
}

int sx_linear_q4_experts_gather_grouped(const void *x, const sx_qview *w, int64_t E, const void *ws, size_t ws_bytes,
                                        int64_t M, int64_t A, void *y, int act, int math, sx_stream stream) {
    const char *fn = "sx_linear_q4_experts_gather_grouped";
    if (int rc = grouped_common(fn, x, w, E, M, A, ws, ws_bytes, y, act, math)) return rc;
    const int64_t N = w->N / E, es = act_bytes(act), S = M * A;
    SX_CHECK(apart(x, M * w->K * es, y, S * N * es), fn, " y overlaps x");
    if (M >= gg::kPrefillMinTokens && gg::eligible(4, w->G, w->K, act) && aligned(w->scale, 4) && aligned(w->minv, 4)) {
        SX_HIP(gg::launch(qmm::GATHER, x, w, y, static_cast<const int32_t *>(ws), M, A, E, act, stream_of(stream)), fn);
        return SX_OK;
    }
    Params p{};
    p.x = x, p.q = w->q, p.scale = w->scale, p.minv = w->minv, p.y = y, p.ws = static_cast<const int32_t *>(ws);
    p.M = M, p.A = A, p.E = E, p.N = N, p.K = w->K, p.G = (int)w->G;
    p.max_rows = rows_that_fit(4, act == SX_ACT_F32 ? 3 : 1, w->K, w->G, (int)(S < 16 ? S : 16));
    const int64_t units = S < S / 16 + E + 2 ? S : S / 16 + E + 2;  // tiles: at most one a slot
    return launch_qmm(fn, qmm::GATHER, 4, act, act, p, units, N, 1, stream_of(stream));
}

int sx_linear_q4_experts_gather_swiglu_grouped(const void *x, const sx_qview *w, int64_t E, const void *ws,
                                               size_t ws_bytes, int64_t M, int64_t A, void *h, int act,
                                               sx_stream stream) {
    const char *fn = "sx_linear_q4_experts_gather_swiglu_grouped";
    if (int rc = grouped_common(fn, x, w, E, M, A, ws, ws_bytes, h, act, SX_MOE_F32)) return rc;
    const int64_t N = w->N / E, es = act_bytes(act), S = M * A;
    SX_CHECK(N % 2 == 0, fn, " SwiGLU gather needs an even row count per expert ([gate | up]), got ", N);
    SX_CHECK(apart(x, M * w->K * es, h, S * (N / 2) * es), fn, " h overlaps x");
    if (M >= gg::kPrefillMinTokens && gg::eligible(4, w->G, w->K, act) && aligned(w->scale, 4) && aligned(w->minv, 4)) {
        SX_HIP(gg::launch(qmm::SWIGLU, x, w, h, static_cast<const int32_t *>(ws), M, A, E, act, stream_of(stream)), fn);
        return SX_OK;
    }
    Params p{};
    p.x = x, p.q = w->q, p.scale = w->scale, p.minv = w->minv, p.y = h, p.ws = static_cast<const int32_t *>(ws);
    p.M = M, p.A = A, p.E = E, p.N = N, p.K = w->K, p.G = (int)w->G;
    p.max_rows = rows_that_fit(4, act == SX_ACT_F32 ? 3 : 1, w->K, w->G, (int)(S < 16 ? S : 16));
    const int64_t units = S < S / 16 + E + 2 ? S : S / 16 + E + 2;
    return launch_qmm(fn, qmm::SWIGLU, 4, act, act, p, units, N / 2, 1, stream_of(stream));
}

int sx_linear_q4_experts_combine_grouped(const void *h, const sx_qview *w, int64_t E, const int32_t *ids,
                                         const float *coef, const void *ws, size_t ws_bytes, float *partial, int64_t M,
                                         int64_t A, void *y, int act, int math, sx_stream stream) {
    const char *fn = "sx_linear_q4_experts_combine_grouped";
    if (int rc = grouped_common(fn, h, w, E, M, A, ws, ws_bytes, y, act, math)) return rc;
    SX_CHECK(ids != nullptr && coef != nullptr && partial != nullptr, fn, " null pointer (ids=", (const void *)ids,
             ", coef=", (const void *)coef, ", partial=", (void *)partial, ")");
    const int64_t N = w->N / E, es = act_bytes(act), S = M * A;
    SX_CHECK(apart(y, M * N * es, h, S * w->K * es), fn, " y overlaps h");
    SX_CHECK(apart(y, M * N * es, partial, S * N * 4), fn, " y overlaps partial");
    SX_CHECK(apart(partial, S * N * 4, h, S * w->K * es), fn, " partial overlaps h");
    if (M >= gg::kPrefillMinTokens && gg::eligible(4, w->G, w->K, act) && aligned(w->scale, 4) && aligned(w->minv, 4)) {
        SX_HIP(gg::launch(qmm::COMBINE, h, w, partial, static_cast<const int32_t *>(ws), M, A, E, SX_ACT_F32,
                          stream_of(stream)), fn);
        return combine_reduce(partial, ids, coef, M, A, E, N, y, act, stream_of(stream));
    }
    Params p{};
    p.x = h, p.q = w->q, p.scale = w->scale, p.minv = w->minv, p.y = partial, p.ws = static_cast<const int32_t *>(ws);
    p.M = M, p.A = A, p.E = E, p.N = N, p.K = w->K, p.G = (int)w->G;
    p.max_rows = rows_that_fit(4, act == SX_ACT_F32 ? 3 : 1, w->K, w->G, (int)(S < 16 ? S : 16));
    const int64_t units = S < S / 16 + E + 2 ? S : S / 16 + E + 2;
    if (int rc = launch_qmm(fn, qmm::COMBINE, 4, act, act, p, units, N, 1, stream_of(stream))) return rc;
    return combine_reduce(partial, ids, coef, M, A, E, N, y, act, stream_of(stream));
}

}  // extern "C"
