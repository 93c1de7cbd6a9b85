// C-ABI entry points of the dequantizing GEMMs: dense linear (q4 / q8) and the per-slot and grouped MoE experts.
// Host-side preconditions follow the reference launchers (kernels/linear_q4.hip:353-440, linear_q8.hip:192-223,
// moe_grouped.hip:476-556); the work runs in qmm_impl.hpp.
#include "common.hpp"
#include <algorithm>
#include <vector>
#include <cstdio>
#include <map>
#include "gemm_grouped.hpp"
#include "qmm.hpp"

#include <cstdlib>

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
    if (const char *e = getenv("SX_TPW")) tpw = atoi(e);  // TEMP
    return (int)(tpw * qmm::kWaves);
}

int launch_qmm(const char *fn, int mode, int bits, int act_x, int act_y, Params &p, int64_t units, int64_t rows_out,
               int64_t grid_y, hipStream_t stream) {
    if (const char *e = getenv("SX_DBG")) p.dbg = atoi(e);
    const int64_t tiles = (rows_out + qmm::kTile - 1) / qmm::kTile;
    p.tiles_per_chunk = tiles_per_chunk(tiles * units);
    p.nchunks = (int)((tiles + p.tiles_per_chunk - 1) / p.tiles_per_chunk);
    const int64_t gx = units * p.nchunks;
    SX_CHECK(gx >= 1 && gx <= 0x7fffffff && grid_y <= 65535, fn, " grid ", gx, " x ", grid_y, " out of range");
    static int tr_n = 0;  // TEMP trace
    const char *te = getenv("SX_TRACE");
    unsigned long long *tb = nullptr;
    const size_t nw = (size_t)gx * grid_y * qmm::kWaves;
    if (te && (tr_n++ % 5) == 4) {
        hipMalloc(&tb, nw * 128);
        hipMemset(tb, 0, nw * 128);
        p.trace = tb;
    }
    SX_HIP(qmm::launch(mode, bits, act_x, act_y, p, dim3((unsigned)gx, (unsigned)grid_y), stream), fn);
    if (tb) {
        hipDeviceSynchronize();
        std::vector<unsigned long long> h(nw * 16);
        hipMemcpy(h.data(), tb, nw * 128, hipMemcpyDeviceToHost);
        hipFree(tb);
        unsigned long long t0 = ~0ull, tend = 0;
        double d[5] = {0, 0, 0, 0, 0};
        int n = 0;
        std::vector<double> starts, ends;
        double e5 = 0, e6 = 0, e7 = 0;
        for (size_t w = 0; w < nw; ++w) {
            const unsigned long long *r = &h[w * 16];
            if (!r[0] || !r[4]) continue;
            if (r[5] && r[6] && r[7]) e7 += (double)(r[7] - r[1]), e5 += (double)(r[5] - r[1]), e6 += (double)(r[6] - r[1]);
            t0 = std::min(t0, r[0]);
            tend = std::max(tend, r[4]);
            for (int i = 1; i < 5; ++i) d[i] += (double)(r[i] - r[i - 1]);
            ++n;
        }
        for (size_t w = 0; w < nw; ++w) {
            const unsigned long long *r = &h[w * 16];
            if (!r[0] || !r[4]) continue;
            starts.push_back((r[0] - t0) * 0.01), ends.push_back((r[4] - t0) * 0.01);
        }
        double intra = 0;
        int nb = 0;
        for (size_t b = 0; b + 4 <= nw; b += 4) {
            unsigned long long lo = ~0ull, hi = 0;
            for (int w = 0; w < 4; ++w)
                if (h[(b + w) * 16 + 4]) lo = std::min(lo, h[(b + w) * 16 + 4]), hi = std::max(hi, h[(b + w) * 16 + 4]);
            if (hi) intra += (double)(hi - lo), ++nb;
        }
        {  // end time by the number of this kernel's blocks on the block's CU
            std::map<unsigned long long, int> per_cu;
            for (size_t b = 0; b < nw; b += 4) if (h[b * 16 + 4]) per_cu[(h[b * 16 + 9] << 32) | ((h[b * 16 + 8] >> 8) & 0xFF)]++;
            std::map<int, std::pair<double, int>> by;
            for (size_t b = 0; b < nw; b += 4) {
                if (!h[b * 16 + 4]) continue;
                const int c = per_cu[(h[b * 16 + 9] << 32) | ((h[b * 16 + 8] >> 8) & 0xFF)];
                by[c].first += (h[b * 16 + 4] - t0) * 0.01, by[c].second++;
            }
            std::map<int, std::pair<double, int>> byx, byse;
            for (size_t b = 0; b < nw; b += 4) {
                if (!h[b * 16 + 4]) continue;
                const int xcc = (int)(h[b * 16 + 9] & 0xF), se = (int)((h[b * 16 + 8] >> 13) & 0x7);
                const double e = (h[b * 16 + 4] - t0) * 0.01;
                byx[xcc].first += e, byx[xcc].second++;
                byse[xcc * 8 + se].first += e, byse[xcc * 8 + se].second++;
            }
            fprintf(stderr, "  by XCC:");
            for (auto &kv : byx) fprintf(stderr, " x%d %d blk %.1f;", kv.first, kv.second.second, kv.second.first / kv.second.second);
            fprintf(stderr, "\n  by XCC.SE:");
            for (auto &kv : byse) fprintf(stderr, " %d.%d:%d/%.1f", kv.first / 8, kv.first % 8, kv.second.second, kv.second.first / kv.second.second);
            fprintf(stderr, "\n");
            fprintf(stderr, "  CUs used %zu;", per_cu.size());
            for (auto &kv : by) fprintf(stderr, " %d blocks/CU: %d blocks, mean end %.2f us;", kv.first, kv.second.second, kv.second.first / kv.second.second);
            fprintf(stderr, "\n");
        }
        fprintf(stderr, "  mean spread of wave end times within a block: %.2f us\n", nb ? intra / nb * 0.01 : 0.0);
        std::sort(starts.begin(), starts.end());
        std::sort(ends.begin(), ends.end());
        auto q = [](std::vector<double> &v, double f) { return v.empty() ? 0.0 : v[(size_t)(f * (v.size() - 1))]; };
        fprintf(stderr, "  stage detail (from decode end): x issued+pre-prime %.2f, first chunk written %.2f, all written %.2f\n", e7 / nw * 0.01, e5 / nw * 0.01, e6 / nw * 0.01);
        fprintf(stderr, "TRACE %s waves=%d/%zu span=%.2fus decode=%.2f stage=%.2f first_group=%.2f rest=%.2f | start q50=%.2f q90=%.2f max=%.2f | end q10=%.2f q50=%.2f q90=%.2f max=%.2f\n",
                fn, n, nw, (tend - t0) * 0.01, d[1] / n * 0.01, d[2] / n * 0.01, d[3] / n * 0.01, d[4] / n * 0.01,
                q(starts, .5), q(starts, .9), q(starts, 1), q(ends, .1), q(ends, .5), q(ends, .9), q(ends, 1));
    }
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
