// Route grouping (moe_group_routes), the grouped combine's reduction, SwiGLU, the shared-expert add, and the C-ABI's
// error channel.
#include "common.hpp"
#include "route_impl.hpp"

#include <climits>
#include <mutex>
#include <vector>

namespace sx {

// ---------------- error channel ----------------

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string &msg) { g_last_error = msg; }

int device_cus() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

namespace {

// ---------------- moe_group_routes ----------------
// Workspace layout (int32), the contract of kernels/moe_grouped.hip:63-81: header [n_tiles, S, E, n_wtiles],
// offsets [E + 2] (bucket b's slots at slots[offsets[b] .. offsets[b + 1]); bucket E = invalid ids), slots [S],
// tile_bucket [Tmax], tile_start [Tmax] (16-slot tiles), wtile_bucket [WTmax], wtile_start [WTmax] (64-slot tiles);
// Tmax = S / 16 + E + 2, WTmax = S / 64 + E + 2 (a bucket of c slots has ceil(c / R) <= c / R + 1 tiles).
constexpr int kRouteThreads = 1024;  // one bucket a thread: E <= 1023 experts + the invalid-id bucket
constexpr int kRouteStage = 32768;   // slots placed in LDS (128 KB) before they go out in order

__global__ void __launch_bounds__(kRouteThreads)
    route_kernel(const int32_t *ids, int S, int E, int Tmax, int WTmax, int32_t *ws, uint32_t *err) {
    __shared__ int cnt[kRouteThreads], cursor[kRouteThreads];
    __shared__ int wtot[kRouteThreads / 64][3];
    __shared__ int first_bad;
    __shared__ int stage[kRouteStage];
    routing::group_in_block<kRouteThreads>([&](int s) { return ids[s]; }, S, E, Tmax, WTmax, ws, err, cnt, cursor,
                                           wtot, &first_bad, stage, kRouteStage);
}

// ---------------- combine reduce ----------------

template <typename T>
__global__ void __launch_bounds__(256) combine_reduce_kernel(const float *partial, const int32_t *ids, const float *coef,
                                                             int64_t M, int64_t A, int64_t E, int64_t N, T *y) {
    const int64_t total = M * N;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = i / N, n = i % N;
        bool ok = true;
        float v = 0.f;
        for (int64_t a = 0; a < A; ++a) {
            const int32_t id = ids[m * A + a];
            ok = ok && id >= 0 && id < E;
            v = fmaf(coef[m * A + a], partial[(m * A + a) * N + n], v);
        }
        store_act(y, i, ok ? v : qnan());
    }
}

// The same sums four outputs a thread (N a multiple of 4, 16-byte aligned partials): a block row is one token, the
// A partial rows' float4 loads go out eight at a time before their FMAs, which run in slot order as above (the
// same value bit for bit), and no 64-bit division a value.
template <typename T>
__global__ void __launch_bounds__(256) combine_reduce4_kernel(const float *partial, const int32_t *ids,
                                                              const float *coef, int64_t A, int64_t E, int64_t N,
                                                              T *y) {
    constexpr int kBatch = 8;
    const int64_t m = blockIdx.y;
    const int64_t n = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (n >= N) return;
    const float *prow = partial + m * A * N + n;
    bool ok = true;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t a0 = 0; a0 < A; a0 += kBatch) {
        float4 pv[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {  // clamped: rows past A load row A - 1 and are not used
            const int64_t a = a0 + b < A ? a0 + b : A - 1;
            pv[b] = *reinterpret_cast<const float4 *>(prow + a * N);
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            if (a0 + b >= A) break;
            const int32_t id = ids[m * A + a0 + b];
            ok = ok && id >= 0 && id < E;
            const float c = coef[m * A + a0 + b];
            v[0] = fmaf(c, pv[b].x, v[0]), v[1] = fmaf(c, pv[b].y, v[1]);
            v[2] = fmaf(c, pv[b].z, v[2]), v[3] = fmaf(c, pv[b].w, v[3]);
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) store_act(y, m * N + n + j, ok ? v[j] : qnan());
}

// ---------------- swiglu ----------------

template <typename T>
__global__ void __launch_bounds__(256) swiglu_kernel(const T *gu, T *h, int64_t rows, int64_t I) {
    const int64_t n = rows * I;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / I, j = i % I;
        const float g = load_act(gu, r * 2 * I + j), u = load_act(gu, r * 2 * I + I + j);
        store_act(h, i, as_stored(silu(g), h) * u);  // BF16: bf16(bf16(silu(g)) * u), kernels/swiglu.hip:31-36
    }
}

// ---------------- shared-expert add (+ residual injection) ----------------

template <typename T, bool INJECT>
__global__ void __launch_bounds__(256) shared_add_kernel(T *y, const T *s, const float *gate_logit, int64_t gate_ld,
                                                         int64_t N, uint32_t gate_index, T *x, const float *w_in,
                                                         uint32_t *err) {
    constexpr int kStreams = 4;
    const int64_t m = blockIdx.y;
    const float gl = gate_logit[m * gate_ld];
    const bool ok = isfinite(gl);
    if (!ok && blockIdx.x == 0 && threadIdx.x == 0) flag_error(err, (uint32_t)m, gate_index);
    const float gate = ok ? 1.f / (1.f + expf(-gl)) : qnan();
    const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    const float v = as_stored(load_act(y, m * N + n) + gate * load_act(s, m * N + n), y);
    store_act(y, m * N + n, v);
    if constexpr (INJECT) {
#pragma unroll
        for (int st = 0; st < kStreams; ++st) {
            const int64_t xi = m * kStreams * N + st * N + n;
            store_act(x, xi, fmaf(w_in[m * kStreams + st], v, load_act(x, xi)));
        }
    }
}

int grid_for(int64_t n, int64_t cap = 65535ll * 16) {
    const int64_t b = (n + 255) / 256;
    return (int)(b < cap ? (b < 1 ? 1 : b) : cap);
}

}  // namespace

Layout layout_of(int64_t M, int64_t A, int64_t E) {
    const int64_t S = M * A;
    return {S, E, S / routing::kR + E + 2, S / routing::kRW + E + 2};
}

int combine_reduce(const float *partial, const int32_t *ids, const float *coef, int64_t M, int64_t A, int64_t E,
                   int64_t N, void *y, int act, hipStream_t stream) {
    if (N % 4 == 0 && aligned(partial, 16) && (N / 4 + 255) / 256 <= 0x7fffffff && M <= 65535) {
        const dim3 grid((unsigned)((N / 4 + 255) / 256), (unsigned)M);
        if (act == SX_ACT_F32)
            combine_reduce4_kernel<float><<<grid, 256, 0, stream>>>(partial, ids, coef, A, E, N, static_cast<float *>(y));
        else
            combine_reduce4_kernel<uint16_t><<<grid, 256, 0, stream>>>(partial, ids, coef, A, E, N,
                                                                       static_cast<uint16_t *>(y));
        SX_LAUNCHED("combine_reduce M=", M, " A=", A, " N=", N);
        return SX_OK;
    }
    const int blocks = grid_for(M * N, 8192);
    if (act == SX_ACT_F32)
        combine_reduce_kernel<float><<<blocks, 256, 0, stream>>>(partial, ids, coef, M, A, E, N, static_cast<float *>(y));
    else
        combine_reduce_kernel<uint16_t><<<blocks, 256, 0, stream>>>(partial, ids, coef, M, A, E, N,
                                                                    static_cast<uint16_t *>(y));
    SX_LAUNCHED("combine_reduce M=", M, " A=", A, " N=", N);
    return SX_OK;
}

}  // namespace sx

using namespace sx;

extern "C" {

const char *sx_last_error(void) { return g_last_error.c_str(); }
const char *sx_version(void) { return "strixite_amd 0.1 gfx950"; }

int sx_report_expert_error(const uint32_t e[3], const char *what) {
    SX_CHECK(e != nullptr, "null error words");
    SX_CHECK(e[0] == 0, what ? what : "experts", ": expert id ", (int32_t)e[1], " at slot ", e[2],
             " (token * A + a) is out of range; outputs for that token are NaN");
    return SX_OK;
}

int sx_report_router_error(const uint32_t e[3], const char *what) {
    SX_CHECK(e != nullptr, "null error words");
    SX_CHECK(e[0] == 0, what ? what : "router", ": non-finite router logit at token ", e[1], ", expert ", e[2],
             " (E = the shared-expert gate); that token's ids are -1 and its coefficients NaN");
    return SX_OK;
}

int sx_moe_route_workspace_bytes(int64_t M, int64_t A, int64_t E, size_t *bytes) {
    SX_CHECK(bytes != nullptr, "null output");
    SX_CHECK(M >= 1 && A >= 1 && E >= 1 && E <= 1023 && M * A <= (1 << 20), "M = ", M, ", A = ", A, ", E = ", E,
             " (E <= 1023, M*A <= 2^20)");
    *bytes = (size_t)layout_of(M, A, E).ints() * 4;
    return SX_OK;
}

int sx_moe_group_routes(const int32_t *ids, int64_t M, int64_t A, int64_t E, void *ws, size_t ws_bytes, uint32_t *err,
                        sx_stream stream) {
    SX_CHECK(ids != nullptr && ws != nullptr && err != nullptr, "null pointer (ids=", (const void *)ids, ", ws=", ws,
             ", err=", (void *)err, ")");
    SX_CHECK(M >= 1 && A >= 1 && A <= 64 && E >= 1 && E <= 1023 && M * A <= (1 << 20), "M = ", M, ", A = ", A,
             ", E = ", E, " (A 1..64, E 1..1023, M*A <= 2^20)");
    const Layout L = layout_of(M, A, E);
    SX_CHECK(ws_bytes >= (size_t)L.ints() * 4, "workspace of ", ws_bytes, " bytes, needs ", L.ints() * 4);
    SX_CHECK(aligned(ws, 4), "workspace must be 4-byte aligned");
    route_kernel<<<1, kRouteThreads, 0, stream_of(stream)>>>(ids, (int)L.S, (int)E, (int)L.Tmax, (int)L.WTmax,
                                                              static_cast<int32_t *>(ws), err);
    SX_LAUNCHED("moe_group_routes M=", M, " A=", A, " E=", E);
    return SX_OK;
}

int sx_swiglu(const void *gu, void *h, int64_t rows, int64_t I, int act, sx_stream stream) {
    SX_CHECK(gu != nullptr && h != nullptr, "null pointer (gu=", gu, ", h=", h, ")");
    SX_CHECK(rows >= 1 && I >= 1, "rows = ", rows, ", I = ", I, ", both must be >= 1");
    SX_CHECK(rows <= (1ll << 40) / I / 2, "rows * 2I = ", rows, " * ", 2 * I, " too large (rows/I swapped?)");
    SX_CHECK(act == SX_ACT_F32 || act == SX_ACT_BF16, "unsupported activation dtype ", act);
    const int64_t es = act_bytes(act), n = rows * I;
    SX_CHECK(apart(h, n * es, gu, 2 * n * es), "output h [", h, ", +", n * es, " B) overlaps input gu [", gu, ", +",
             2 * n * es, " B)");
    const int blocks = grid_for(n);
    if (act == SX_ACT_F32)
        swiglu_kernel<float><<<blocks, 256, 0, stream_of(stream)>>>(static_cast<const float *>(gu),
                                                                     static_cast<float *>(h), rows, I);
    else
        swiglu_kernel<uint16_t><<<blocks, 256, 0, stream_of(stream)>>>(static_cast<const uint16_t *>(gu),
                                                                        static_cast<uint16_t *>(h), rows, I);
    SX_LAUNCHED("swiglu rows=", rows, " I=", I);
    return SX_OK;
}

int sx_moe_shared_add(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                      uint32_t gate_index, int act, uint32_t *err, sx_stream stream) {
    SX_CHECK(y && s && gate_logit && err, "null pointer (y=", y, ", s=", s, ", gate_logit=", (const void *)gate_logit,
             ", err=", (void *)err, ")");
    SX_CHECK(M >= 1 && M <= 65535, "M = ", M, " tokens, expected 1..65535");
    SX_CHECK(N >= 1 && N <= (1ll << 24), "N = ", N, ", expected 1..2^24");
    SX_CHECK(gate_ld >= 1, "gate_ld = ", gate_ld, ", expected >= 1");
    SX_CHECK(act == SX_ACT_F32 || act == SX_ACT_BF16, "unsupported activation dtype ", act);
    const int64_t bytes = M * N * act_bytes(act);
    SX_CHECK(apart(y, bytes, s, bytes), "s overlaps y");
    const dim3 grid((unsigned)((N + 255) / 256), (unsigned)M);
    if (act == SX_ACT_F32)
        shared_add_kernel<float, false><<<grid, 256, 0, stream_of(stream)>>>(
            static_cast<float *>(y), static_cast<const float *>(s), gate_logit, gate_ld, N, gate_index, nullptr,
            nullptr, err);
    else
        shared_add_kernel<uint16_t, false><<<grid, 256, 0, stream_of(stream)>>>(
            static_cast<uint16_t *>(y), static_cast<const uint16_t *>(s), gate_logit, gate_ld, N, gate_index, nullptr,
            nullptr, err);
    SX_LAUNCHED("moe_shared_add M=", M, " N=", N);
    return SX_OK;
}

int sx_moe_shared_add_inject(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                             uint32_t gate_index, void *x, const float *w_in, int64_t H, int act, uint32_t *err,
                             sx_stream stream) {
    SX_CHECK(y && s && gate_logit && err && x && w_in, "null pointer");
    SX_CHECK(M >= 1 && M <= 65535, "M = ", M, " tokens, expected 1..65535");
    SX_CHECK(N >= 1 && N <= (1ll << 24), "N = ", N, ", expected 1..2^24");
    SX_CHECK(H == 4, "H = ", H, " streams, expected 4 (qwen4_exp's hc_count)");
    SX_CHECK(gate_ld >= 1, "gate_ld = ", gate_ld, ", expected >= 1");
    SX_CHECK(act == SX_ACT_F32 || act == SX_ACT_BF16, "unsupported activation dtype ", act);
    const int64_t es = act_bytes(act), yb = M * N * es, xb = M * H * N * es;
    SX_CHECK(apart(y, yb, s, yb), "s overlaps y");
    SX_CHECK(apart(x, xb, y, yb) && apart(x, xb, s, yb), "x overlaps y or s");
    const dim3 grid((unsigned)((N + 255) / 256), (unsigned)M);
    if (act == SX_ACT_F32)
        shared_add_kernel<float, true><<<grid, 256, 0, stream_of(stream)>>>(
            static_cast<float *>(y), static_cast<const float *>(s), gate_logit, gate_ld, N, gate_index,
            static_cast<float *>(x), w_in, err);
    else
        shared_add_kernel<uint16_t, true><<<grid, 256, 0, stream_of(stream)>>>(
            static_cast<uint16_t *>(y), static_cast<const uint16_t *>(s), gate_logit, gate_ld, N, gate_index,
            static_cast<uint16_t *>(x), w_in, err);
    SX_LAUNCHED("moe_shared_add_inject M=", M, " N=", N);
    return SX_OK;
}

}  // extern "C"
