// MoE routing on gfx950: the router projection (FP32 weights) and the top-k router (kernels/moe_router.hpp:11-40).
#include "common.hpp"

#include <climits>

namespace sx {
namespace {

// ---------------- router projection: y[M, N] = x[M, K] . W[N, K]^T, FP32 weights ----------------
// The router weight (E x d FP32, 8 MB at E = 512, d = 4096) is read once; it is the whole cost. A block takes kF32wRows
// weight rows and NT tokens; each thread owns every 256th float4 column of those rows, issues all of its weight loads
// before it uses any (K = 4096: 4 float4 a row in flight a thread), and reads the tokens' x values straight from
// L2 (x is a few KB a token). Per (row, token) the thread's partial sum goes through a wave butterfly and the four
// waves' sums through LDS. Further tokens run in further grid rows.
constexpr int kF32wTokens = 8, kF32wRows = 2, kF32wUnroll = 4;

template <typename TX>
__device__ __forceinline__ float4 load4(const TX *p) {
    if constexpr (sizeof(TX) == 4) {
        return *reinterpret_cast<const float4 *>(p);
    } else {
        const uint2 u = *reinterpret_cast<const uint2 *>(p);
        return float4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xFFFF0000u), __uint_as_float(u.y << 16),
                      __uint_as_float(u.y & 0xFFFF0000u)};
    }
}

template <typename TX, int NT>
__global__ void __launch_bounds__(256) linear_f32w_kernel(const TX *x, const float *W, float *y, int64_t M, int64_t N,
                                                          int64_t K) {
    __shared__ float part[4][kF32wRows * NT];
    const int64_t m0 = (int64_t)blockIdx.y * NT, n0 = (int64_t)blockIdx.x * kF32wRows;
    const int T = (int)min((int64_t)NT, M - m0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t K4 = K / 4;
    const float4 *wr[kF32wRows];
#pragma unroll
    for (int r = 0; r < kF32wRows; ++r) wr[r] = reinterpret_cast<const float4 *>(W + min(n0 + r, N - 1) * K);
    float acc[kF32wRows][NT];
#pragma unroll
    for (int r = 0; r < kF32wRows; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[r][t] = 0.f;
    // Every load is unconditional (clamped column and token, the weight zeroed past K) so that none waits for another.
    const TX *xt[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) xt[t] = x + (m0 + min(t, T - 1)) * K;
    for (int64_t base = 0; base < K4; base += 256 * kF32wUnroll) {
        float4 w[kF32wUnroll][kF32wRows], xv[kF32wUnroll][NT];
#pragma unroll
        for (int u = 0; u < kF32wUnroll; ++u) {
            const int64_t k4 = min(base + u * 256 + tid, K4 - 1);
#pragma unroll
            for (int r = 0; r < kF32wRows; ++r) w[u][r] = wr[r][k4];
#pragma unroll
            for (int t = 0; t < NT; ++t) xv[u][t] = load4(xt[t] + 4 * k4);
        }
        __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the first use
#pragma unroll
        for (int u = 0; u < kF32wUnroll; ++u) {
            const float on = base + u * 256 + tid < K4 ? 1.f : 0.f;
#pragma unroll
            for (int r = 0; r < kF32wRows; ++r) {
                const float4 wv = float4{w[u][r].x * on, w[u][r].y * on, w[u][r].z * on, w[u][r].w * on};
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    acc[r][t] = fmaf(wv.x, xv[u][t].x, fmaf(wv.y, xv[u][t].y,
                                     fmaf(wv.z, xv[u][t].z, fmaf(wv.w, xv[u][t].w, acc[r][t]))));
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kF32wRows; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float v = acc[r][t];
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
            if (lane == 0) part[wave][r * NT + t] = v;
        }
    __syncthreads();
    if (tid < kF32wRows * NT) {
        const int r = tid / NT, t = tid % NT;
        if (t < T && n0 + r < N) y[(m0 + t) * N + n0 + r] = part[0][tid] + part[1][tid] + part[2][tid] + part[3][tid];
    }
}

// ---------------- top-k router ----------------
// One wave64 per token. The E logits stay in registers (lane l holds experts l, l + 64, ...); a pick is a wave-wide
// maximum of 64-bit keys (value bits made monotone in the high word, ~index in the low word), so the larger logit
// wins and a tie goes to the lower index (kernels/moe_router.hpp:11-13) with one integer compare. Only the lane whose
// expert was picked rescans its registers. Then the softmax over the k picks.
__device__ __forceinline__ uint64_t route_key(float v, int idx) {
    const uint32_t b = v == 0.f ? 0u : __float_as_uint(v);  // -0 ties +0, as a float compare does
    const uint32_t hi = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)hi << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)idx);
}

// The logit a key was made from (a -0 logit comes back as +0, which no later use tells apart).
__device__ __forceinline__ float key_value(uint64_t key) {
    const uint32_t hi = (uint32_t)(key >> 32);
    return __uint_as_float((hi & 0x80000000u) ? (hi & 0x7FFFFFFFu) : ~hi);
}

// Wave-wide maximum of 64-bit keys. Within a row of 16 lanes the partners come through DPP (quad [1,0,3,2],
// quad [2,3,0,1], half-row mirror, row mirror: after each step every lane holds the maximum over 2, 4, 8, 16 lanes,
// since max needs no particular pairing); across the four rows two LDS-routed shuffles.
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_max(uint64_t k) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)k, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(k >> 32), CTRL, 0xF, 0xF, false);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    return o > k ? o : k;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
    k = dpp_max<0xB1>(k);   // quad_perm [1,0,3,2]
    k = dpp_max<0x4E>(k);   // quad_perm [2,3,0,1]
    k = dpp_max<0x141>(k);  // row_half_mirror
    k = dpp_max<0x140>(k);  // row_mirror
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)k, off), hi = __shfl_xor((uint32_t)(k >> 32), off);
        const uint64_t o = ((uint64_t)hi << 32) | lo;
        k = o > k ? o : k;
    }
    return k;
}

template <typename T, int NV>
__global__ void __launch_bounds__(64) moe_router_kernel(const T *logits, int64_t ld, int E, int k, const T *shared,
                                                        int64_t shared_ld, int32_t shared_id, int32_t *ids,
                                                        float *coef, int A, uint32_t *err) {
    const int64_t m = blockIdx.x;
    const int lane = threadIdx.x;
    const T *row = logits + m * ld;
    float v[NV];
    int bad = INT_MAX;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = lane + 64 * j;
        const float xv = e < E ? load_act(row, e) : -INFINITY;
        v[j] = xv;
        if (e < E && !isfinite(xv) && e < bad) bad = e;
    }
    float sl = 0.f;
    if (shared != nullptr) {
        sl = load_act(shared, m * shared_ld);
        if (!isfinite(sl) && E < bad) bad = E;
    }
    for (int off = 32; off > 0; off >>= 1) bad = min(bad, __shfl_xor(bad, off));
    int32_t *id_row = ids + m * A;
    float *coef_row = coef + m * A;
    if (bad != INT_MAX) {  // a non-finite logit fails the token (moe_router.hpp:19-23)
        if (lane == 0) flag_error(err, (uint32_t)m, (uint32_t)bad);
        for (int a = lane; a < A; a += 64) id_row[a] = -1, coef_row[a] = qnan();
        return;
    }
    // Padding past E must never win: its key is below every finite logit's.
    auto lane_best = [&]() {
        uint64_t b = 0;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int e = lane + 64 * j;
            const uint64_t key = e < E ? route_key(v[j], e) : 0;
            b = key > b ? key : b;
        }
        return b;
    };
    uint64_t mine = lane_best();
    float my_v = -INFINITY, top = 0.f;
    int my_i = -1;
    for (int r = 0; r < k; ++r) {
        const uint64_t best = wave_max_u64(mine);
        const int bi = (int)(0xFFFFFFFFu - (uint32_t)best);
        const float bv = key_value(best);
        if (r == 0) top = bv;
        if (lane == r) my_v = bv, my_i = bi;
        if ((bi & 63) == lane) {  // the picked expert is this lane's
#pragma unroll
            for (int j = 0; j < NV; ++j)
                if (lane + 64 * j == bi) v[j] = -INFINITY;
            mine = 0;
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int e = lane + 64 * j;
                if (e < E && v[j] != -INFINITY) {
                    const uint64_t key = route_key(v[j], e);
                    mine = key > mine ? key : mine;
                }
            }
        }
    }
    const float ex = lane < k ? expf(my_v - top) : 0.f;
    float sum = ex;
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    if (lane < k) id_row[lane] = my_i, coef_row[lane] = ex / sum;
    if (shared != nullptr && lane == 0) id_row[k] = shared_id, coef_row[k] = 1.0f / (1.0f + expf(-sl));
}

}  // namespace
}  // namespace sx

using namespace sx;

extern "C" {

int sx_linear_f32w(const void *x, const float *W, int64_t N, int64_t K, float *y, int64_t M, int act,
                   sx_stream stream) {
    SX_CHECK(x != nullptr && W != nullptr && y != nullptr, "null pointer");
    SX_CHECK(N >= 1 && K >= 4 && K % 4 == 0 && M >= 1, "N = ", N, ", K = ", K, " (a positive multiple of 4), M = ", M);
    SX_CHECK(aligned(W, 16) && aligned(x, 8), "W must be 16-byte and x 8-byte aligned");
    SX_CHECK(act == SX_ACT_F32 || act == SX_ACT_BF16, "unsupported activation dtype ", act);
    SX_CHECK((M + kF32wTokens - 1) / kF32wTokens <= 65535, "M = ", M, " too large");
    SX_CHECK((N + kF32wRows - 1) / kF32wRows <= 0x7fffffff, "N = ", N, " too large");
    SX_CHECK(apart(y, M * N * 4, x, M * K * act_bytes(act)) && apart(y, M * N * 4, W, N * K * 4), "y overlaps inputs");
    const dim3 grid((unsigned)((N + kF32wRows - 1) / kF32wRows), (unsigned)((M + kF32wTokens - 1) / kF32wTokens));
    if (act == SX_ACT_F32)
        linear_f32w_kernel<float, kF32wTokens><<<grid, 256, 0, stream_of(stream)>>>(static_cast<const float *>(x), W, y,
                                                                                   M, N, K);
    else
        linear_f32w_kernel<uint16_t, kF32wTokens><<<grid, 256, 0, stream_of(stream)>>>(
            static_cast<const uint16_t *>(x), W, y, M, N, K);
    SX_LAUNCHED("linear_f32w M=", M, " N=", N, " K=", K);
    return SX_OK;
}

int sx_moe_router(const void *logits, int64_t ld, int64_t M, int64_t E, int64_t k, const void *shared_logit,
                  int64_t shared_ld, int32_t shared_id, int32_t *ids, float *coef, int act, uint32_t *err,
                  sx_stream stream) {
    SX_CHECK(logits != nullptr && ids != nullptr && coef != nullptr && err != nullptr, "null pointer (logits=", logits,
             ", ids=", (const void *)ids, ", coef=", (const void *)coef, ", err=", (void *)err, ")");
    SX_CHECK(M >= 1 && M <= 0x7fffffff, "M = ", M, " tokens, expected 1..", 0x7fffffff);
    SX_CHECK(E >= 1 && E <= 1024, "E = ", E, " experts, expected 1..1024");
    SX_CHECK(k >= 1 && k <= E && k <= 32, "k = ", k, ", expected 1..min(E = ", E, ", 32)");
    SX_CHECK(ld >= E, "logits row stride ld = ", ld, " < E = ", E);
    if (shared_logit != nullptr) {
        SX_CHECK(shared_ld >= 1, "shared_ld = ", shared_ld, ", expected >= 1");
        SX_CHECK(shared_id >= 0, "shared_id = ", shared_id, ", expected >= 0 (its expert row block)");
    }
    SX_CHECK((const void *)ids != (const void *)coef, "ids and coef are the same buffer");
    SX_CHECK(act == SX_ACT_F32 || act == SX_ACT_BF16, "unsupported activation dtype ", act);
    const int A = (int)k + (shared_logit != nullptr ? 1 : 0);
    const int nv = E <= 256 ? 4 : E <= 512 ? 8 : 16;
    auto go = [&](auto tag, auto nvc) {
        using T = decltype(tag);
        moe_router_kernel<T, decltype(nvc)::value><<<(unsigned)M, 64, 0, stream_of(stream)>>>(
            static_cast<const T *>(logits), ld, (int)E, (int)k, static_cast<const T *>(shared_logit), shared_ld,
            shared_id, ids, coef, A, err);
    };
    auto by_nv = [&](auto tag) {
        if (nv == 4) go(tag, std::integral_constant<int, 4>{});
        else if (nv == 8) go(tag, std::integral_constant<int, 8>{});
        else go(tag, std::integral_constant<int, 16>{});
    };
    if (act == SX_ACT_F32) by_nv(float{});
    else by_nv(uint16_t{});
    SX_LAUNCHED("moe_router M=", M, " E=", E, " k=", k);
    return SX_OK;
}

}  // extern "C"
