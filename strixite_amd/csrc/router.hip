// MoE routing on gfx950: the router projection (FP32 weights) and the top-k router (kernels/moe_router.hpp:11-40).
#include "common.hpp"

#include <climits>

namespace sx {
namespace {

// ---------------- router projection: y[M, N] = x[M, K] . W[N, K]^T, FP32 weights ----------------
// A wave per output row n, 4 rows a block; the block's x rows (8 BF16 or 4 FP32 tokens) are staged in LDS. Each lane
// walks the row in float4 steps (coalesced 1 KB per wave step) and keeps one FP32 accumulator per token; the wave
// reduction at the end is a butterfly. Further tokens run in further grid rows.
constexpr int kF32wTokens = 8;

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

// x rows are staged in LDS in their own dtype (BF16: 8 tokens x K = 4096 in 64 KB).
template <typename TX, int NT>
__global__ void __launch_bounds__(256) linear_f32w_kernel(const TX *x, const float *W, float *y, int64_t M, int64_t N,
                                                          int64_t K) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
    TX *xs = reinterpret_cast<TX *>(smem_raw);  // [tokens][K]
    const int64_t m0 = (int64_t)blockIdx.y * NT;
    const int T = (int)min((int64_t)NT, M - m0);
    for (int64_t i = threadIdx.x; i < (int64_t)T * K; i += blockDim.x) xs[i] = x[m0 * K + i];
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t n = (int64_t)blockIdx.x * 4 + wave;
    if (n >= N) return;  // after the only barrier
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.f;
    const float4 *wr = reinterpret_cast<const float4 *>(W + n * K);
    for (int64_t k4 = lane; k4 < K / 4; k4 += 64) {
        const float4 w = wr[k4];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t < T) {
                const float4 xv = load4(xs + (int64_t)t * K + 4 * k4);
                acc[t] = fmaf(w.x, xv.x, fmaf(w.y, xv.y, fmaf(w.z, xv.z, fmaf(w.w, xv.w, acc[t]))));
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
        for (int off = 32; off > 0; off >>= 1) acc[t] += __shfl_xor(acc[t], off);
    if (lane == 0)
        for (int t = 0; t < T; ++t) y[(m0 + t) * N + n] = acc[t];
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

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
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
        const float bv = load_act(row, bi);
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
    const int nt = act == SX_ACT_F32 ? kF32wTokens / 2 : kF32wTokens;
    const size_t lds = (size_t)nt * K * act_bytes(act);
    SX_CHECK(lds <= 64 * 1024, "K = ", K, " too long for the LDS-staged projection");
    SX_CHECK((M + nt - 1) / nt <= 65535, "M = ", M, " too large");
    SX_CHECK(apart(y, M * N * 4, x, M * K * act_bytes(act)) && apart(y, M * N * 4, W, N * K * 4), "y overlaps inputs");
    const dim3 grid((unsigned)((N + 3) / 4), (unsigned)((M + nt - 1) / nt));
    if (act == SX_ACT_F32)
        linear_f32w_kernel<float, kF32wTokens / 2><<<grid, 256, lds, stream_of(stream)>>>(static_cast<const float *>(x), W,
                                                                                          y, M, N, K);
    else
        linear_f32w_kernel<uint16_t, kF32wTokens><<<grid, 256, lds, stream_of(stream)>>>(
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
