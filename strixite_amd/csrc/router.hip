// MoE routing on gfx950: the router projection (FP32 weights) and the top-k router (kernels/moe_router.hpp:11-40).
#include "common.hpp"
#include "route_impl.hpp"

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
__device__ __forceinline__ void project_rows(const TX *x, const float *W, float *y, int64_t M, int64_t N, int64_t K,
                                             float (*part)[kF32wRows * NT]) {
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
    // Wave reduction of the kF32wRows * NT (= 16) sums: halve the vector at each of the xor-32, 16, 8, 4 steps (a
    // lane keeps the half its lane bit selects and adds its partner's copy of it), then xor 2 and 1 on the last
    // value: 17 shuffles instead of 6 a sum. Lane bits 5..2 then name the sum a lane holds.
    static_assert(kF32wRows * NT == 16, "the reduction halves 16 sums");
    float v16[16];
#pragma unroll
    for (int r = 0; r < kF32wRows; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t) v16[r * NT + t] = acc[r][t];
#pragma unroll
    for (int n = 8, bit = 32; n >= 1; n >>= 1, bit >>= 1) {
        const bool upper = (lane & bit) != 0;
#pragma unroll
        for (int i = 0; i < n; ++i) {
            const float keep = upper ? v16[n + i] : v16[i], give = upper ? v16[i] : v16[n + i];
            v16[i] = keep + __shfl_xor(give, bit);
        }
    }
    float tot = v16[0];
    tot += __shfl_xor(tot, 2);
    tot += __shfl_xor(tot, 1);
    if ((lane & 3) == 0) part[wave][((lane >> 5) & 1) * 8 + ((lane >> 4) & 1) * 4 + ((lane >> 3) & 1) * 2 + ((lane >> 2) & 1)] = tot;
    __syncthreads();
    if (tid < kF32wRows * NT) {
        const int r = tid / NT, t = tid % NT;
        if (t < T && n0 + r < N) y[(m0 + t) * N + n0 + r] = part[0][tid] + part[1][tid] + part[2][tid] + part[3][tid];
    }
}

template <typename TX, int NT>
__global__ void __launch_bounds__(256) linear_f32w_kernel(const TX *x, const float *W, float *y, int64_t M, int64_t N,
                                                          int64_t K) {
    __shared__ float part[4][kF32wRows * NT];
    project_rows<TX, NT>(x, W, y, M, N, K, part);
}

// ---------------- router projection at prefill width (M >= 64, BF16 x): MFMA ----------------
// Each FP32 weight is the exact sum of three BF16 terms (hi = rne(w), mid = rne(w - hi), lo = rne(w - hi - mid)), so
// x . W = x . hi + x . mid + x . lo with every product exact in v_mfma_f32_16x16x32_bf16 and FP32 accumulation, as
// the scalar kernel's (up to the order of the FP32 additions). A block owns 64 weight rows x 64 tokens and splits K in
// two halves over its 8 waves; a wave 16 rows x the 64 tokens of its half (4 MFMA tiles sharing each split weight
// fragment). A half's 64 activation rows of a K step (4 KB) are loaded once, a 16-byte chunk a thread, and shared
// through a double-buffered LDS tile (rows 80 bytes apart: the operand reads are free of bank conflicts), so the
// activations are read once per 64 weight rows rather than once per wave. 4096 x 512 at M = 2048: 39 us against 45.6
// with one wave a SIMD over the whole K (the time is the chain of K steps, nearly the same at M = 128).
typedef __bf16 pw_bf16x8 __attribute__((ext_vector_type(8)));
typedef float pw_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t pw_u32x4 __attribute__((ext_vector_type(4)));  // a vector, not an aggregate: copies stay in registers
constexpr int kPwTok = 64, kPwRows = 64, kPwMinTokens = 64, kPwKs = 1;
constexpr int kPwLd = 40;  // BF16 a token row of the LDS tile (32 of the step + 8 of padding)

__device__ __forceinline__ void split3(const float4 &a, const float4 &b, pw_bf16x8 &hi, pw_bf16x8 &mid, pw_bf16x8 &lo) {
    // hardware RNE conversions (v_cvt_pk_bf16_f32); the weights are finite, so NaN payloads never matter here
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const __bf16 h = (__bf16)v[j];
        const float r1 = v[j] - (float)h;
        const __bf16 m = (__bf16)r1;
        hi[j] = h, mid[j] = m, lo[j] = (__bf16)(r1 - (float)m);
    }
}

// KS K sub-steps of 32 a barrier (a step), kPwDepth steps of loads in flight. The three BF16 terms accumulate in
// three independent sums (no MFMA waits on the one before it), added once at the end. The block's 8 waves are two
// halves of K (waves 4..7 the second, from K step ceil(nk / 2)), each with its own activation tiles: two waves a
// SIMD, so one's split and LDS traffic overlaps the other's MFMAs; the halves' sums meet in LDS at the end and are
// added first half first.
template <int KS>
__global__ void __launch_bounds__(512) linear_f32w_mfma_kernel(const uint16_t *x, const float *W, float *y, int64_t M,
                                                               int64_t N, int64_t K) {
    __shared__ __attribute__((aligned(16))) uint16_t xt[2][2][KS][kPwTok * kPwLd];  // [half][buffer][sub-step]
    __shared__ __attribute__((aligned(16))) float red[4][16][64];                   // the second half's sums
    const int tid = threadIdx.x & 255, kh = threadIdx.x >> 8, lane = tid & 63, wave = tid >> 6, n16 = lane & 15,
              g = lane >> 4;
    const int64_t row = (int64_t)blockIdx.x * kPwRows + wave * 16 + n16, t0 = (int64_t)blockIdx.y * kPwTok;
    const int nk_all = (int)(K / 32), kbeg = kh ? (nk_all + 1) / 2 : 0;
    const int nk = kh ? nk_all - kbeg : (nk_all + 1) / 2;  // this half's sub-steps (the second may have one fewer)
    const int64_t kb = nk > 0 ? (int64_t)kbeg * 32 : 0;  // a half with no steps (K = 32) reads step 0, never used
    const float *wr = W + min(row, N - 1) * K + kb + g * 8;
    // this thread's chunk of every sub-step's activation tile: token tid / 4 (clamped), 16 bytes at (tid % 4) * 8
    const uint16_t *xc = x + min(t0 + tid / 4, M - 1) * K + kb + (tid % 4) * 8;
    const int xs_off = (tid / 4) * kPwLd + (tid % 4) * 8;
    auto xt_at = [&](int buf, int q) -> uint16_t * { return xt[kh][buf][q]; };
    pw_f32x4 acc[3][4];  // [term: lo, mid, hi][token tile]
#pragma unroll
    for (int pl = 0; pl < 3; ++pl)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc[pl][tt] = pw_f32x4{0.f, 0.f, 0.f, 0.f};
    // kPwDepth steps of loads in flight: step s + kPwDepth is issued into the slot step s frees (sub-steps past the
    // end re-load the last one, never used)
    constexpr int kPwDepth = KS == 1 ? 4 : 2;
    float4 wb[kPwDepth][KS][2];
    pw_u32x4 xb[kPwDepth][KS];
    auto issue = [&](int step, int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < KS; ++q) {
            const int64_t k0 = (int64_t)max(min(step * KS + q, nk - 1), 0) * 32;
            wb[slot][q][0] = *reinterpret_cast<const float4 *>(wr + k0);
            wb[slot][q][1] = *reinterpret_cast<const float4 *>(wr + k0 + 4);
            xb[slot][q] = *reinterpret_cast<const pw_u32x4 *>(xc + k0);
        }
    };
#pragma unroll
    for (int d = 0; d < kPwDepth; ++d) {
        issue(d, d);
        __builtin_amdgcn_sched_barrier(0);  // in slot order, as the loop issues them (exact wait counts at its head)
    }
    // one step on ring slot D (a constant: the slots stay in registers)
    auto step = [&](int s0, auto d_tag) __attribute__((always_inline)) {
        constexpr int D = decltype(d_tag)::value, BUF = D & 1;  // kPwDepth is even: the LDS buffer of step s0 + D
        // the slot's activation chunks into LDS and its weights split before the slot is reloaded (a value still
        // live at the reload would make the loop rotate the ring through copies that wait for every load)
        pw_bf16x8 hi[KS], mid[KS], lo[KS];
#pragma unroll
        for (int q = 0; q < KS; ++q) {
            *reinterpret_cast<pw_u32x4 *>(xt_at(BUF, q) + xs_off) = xb[D][q];
            split3(wb[D][q][0], wb[D][q][1], hi[q], mid[q], lo[q]);
            // a sub-step past the end multiplies zeros: no branch inside the loop, which would make the wait-count
            // pass wait for every load in flight at the loop head
            if ((s0 + D) * KS + q >= nk) hi[q] = pw_bf16x8{}, mid[q] = pw_bf16x8{}, lo[q] = pw_bf16x8{};
        }
        __builtin_amdgcn_sched_barrier(0);  // the reload stays after the last use of the slot
        issue(s0 + D + kPwDepth, D);
        // the tile of this step is complete; the other buffer's reads (the step before) are done. LDS-only fences:
        // a __syncthreads() would also wait for the loads of the steps in flight.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
#pragma unroll
        for (int q = 0; q < KS; ++q)
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                const pw_bf16x8 A = *reinterpret_cast<const pw_bf16x8 *>(xt_at(BUF, q) + (tt * 16 + n16) * kPwLd + g * 8);
                acc[0][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, lo[q], acc[0][tt], 0, 0, 0);
                acc[1][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, mid[q], acc[1][tt], 0, 0, 0);
                acc[2][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, hi[q], acc[2][tt], 0, 0, 0);
            }
    };
    const int nsteps = (((nk_all + 1) / 2) + KS - 1) / KS;  // both halves take the same steps (the barriers pair up)
    if constexpr (kPwDepth == 4) {
        for (int s0 = 0; s0 < nsteps; s0 += 4) {
            step(s0, std::integral_constant<int, 0>{});
            step(s0, std::integral_constant<int, 1>{});
            step(s0, std::integral_constant<int, 2>{});
            step(s0, std::integral_constant<int, 3>{});
        }
    } else {
        for (int s0 = 0; s0 < nsteps; s0 += 2) {
            step(s0, std::integral_constant<int, 0>{});
            step(s0, std::integral_constant<int, 1>{});
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clamped loads past the end land before the wave exits
    if (kh == 1) {
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
            for (int v = 0; v < 4; ++v) red[wave][tt * 4 + v][lane] = (acc[0][tt][v] + acc[1][tt][v]) + acc[2][tt][v];
    }
    __syncthreads();
    if (kh == 1 || row >= N) return;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t t = t0 + tt * 16 + 4 * g + v;
            if (t < M) y[t * N + row] = ((acc[0][tt][v] + acc[1][tt][v]) + acc[2][tt][v]) + red[wave][tt * 4 + v][lane];
        }
}

// ---------------- top-k router: one wave a token (routing::route_token) ----------------
template <typename T, int NV>
__global__ void __launch_bounds__(64) moe_router_kernel(const T *logits, int64_t ld, int E, int k, const T *shared,
                                                        int64_t shared_ld, int32_t shared_id, int32_t *ids,
                                                        float *coef, int A, uint32_t *err) {
    const int64_t m = blockIdx.x;
    const T *row = logits + m * ld;
    const float sl = shared != nullptr ? load_act(shared, m * shared_ld) : 0.f;
    routing::route_token<NV>([&](int e) { return load_act(row, e); }, E, k, shared != nullptr, sl, shared_id, m,
                             ids + m * A, coef + m * A, nullptr, err);
}

// ---------------- top-k routing + grouping in one block (verify width) ----------------
// moe_router and moe_group_routes fused where one block can hold the slots: 16 waves route 16 tokens at a time
// (routing::route_token), the ids also land in LDS, then the 1024 threads counting-sort the slots into the
// workspace (routing::group_in_block). One launch and no global round trip between the two.
constexpr int kRgThreads = 1024, kRgMaxSlots = 2048;

template <typename T, int NV>
__global__ void __launch_bounds__(kRgThreads)
    router_group_kernel(const T *logits, int64_t ld, int M, int E, int k, int32_t *ids, float *coef,
                        uint32_t *router_err, int32_t *ws, int Tmax, int WTmax, uint32_t *expert_err) {
    __shared__ int32_t lds_ids[kRgMaxSlots];
    __shared__ int cnt[kRgThreads], cursor[kRgThreads];
    __shared__ int wtot[kRgThreads / 64][3];
    __shared__ int first_bad;
    const int wave = threadIdx.x >> 6;
    for (int m = wave; m < M; m += kRgThreads / 64) {
        const T *row = logits + (int64_t)m * ld;
        routing::route_token<NV>([&](int e) { return load_act(row, e); }, E, k, false, 0.f, 0, m,
                                 ids + (int64_t)m * k, coef + (int64_t)m * k, lds_ids + m * k, router_err);
    }
    __syncthreads();
    routing::group_in_block<kRgThreads>([&](int s) { return lds_ids[s]; }, M * k, E, Tmax, WTmax, ws, expert_err,
                                        cnt, cursor, wtot, &first_bad);
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
    if (act == SX_ACT_BF16 && M >= kPwMinTokens && K % 32 == 0 && aligned(x, 16) && (M + kPwTok - 1) / kPwTok <= 65535) {
        const dim3 g2((unsigned)((N + kPwRows - 1) / kPwRows), (unsigned)((M + kPwTok - 1) / kPwTok));
        linear_f32w_mfma_kernel<kPwKs><<<g2, 512, 0, stream_of(stream)>>>(static_cast<const uint16_t *>(x), W, y, M, N, K);
        SX_LAUNCHED("linear_f32w (MFMA) M=", M, " N=", N, " K=", K);
        return SX_OK;
    }
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

int sx_moe_router_group(const void *logits, int64_t ld, int64_t M, int64_t E, int64_t k, int act, int32_t *ids,
                        float *coef, uint32_t *router_err, void *ws, size_t ws_bytes, uint32_t *expert_err,
                        sx_stream stream) {
    SX_CHECK(logits != nullptr && ids != nullptr && coef != nullptr && router_err != nullptr && ws != nullptr &&
                 expert_err != nullptr,
             "null pointer");
    SX_CHECK(M >= 1 && E >= 1 && E <= 1023 && k >= 1 && k <= E && k <= 32 && M * k <= kRgMaxSlots, "M = ", M,
             ", E = ", E, ", k = ", k, " (E <= 1023, k <= min(E, 32), M*k <= ", kRgMaxSlots,
             "; larger: moe_router + moe_group_routes)");
    SX_CHECK(ld >= E, "logits row stride ld = ", ld, " < E = ", E);
    SX_CHECK((const void *)ids != (const void *)coef, "ids and coef are the same buffer");
    SX_CHECK(act == SX_ACT_F32 || act == SX_ACT_BF16, "unsupported activation dtype ", act);
    SX_CHECK(aligned(ws, 4), "workspace must be 4-byte aligned");
    const Layout L = layout_of(M, k, E);
    SX_CHECK(ws_bytes >= (size_t)L.ints() * 4, "workspace of ", ws_bytes, " bytes, needs ", L.ints() * 4);
    const int nv = E <= 256 ? 4 : E <= 512 ? 8 : 16;
    auto go = [&](auto tag, auto nvc) {
        using T = decltype(tag);
        router_group_kernel<T, decltype(nvc)::value><<<1, kRgThreads, 0, stream_of(stream)>>>(
            static_cast<const T *>(logits), ld, (int)M, (int)E, (int)k, ids, coef, router_err,
            static_cast<int32_t *>(ws), (int)L.Tmax, (int)L.WTmax, expert_err);
    };
    auto by_nv = [&](auto tag) {
        if (nv == 4) go(tag, std::integral_constant<int, 4>{});
        else if (nv == 8) go(tag, std::integral_constant<int, 8>{});
        else go(tag, std::integral_constant<int, 16>{});
    };
    if (act == SX_ACT_F32) by_nv(float{});
    else by_nv(uint16_t{});
    SX_LAUNCHED("moe_router_group M=", M, " E=", E, " k=", k);
    return SX_OK;
}

}  // extern "C"
