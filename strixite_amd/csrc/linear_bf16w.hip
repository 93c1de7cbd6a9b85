// BF16-weight linear on gfx950: y[M, N] = x[M, K] . W[N, K]^T with W as raw BF16 bits (kernels/linear.hpp:14-24) and
// its prefill form linear_bf16w_wmma (kernels/linear_wmma.hpp:25-28). In the served model this is the MoE router
// projection (W [E + 1, d]: 512 experts + the shared-expert gate, runtime/qwen4exp.cpp:1132-1137) with FP32 logits out.
//
// Three kernels:
//   - rows (K % 8 == 0, aligned): a block takes 2 weight rows x 8 tokens; each thread owns every 256th 16-byte chunk
//     (8 weights) of those rows and issues all of its weight and activation loads before the first use, then the
//     per-(row, token) sums meet in a halving wave butterfly and across the four waves in LDS. The weight bytes are the
//     whole cost (4.2 MB for the served router) and are read once.
//   - mfma (BF16 or F32 x, M >= 64, K % 32 == 0): 64 weight rows x 64 tokens a block; a wave 16 rows x 64 tokens as
//     four v_mfma_f32_16x16x32_bf16 tiles sharing each weight fragment; the block's activation tile of a K step
//     (64 tokens x 32) is loaded once and shared through a double-buffered LDS tile. BF16 x: every product is exact
//     (8-bit significands), so only the FP32 summation order differs from the rows kernel. F32 x: linear_bf16w splits
//     each value into three BF16 terms (exact to 24 bits, three MFMAs a tile); linear_bf16w_wmma rounds it to BF16
//     once (the reference's WMMA semantics: "y = bf16(x) * W^T").
//   - generic (any K or alignment): a block a (row, 8 tokens), threads striding K, an LDS tree sum.
#include "common.hpp"

namespace sx {
namespace {

// ---------------- rows kernel ----------------
constexpr int kBwRows = 2, kBwTokens = 8, kBwUnroll = 2;

template <typename TX>
__device__ __forceinline__ void load8(const TX *p, float (&v)[8]) {
    if constexpr (sizeof(TX) == 4) {
        const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else {
        const uint4 u = *reinterpret_cast<const uint4 *>(p);
        const uint32_t d[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) v[2 * i] = __uint_as_float(d[i] << 16), v[2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
    }
}

template <typename TX, typename TY>
__global__ void __launch_bounds__(256) linear_bf16w_rows_kernel(const TX *x, const uint16_t *W, TY *y, int64_t M,
                                                                int64_t N, int64_t K) {
    __shared__ float part[4][kBwRows * kBwTokens];
    const int64_t m0 = (int64_t)blockIdx.y * kBwTokens, n0 = (int64_t)blockIdx.x * kBwRows;
    const int T = (int)min((int64_t)kBwTokens, M - m0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t K8 = K / 8;
    const uint4 *wr[kBwRows];
#pragma unroll
    for (int r = 0; r < kBwRows; ++r) wr[r] = reinterpret_cast<const uint4 *>(W + min(n0 + r, N - 1) * K);
    const TX *xt[kBwTokens];
#pragma unroll
    for (int t = 0; t < kBwTokens; ++t) xt[t] = x + (m0 + min(t, T - 1)) * K;
    float acc[kBwRows][kBwTokens];
#pragma unroll
    for (int r = 0; r < kBwRows; ++r)
#pragma unroll
        for (int t = 0; t < kBwTokens; ++t) acc[r][t] = 0.f;
    for (int64_t base = 0; base < K8; base += 256 * kBwUnroll) {
        // every load unconditional (the chunk index clamped, the weights zeroed past K) so that none waits for another
        uint4 w[kBwUnroll][kBwRows];
        float xv[kBwUnroll][kBwTokens][8];
#pragma unroll
        for (int u = 0; u < kBwUnroll; ++u) {
            const int64_t c = min(base + u * 256 + tid, K8 - 1);
#pragma unroll
            for (int r = 0; r < kBwRows; ++r) w[u][r] = wr[r][c];
#pragma unroll
            for (int t = 0; t < kBwTokens; ++t) load8(xt[t] + 8 * c, xv[u][t]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < kBwUnroll; ++u) {
            const bool on = base + u * 256 + tid < K8;
#pragma unroll
            for (int r = 0; r < kBwRows; ++r) {
                const uint32_t d[4] = {on ? w[u][r].x : 0u, on ? w[u][r].y : 0u, on ? w[u][r].z : 0u, on ? w[u][r].w : 0u};
                float wv[8];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    wv[2 * i] = __uint_as_float(d[i] << 16), wv[2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
#pragma unroll
                for (int t = 0; t < kBwTokens; ++t)
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[r][t] = fmaf(xv[u][t][e], wv[e], acc[r][t]);
            }
        }
    }
    // the 16 sums through a halving butterfly (a lane keeps the half its lane bit selects), then xor 2 and 1
    static_assert(kBwRows * kBwTokens == 16, "the reduction halves 16 sums");
    float v16[16];
#pragma unroll
    for (int r = 0; r < kBwRows; ++r)
#pragma unroll
        for (int t = 0; t < kBwTokens; ++t) v16[r * kBwTokens + t] = acc[r][t];
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
    if ((lane & 3) == 0)
        part[wave][((lane >> 5) & 1) * 8 + ((lane >> 4) & 1) * 4 + ((lane >> 3) & 1) * 2 + ((lane >> 2) & 1)] = tot;
    __syncthreads();
    if (tid < kBwRows * kBwTokens) {
        const int r = tid / kBwTokens, t = tid % kBwTokens;
        if (t < T && n0 + r < N)
            store_act(y, (m0 + t) * N + n0 + r, part[0][tid] + part[1][tid] + part[2][tid] + part[3][tid]);
    }
}

// ---------------- generic kernel (any K, any alignment) ----------------
template <typename TX, typename TY>
__global__ void __launch_bounds__(256) linear_bf16w_generic_kernel(const TX *x, const uint16_t *W, TY *y, int64_t M,
                                                                   int64_t N, int64_t K) {
    __shared__ float red[kBwTokens][256];
    const int64_t n = blockIdx.x, m0 = (int64_t)blockIdx.y * kBwTokens;
    const int T = (int)min((int64_t)kBwTokens, M - m0);
    float acc[kBwTokens];
#pragma unroll
    for (int t = 0; t < kBwTokens; ++t) acc[t] = 0.f;
    for (int64_t k = threadIdx.x; k < K; k += 256) {
        const float w = bf16_to_f32(W[n * K + k]);
#pragma unroll
        for (int t = 0; t < kBwTokens; ++t)
            if (t < T) acc[t] = fmaf(load_act(x, (m0 + t) * K + k), w, acc[t]);
    }
#pragma unroll
    for (int t = 0; t < kBwTokens; ++t) red[t][threadIdx.x] = acc[t];
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s)
#pragma unroll
            for (int t = 0; t < kBwTokens; ++t) red[t][threadIdx.x] += red[t][threadIdx.x + s];
        __syncthreads();
    }
    if ((int)threadIdx.x < T) store_act(y, (m0 + threadIdx.x) * N + n, red[threadIdx.x][0]);
}

// ---------------- MFMA kernel (prefill width) ----------------
typedef __bf16 bw_bf16x8 __attribute__((ext_vector_type(8)));
typedef float bw_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t bw_u32x4 __attribute__((ext_vector_type(4)));
constexpr int kBmTok = 64, kBmRows = 64, kBmMinTokens = 64;
constexpr int kBmLd = 40;  // BF16 a token row of the LDS tile: 32 of the step + 8 of padding (conflict-free reads)

// NPLANE BF16 planes of the activation tile: 1 (BF16 x, or F32 x rounded once), 3 (F32 x split exactly).
template <typename TX, int NPLANE>
__global__ void __launch_bounds__(256) linear_bf16w_mfma_kernel(const TX *x, const uint16_t *W, void *y, int out_f32,
                                                                int64_t M, int64_t N, int64_t K) {
    __shared__ __attribute__((aligned(16))) uint16_t xt[2][NPLANE][kBmTok * kBmLd];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n16 = lane & 15, g = lane >> 4;
    const int64_t row = (int64_t)blockIdx.x * kBmRows + wave * 16 + n16, t0 = (int64_t)blockIdx.y * kBmTok;
    const uint16_t *wr = W + min(row, N - 1) * K + g * 8;
    // this thread's chunk of every step's activation tile: token tid / 4 (clamped), 8 values at (tid % 4) * 8
    const TX *xc = x + min(t0 + tid / 4, M - 1) * K + (tid % 4) * 8;
    const int xs_off = (tid / 4) * kBmLd + (tid % 4) * 8;
    bw_f32x4 acc[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) acc[tt] = bw_f32x4{0.f, 0.f, 0.f, 0.f};
    constexpr int kDepth = 4;  // K steps of loads in flight
    constexpr int kXWords = sizeof(TX) == 4 ? 8 : 4;
    const int nk = (int)(K / 32);
    uint4 wb[kDepth];
    uint32_t xb[kDepth][kXWords];
    auto issue = [&](int step, int slot) __attribute__((always_inline)) {
        const int64_t k0 = (int64_t)min(step, nk - 1) * 32;
        wb[slot] = *reinterpret_cast<const uint4 *>(wr + k0);
        const uint4 *px = reinterpret_cast<const uint4 *>(xc + k0);
#pragma unroll
        for (int i = 0; i < kXWords / 4; ++i) {
            const uint4 v = px[i];
            xb[slot][4 * i] = v.x, xb[slot][4 * i + 1] = v.y, xb[slot][4 * i + 2] = v.z, xb[slot][4 * i + 3] = v.w;
        }
    };
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
        issue(d, d);
        __builtin_amdgcn_sched_barrier(0);  // in slot order, as the loop issues them (exact wait counts at its head)
    }
    auto step = [&](int s0, auto d_tag) __attribute__((always_inline)) {
        constexpr int D = decltype(d_tag)::value, BUF = D & 1;
        // the slot's activations into LDS (as NPLANE BF16 planes) and its weights into an operand before the reload
        if constexpr (sizeof(TX) == 2) {
            *reinterpret_cast<bw_u32x4 *>(&xt[BUF][0][xs_off]) = bw_u32x4{xb[D][0], xb[D][1], xb[D][2], xb[D][3]};
        } else {
            bw_bf16x8 pl[NPLANE];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = __uint_as_float(xb[D][e]);
                const __bf16 a = (__bf16)v;
                pl[0][e] = a;
                if constexpr (NPLANE == 3) {
                    const float r1 = v - (float)a;
                    const __bf16 b = (__bf16)r1;
                    pl[1][e] = b, pl[2][e] = (__bf16)(r1 - (float)b);
                }
            }
#pragma unroll
            for (int pp = 0; pp < NPLANE; ++pp) *reinterpret_cast<bw_bf16x8 *>(&xt[BUF][pp][xs_off]) = pl[pp];
        }
        // the weight operand copied out by asm: the slot's registers are then dead before their reload (an operand
        // aliasing them would make the loop rotate the ring through copies that wait for every load in flight).
        // The compiler's wait-count pass does not look at an asm statement's operands, so nothing waits for wb[D]
        // on the asm's behalf: it has landed because issue() loads the slot's activations after its weights, loads
        // complete in issue order, and the activations' LDS store above (an ordinary store, waited for by the
        // compiler, and before the volatile asm) needs them.
        uint4 bw;
        asm volatile("v_mov_b32 %0, %4\n\tv_mov_b32 %1, %5\n\tv_mov_b32 %2, %6\n\tv_mov_b32 %3, %7"
                     : "=v"(bw.x), "=v"(bw.y), "=v"(bw.z), "=v"(bw.w)
                     : "v"(wb[D].x), "v"(wb[D].y), "v"(wb[D].z), "v"(wb[D].w));
        // a step past the end (the unrolled loop's last round) multiplies zeros: no branch inside the loop, which
        // would make the wait-count pass wait for every load in flight at the loop head
        const bool live = s0 + D < nk;
        bw.x = live ? bw.x : 0u, bw.y = live ? bw.y : 0u, bw.z = live ? bw.z : 0u, bw.w = live ? bw.w : 0u;
        const bw_bf16x8 B = __builtin_bit_cast(bw_bf16x8, bw);
        __builtin_amdgcn_sched_barrier(0);
        issue(s0 + D + kDepth, D);
        lds_barrier();  // this step's tile complete; the other buffer's reads (the step before) done
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
            for (int pp = NPLANE - 1; pp >= 0; --pp) {
                const bw_bf16x8 A = *reinterpret_cast<const bw_bf16x8 *>(&xt[BUF][pp][(tt * 16 + n16) * kBmLd + g * 8]);
                acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B, acc[tt], 0, 0, 0);
            }
    };
    static_assert(kDepth == 4, "the K loop below is unrolled by four");
    for (int s0 = 0; s0 < nk; s0 += kDepth) {
        step(s0, std::integral_constant<int, 0>{});
        step(s0, std::integral_constant<int, 1>{});
        step(s0, std::integral_constant<int, 2>{});
        step(s0, std::integral_constant<int, 3>{});
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clamped loads past the end land before the wave exits
    if (row >= N) return;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t t = t0 + tt * 16 + 4 * g + v;
            if (t >= M) continue;
            if (out_f32) static_cast<float *>(y)[t * N + row] = acc[tt][v];
            else store_act(static_cast<uint16_t *>(y), t * N + row, acc[tt][v]);
        }
}

// Host side shared by both entry points. wmma: x rounded to BF16 before the products (linear_bf16w_wmma).
int linear_bf16w_impl(const char *fn, const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, int act,
                      int out_act, bool wmma, hipStream_t s) {
    SX_CHECK(x != nullptr && w != nullptr && y != nullptr, fn, ": null pointer (x=", x, ", w=", (const void *)w,
             ", y=", y, ")");
    SX_CHECK(M >= 1 && M <= 65535ll * kBwTokens, fn, ": M (rows of x) = ", M, ", expected 1..", 65535ll * kBwTokens);
    SX_CHECK(N >= 1 && N <= 0x7fffffff, fn, ": N (rows of W / outputs) = ", N, ", expected 1..", 0x7fffffff);
    SX_CHECK(K >= 1 && K <= (1 << 24), fn, ": K (inner dim) = ", K, ", expected 1..", 1 << 24);
    SX_CHECK(act == SX_ACT_F32 || act == SX_ACT_BF16, fn, ": unsupported activation dtype ", act);
    SX_CHECK(out_act == act || (act == SX_ACT_BF16 && out_act == SX_ACT_F32), fn, ": output dtype ", out_act,
             " with input ", act, " unsupported (same dtype, or BF16 -> F32)");
    SX_CHECK(apart(y, M * N * act_bytes(out_act), x, M * K * act_bytes(act)), fn, ": output y [", y, ", +",
             M * N * act_bytes(out_act), " B) overlaps input x [", x, ", +", M * K * act_bytes(act),
             " B); in-place isn't supported");
    if (wmma) {
        SX_CHECK(K % 64 == 0 && aligned(w, 16) && aligned(x, 16), fn, ": K = ", K,
                 " must be a multiple of 64 with 16-byte aligned x and W rows (kernels/linear_wmma.hpp:25)");
    }
    const bool vec = K % 8 == 0 && aligned(w, 16) && aligned(x, 16);
    const bool mfma = vec && K % 32 == 0 && (M >= kBmMinTokens || (wmma && act == SX_ACT_F32)) &&
                      (M + kBmTok - 1) / kBmTok <= 65535 && (N + kBmRows - 1) / kBmRows <= 0x7fffffff;
    if (mfma) {
        const dim3 grid((unsigned)((N + kBmRows - 1) / kBmRows), (unsigned)((M + kBmTok - 1) / kBmTok));
        const int f32 = out_act == SX_ACT_F32;
        if (act == SX_ACT_BF16)
            linear_bf16w_mfma_kernel<uint16_t, 1><<<grid, 256, 0, s>>>(static_cast<const uint16_t *>(x), w, y, f32, M,
                                                                        N, K);
        else if (wmma)
            linear_bf16w_mfma_kernel<float, 1><<<grid, 256, 0, s>>>(static_cast<const float *>(x), w, y, f32, M, N, K);
        else
            linear_bf16w_mfma_kernel<float, 3><<<grid, 256, 0, s>>>(static_cast<const float *>(x), w, y, f32, M, N, K);
        SX_LAUNCHED(fn, " (MFMA) M=", M, " N=", N, " K=", K);
        return SX_OK;
    }
    const dim3 grid((unsigned)(vec ? (N + kBwRows - 1) / kBwRows : N), (unsigned)((M + kBwTokens - 1) / kBwTokens));
    auto go = [&](auto tx, auto ty) {
        using TX = decltype(tx);
        using TY = decltype(ty);
        if (vec)
            linear_bf16w_rows_kernel<TX, TY><<<grid, 256, 0, s>>>(static_cast<const TX *>(x), w, static_cast<TY *>(y), M,
                                                                 N, K);
        else
            linear_bf16w_generic_kernel<TX, TY><<<grid, 256, 0, s>>>(static_cast<const TX *>(x), w,
                                                                    static_cast<TY *>(y), M, N, K);
    };
    if (act == SX_ACT_F32) go(float{}, float{});
    else if (out_act == SX_ACT_F32) go(uint16_t{}, float{});
    else go(uint16_t{}, uint16_t{});
    SX_LAUNCHED(fn, " M=", M, " N=", N, " K=", K);
    return SX_OK;
}

}  // namespace
}  // namespace sx

using namespace sx;

extern "C" {

int sx_linear_bf16w(const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, int act, int out_act,
                    sx_stream stream) {
    return linear_bf16w_impl("sx_linear_bf16w", x, w, y, M, N, K, act, out_act, false, stream_of(stream));
}

int sx_linear_bf16w_wmma(const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, int act,
                         int out_act, sx_stream stream) {
    return linear_bf16w_impl("sx_linear_bf16w_wmma", x, w, y, M, N, K, act, out_act, true, stream_of(stream));
}

}  // extern "C"
