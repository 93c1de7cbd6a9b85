// Prefill-width grouped expert GEMM on the matrix cores: q4 experts (G = 128), BF16 activations, any bucket size.
//
// The verify kernel (qmm) stages every activation row of a unit over the whole K in LDS and passes the weights once
// per 16 rows; with hundreds of rows a bucket (kernels/moe_grouped.hpp:5-17: the prefill path) that re-streams each
// expert's weights per 16 rows. Here a block owns a 64-slot tile of one bucket (the workspace's wide tiles,
// moe_grouped.hip:63-81) times 128 weight rows (4 waves x 2 tiles of 16), and walks K in blocks of 2 spans (256
// codes): the activation rows of the block go through LDS, double-buffered, while each wave's weight codes load
// straight into the MFMA B layout (16 rows x 64 B a load, as in qmm) and feed 4 token blocks of 16 slots each, so a
// code fragment is reused 4 times and each weight tile is read once a 64-slot tile (the other tiles of the same
// bucket run next to it and find it in L2). Per span (one quantization group):
//   acc[token][row] += s[row] * D + (m[row] - 128 s[row]) * sum_span x[token]
// with D = sum x * (128 + code) exactly from v_mfma_f32_16x16x32_bf16 (the same identity as qmm).
// Epilogues: SwiGLU (gate and up tiles of the same 16 features in one wave), plain gather, FP32 partials (combine).
#include "gemm_grouped.hpp"
#include "qmm_impl.hpp"

namespace sx::gg {
namespace {

using qmm::detail::bf16x8;
using qmm::detail::f32x4;

constexpr int kThreads = 256, kWaves = 4;
constexpr int kBM = 64;                      // slots a block tile
constexpr int kSpan = 128, kSpanBytes = 64;  // q4 codes / bytes a span (= one G = 128 group)
constexpr int kBKS = 2;                      // spans a K block
constexpr int kBK = kBKS * kSpan;            // codes a K block
constexpr int kLdx = kBK + 8;                // LDS row stride (BF16): +16 B staggers the rows over the banks
constexpr int kTW = 2;                       // 16-row weight tiles a wave
constexpr int kXLoads = kBM * (kBK / 8) / kThreads;  // 16-byte activation loads a thread a K block (8)

struct Params {
    const uint16_t *x;  // BF16 activations [tokens or slots, K]
    const uint8_t *q;
    const uint16_t *scale, *minv;
    void *y;
    const int32_t *ws;
    int64_t A, N, K;  // slots a token; rows an expert (SWIGLU: 2I); K
    int64_t E;
};

size_t lds_bytes() { return (size_t)2 * kBM * kLdx * 2 + (size_t)2 * kBKS * kBM * 4; }

template <int MODE, typename TY>
__global__ void __launch_bounds__(kThreads) gg_kernel(Params p) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    uint16_t *xs = reinterpret_cast<uint16_t *>(smem);                         // [2][kBM][kLdx] code order
    float *xsum = reinterpret_cast<float *>(smem + (size_t)2 * kBM * kLdx * 2);  // [2][kBKS][kBM]
    __shared__ int64_t s_xrow[kBM], s_out[kBM];
    __shared__ int s_T, s_bucket;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n16 = lane & 15, g = lane >> 4;
    const int64_t K = p.K;
    const int E = (int)p.E;

    // ---- the 64-slot tile: bucket, slots (wave 0, lane r fills row r) ----
    if (tid < 64) {
        const int32_t *ws = p.ws;
        const int32_t n_wt = ws[3], S = ws[1];
        int T = 0, bucket = -1;
        const int u = (int)blockIdx.x;
        if (u < n_wt) {
            const int32_t *offsets = ws + 4, *slots = offsets + E + 2;
            const int64_t Tmax = (int64_t)S / 16 + E + 2, WTmax = (int64_t)S / 64 + E + 2;
            const int32_t *wtile_bucket = slots + S + 2 * Tmax, *wtile_start = wtile_bucket + WTmax;
            bucket = wtile_bucket[u];
            const int32_t st = wtile_start[u];
            T = min(kBM, offsets[bucket + 1] - st);
            if (lane < T) {
                const int64_t slot = slots[st + lane];
                s_xrow[lane] = (MODE == qmm::COMBINE ? slot : slot / p.A) * K;
                s_out[lane] = slot;
            }
        }
        if (lane == 0) s_T = T, s_bucket = bucket;
    }
    __syncthreads();
    const int T = __builtin_amdgcn_readfirstlane(s_T), bucket = __builtin_amdgcn_readfirstlane(s_bucket);
    if (T == 0) return;  // past the tile count: uniform for the block
    const int64_t Nrows = MODE == qmm::SWIGLU ? p.N / 2 : p.N;  // output rows (features) an expert
    constexpr int kOutRows = MODE == qmm::SWIGLU ? kWaves * 16 : kWaves * kTW * 16;  // output rows a block
    const int64_t r0 = (int64_t)blockIdx.y * kOutRows;
    if (bucket == E) {  // invalid ids (reported by the grouping): NaN rows, never an out-of-range weight read
        for (int i = tid; i < T * kOutRows; i += kThreads) {
            const int r = i / kOutRows;
            const int64_t n = r0 + i % kOutRows;
            if (n >= Nrows) continue;
            if constexpr (MODE == qmm::COMBINE) static_cast<float *>(p.y)[s_out[r] * Nrows + n] = qnan();
            else store_act(static_cast<TY *>(p.y), s_out[r] * Nrows + n, qnan());
        }
        return;
    }

    // ---- this lane's weight rows: tile t of the wave, row n16 (clamped into the expert; stores are masked) ----
    const int64_t rowbytes = K / 2, ngroups = K / 128;
    const uint8_t *qrow[kTW];
    const uint32_t *srow[kTW], *mrow[kTW];  // two BF16 groups (one K block) a word
    int64_t feat[kTW];
#pragma unroll
    for (int t = 0; t < kTW; ++t) {
        int64_t n;  // row within the expert
        if constexpr (MODE == qmm::SWIGLU) n = (t == 0 ? 0 : Nrows) + r0 + wave * 16 + n16;  // gate, up
        else n = r0 + (wave * kTW + t) * 16 + n16;
        feat[t] = MODE == qmm::SWIGLU ? r0 + wave * 16 + n16 : n;
        const int64_t nn = min(n, (MODE == qmm::SWIGLU ? 2 * Nrows : Nrows) - 1);
        const int64_t row = (int64_t)bucket * p.N + nn;
        qrow[t] = p.q + row * rowbytes + g * 16;
        srow[t] = reinterpret_cast<const uint32_t *>(p.scale + row * ngroups);
        mrow[t] = reinterpret_cast<const uint32_t *>(p.minv + row * ngroups);
    }

    // ---- the pipeline: K block kb's loads go out while kb - 1 is computed ----
    const int nkb = (int)(K / kBK);
    uint4 wq[2][kTW][kBKS];
    uint32_t wsc[2][kTW], wmn[2][kTW];
    uint4 xr[kXLoads];
    auto issue = [&](int kb, auto slot_tag) {  // kb past the end re-loads the last block (never used)
        constexpr int R = decltype(slot_tag)::value;
        const int k = min(kb, nkb - 1);
#pragma unroll
        for (int b = 0; b < kXLoads; ++b) {
            const int i = b * kThreads + tid, r = min(i >> 5, T - 1), c8 = i & 31;  // rows past T repeat row T - 1
            xr[b] = *reinterpret_cast<const uint4 *>(p.x + s_xrow[r] + (int64_t)k * kBK + c8 * 8);
        }
#pragma unroll
        for (int t = 0; t < kTW; ++t) {
#pragma unroll
            for (int s = 0; s < kBKS; ++s)
                wq[R][t][s] = *reinterpret_cast<const uint4 *>(qrow[t] + (int64_t)k * (kBKS * kSpanBytes) + s * kSpanBytes);
            wsc[R][t] = srow[t][k], wmn[R][t] = mrow[t][k];
        }
    };
    auto stage = [&](int buf) {  // the activation registers of one K block -> LDS (code order) + per-span sums
        uint16_t *xb = xs + (size_t)buf * kBM * kLdx;
        float *sb = xsum + (size_t)buf * kBKS * kBM;
#pragma unroll
        for (int b = 0; b < kXLoads; ++b) {
            const int i = b * kThreads + tid, r = i >> 5, c8 = i & 31;
            uint4 planes[1];
            float sum;
            qmm::detail::chunk_planes<4, 1, uint16_t>(xr[b], planes, sum);
            *reinterpret_cast<uint4 *>(xb + r * kLdx + c8 * 8) = planes[0];
            sum = qmm::detail::group_sum_c<16>(sum);  // 16 chunks of 8 = one span
            if ((c8 & 15) == 0) sb[(c8 >> 4) * kBM + r] = sum;
        }
    };

    f32x4 acc[kTW][4];
#pragma unroll
    for (int t = 0; t < kTW; ++t)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) acc[t][tb] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int buf, auto slot_tag) {
        constexpr int R = decltype(slot_tag)::value;
        const uint16_t *xb = xs + (size_t)buf * kBM * kLdx;
        const float *sb = xsum + (size_t)buf * kBKS * kBM;
#pragma unroll
        for (int s = 0; s < kBKS; ++s) {
            bf16x8 B[kTW][4];
            float sc[kTW], cm[kTW];
#pragma unroll
            for (int t = 0; t < kTW; ++t) {
#pragma unroll
                for (int c = 0; c < 4; ++c) B[t][c] = qmm::detail::codes_b<4>(wq[R][t][s], c);
                const uint32_t sw = wsc[R][t], mw = wmn[R][t];
                sc[t] = __uint_as_float(s ? (sw & 0xFFFF0000u) : (sw << 16));
                const float mv = __uint_as_float(s ? (mw & 0xFFFF0000u) : (mw << 16));
                cm[t] = fmaf(-128.f, sc[t], mv);
            }
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                bf16x8 Aop[4];
                const uint16_t *xa = xb + (tb * 16 + n16) * kLdx + s * kSpan + g * 32;
#pragma unroll
                for (int c = 0; c < 4; ++c) Aop[c] = *reinterpret_cast<const bf16x8 *>(xa + c * 8);
                const float4 xv = *reinterpret_cast<const float4 *>(sb + s * kBM + tb * 16 + 4 * g);
#pragma unroll
                for (int t = 0; t < kTW; ++t) {
                    f32x4 D = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int c = 0; c < 4; ++c) D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Aop[c], B[t][c], D, 0, 0, 0);
                    acc[t][tb][0] = fmaf(sc[t], D[0], fmaf(cm[t], xv.x, acc[t][tb][0]));
                    acc[t][tb][1] = fmaf(sc[t], D[1], fmaf(cm[t], xv.y, acc[t][tb][1]));
                    acc[t][tb][2] = fmaf(sc[t], D[2], fmaf(cm[t], xv.z, acc[t][tb][2]));
                    acc[t][tb][3] = fmaf(sc[t], D[3], fmaf(cm[t], xv.w, acc[t][tb][3]));
                }
            }
        }
    };

    // prologue: block 0 into LDS buffer 0, block 1's loads in flight
    issue(0, std::integral_constant<int, 0>{});
    stage(0);
    issue(1, std::integral_constant<int, 1>{});
    __syncthreads();
    // two K blocks a trip, so that the register slots are constants; block kb computes from LDS buffer kb & 1
    for (int kb = 0; kb < nkb; kb += 2) {
        compute(0, std::integral_constant<int, 0>{});
        if (kb + 1 >= nkb) break;  // uniform
        stage(1);                  // block kb + 1 (its loads are in xr)
        issue(kb + 2, std::integral_constant<int, 0>{});
        __syncthreads();
        compute(1, std::integral_constant<int, 1>{});
        if (kb + 2 >= nkb) break;
        stage(0);  // block kb + 2
        issue(kb + 3, std::integral_constant<int, 1>{});
        __syncthreads();
    }

    // ---- stores: D row = token block tb, rows 4g..4g+3; column = the lane's weight row ----
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int r = tb * 16 + 4 * g + v;
            if (r >= T) continue;
            const int64_t o = s_out[r] * Nrows;
            if constexpr (MODE == qmm::SWIGLU) {
                if (feat[0] < Nrows) {
                    TY *h = static_cast<TY *>(p.y);
                    const float gv = as_stored(acc[0][tb][v], h), uv = as_stored(acc[1][tb][v], h);
                    store_act(h, o + feat[0], as_stored(silu(gv), h) * uv);
                }
            } else {
#pragma unroll
                for (int t = 0; t < kTW; ++t) {
                    if (feat[t] >= Nrows) continue;
                    if constexpr (MODE == qmm::COMBINE) static_cast<float *>(p.y)[o + feat[t]] = acc[t][tb][v];
                    else store_act(static_cast<TY *>(p.y), o + feat[t], acc[t][tb][v]);
                }
            }
        }
}

template <int MODE, typename TY>
hipError_t go(const Params &p, dim3 grid, hipStream_t stream) {
    auto k = gg_kernel<MODE, TY>;
    const size_t lds = lds_bytes();
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k, grid, dim3(kThreads), lds, stream, p);
    return hipGetLastError();
}

}  // namespace

bool eligible(int bits, int64_t G, int64_t K, int act) {
    return bits == 4 && G == 128 && K % kBK == 0 && K >= kBK && act == SX_ACT_BF16;
}

hipError_t launch(int mode, const void *x, const sx_qview *w, void *y, const int32_t *ws, int64_t M, int64_t A,
                  int64_t E, int out_act, hipStream_t stream) {
    Params p{};
    p.x = static_cast<const uint16_t *>(x), p.q = static_cast<const uint8_t *>(w->q);
    p.scale = static_cast<const uint16_t *>(w->scale), p.minv = static_cast<const uint16_t *>(w->minv);
    p.y = y, p.ws = ws, p.A = A, p.N = w->N / E, p.K = w->K, p.E = E;
    const int64_t S = M * A;
    const int64_t wtiles = S / kBM + E + 2;  // WTmax: an upper bound of the 64-slot tiles; the rest exit at once
    const int64_t out_rows = mode == qmm::SWIGLU ? p.N / 2 : p.N;
    const int64_t per_block = mode == qmm::SWIGLU ? kWaves * 16 : kWaves * kTW * 16;
    const dim3 grid((unsigned)wtiles, (unsigned)((out_rows + per_block - 1) / per_block));
    switch (mode) {
    case qmm::SWIGLU:
        return out_act == SX_ACT_F32 ? go<qmm::SWIGLU, float>(p, grid, stream) : go<qmm::SWIGLU, uint16_t>(p, grid, stream);
    case qmm::GATHER:
        return out_act == SX_ACT_F32 ? go<qmm::GATHER, float>(p, grid, stream) : go<qmm::GATHER, uint16_t>(p, grid, stream);
    default:
        return go<qmm::COMBINE, float>(p, grid, stream);
    }
}

}  // namespace sx::gg
