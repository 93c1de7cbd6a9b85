// Prefill-width grouped expert GEMM on the matrix cores: q4 experts (G = 128), BF16 activations, any bucket size.
//
// The verify kernel (qmm) stages every activation row of a unit over the whole K in LDS and passes the weights once
// per 16 rows; with hundreds of rows a bucket (kernels/moe_grouped.hpp:5-17: the prefill path) that re-streams each
// expert's weights per 16 rows. Here a block owns a 64-slot tile of one bucket (the workspace's wide tiles,
// moe_grouped.hip:63-81) times 256 weight rows (8 waves x 2 tiles of 16; SwiGLU: 128 features, gate and up), and
// walks K in blocks of 2 spans (256 codes) through a 3-stage pipeline: the block's activation rows go to LDS by
// direct global->LDS loads ([chunk][row] 16-byte units, so the MFMA reads are conflict-free), two blocks ahead,
// while each wave's weight codes load straight into the MFMA B layout (16 rows x 64 B a load, as in qmm) and feed
// 4 token blocks of 16 slots each: a code fragment is used 4 times and each weight tile is read once a 64-slot tile
// (the other tiles of the same bucket run next to it and find it in L2). Per span (one quantization group):
//   acc[token][row] += s[row] * D + (m[row] - 128 s[row]) * sum_span x[token]
// with D = sum x * (128 + code) exactly from v_mfma_f32_16x16x32_bf16 (the same identity as qmm).
// Epilogues: SwiGLU (gate and up tiles of the same 16 features in one wave), plain gather, FP32 partials (combine).
#include "gemm_grouped.hpp"
#include "qmm_impl.hpp"

namespace sx::gg {
namespace {

using qmm::detail::bf16x8;
using qmm::detail::f32x4;

constexpr int kThreads = 512, kWaves = 8;
constexpr int kBM = 64;                      // slots a block tile
constexpr int kSpan = 128, kSpanBytes = 64;  // q4 codes / bytes a span (= one G = 128 group)
constexpr int kBKS = 2;                      // spans a K block
constexpr int kBK = kBKS * kSpan;            // codes a K block
constexpr int kChunks = kBK / 8;             // 16-byte chunks of a row a K block (32): 4 a wave
constexpr int kStages = 3;                   // K blocks in LDS: two in flight while one is computed
constexpr int kTW = 2;                       // 16-row weight tiles a wave
constexpr size_t kStageBytes = (size_t)kChunks * kBM * 16;  // [chunk][row] 16-byte units: 32 KB
constexpr size_t kSumBytes = (size_t)kBKS * kBM * 4;         // [span][row] FP32
constexpr int kLoadsPerIssue = kChunks / kWaves + kTW * kBKS + 2 * kTW;  // VMEM instructions a wave a K block

struct Params {
    const uint16_t *x;  // BF16 activations [tokens or slots, K]
    const uint8_t *q;
    const uint16_t *scale, *minv;
    void *y;
    const int32_t *ws;
    int64_t A, N, K;  // slots a token; rows an expert (SWIGLU: 2I); K
    int64_t E;
};


// B operand of MFMA c from a lane's 16 code bytes in natural code order: dword c's nibbles j = 0..7 (codes
// k0 + j, the low nibble the even code) as BF16 128 + code, pairs assembled by byte selects.
__device__ __forceinline__ bf16x8 codes_nat(const uint4 &w, int c) {
    const uint32_t d = qmm::detail::dword(w, c), lo = d & 0x0F0F0F0Fu, hi = (d >> 4) & 0x0F0F0F0Fu;
    uint4 v;
    v.x = __builtin_amdgcn_perm(hi, lo, 0x0C040C00u) | 0x43004300u;
    v.y = __builtin_amdgcn_perm(hi, lo, 0x0C050C01u) | 0x43004300u;
    v.z = __builtin_amdgcn_perm(hi, lo, 0x0C060C02u) | 0x43004300u;
    v.w = __builtin_amdgcn_perm(hi, lo, 0x0C070C03u) | 0x43004300u;
    return __builtin_bit_cast(bf16x8, v);
}

template <int MODE, typename TY>
__global__ void __launch_bounds__(kThreads) gg_kernel(Params p) {
    // One array a stage, so that the wait-count pass tells a stage's LDS DMA apart from the others'.
    __shared__ __attribute__((aligned(16))) unsigned char xs0[kStageBytes], xs1[kStageBytes], xs2[kStageBytes];
    __shared__ __attribute__((aligned(16))) float ss[kStages][kBKS * kBM];
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
    // the activation row this lane stages (rows past T repeat row T - 1; their outputs are never stored)
    const uint16_t *xlane = p.x + s_xrow[min(lane, T - 1)];

    // ---- the pipeline: K block kb + 2 is loading while kb is summed and computed ----
    const int nkb = (int)(K / kBK);
    uint4 wq[kStages][kTW][kBKS];
    uint32_t wsc[kStages][kTW], wmn[kStages][kTW];
    auto stage_at = [&](int st) -> unsigned char * { return st == 0 ? xs0 : st == 1 ? xs1 : xs2; };
    auto sums_at = [&](int st) -> float * { return ss[st]; };
    // K block kb (clamped: past the end it re-loads the last block, never used): this wave's 4 activation chunks of
    // all 64 rows straight into LDS ([chunk][row], lane = row), then its weight codes, scales and mins into registers.
    auto issue = [&](int kb, int st, auto slot_tag) {
        constexpr int R = decltype(slot_tag)::value;
        const int k = min(kb, nkb - 1);
#pragma unroll
        for (int i = 0; i < kChunks / kWaves; ++i) {
            const int c = wave * (kChunks / kWaves) + i;
            __builtin_amdgcn_global_load_lds(
                (const void *)(xlane + (int64_t)k * kBK + c * 8),
                (__attribute__((address_space(3))) void *)(stage_at(st) + (size_t)c * kBM * 16), 16, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < kTW; ++t) {
#pragma unroll
            for (int s = 0; s < kBKS; ++s)
                wq[R][t][s] = *reinterpret_cast<const uint4 *>(qrow[t] + (int64_t)k * (kBKS * kSpanBytes) + s * kSpanBytes);
            wsc[R][t] = srow[t][k], wmn[R][t] = mrow[t][k];
        }
    };
    // Span sums of the staged rows: 4 threads a (span, row), 32 codes each, added across the quad.
    auto sum_spans = [&](int st) {
        const int q = tid >> 2, part = tid & 3, s = q >> 6, r = q & (kBM - 1);
        const unsigned char *xb = stage_at(st);
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v[8];
            qmm::detail::unpack8(*reinterpret_cast<const uint4 *>(xb + ((size_t)(s * 16 + part * 4 + i) * kBM + r) * 16), v);
#pragma unroll
            for (int j = 0; j < 8; ++j) sum += v[j];
        }
        sum = qmm::detail::group_sum_c<4>(sum);
        if (part == 0) sums_at(st)[s * kBM + r] = sum;
    };

    f32x4 acc[kTW][4];
#pragma unroll
    for (int t = 0; t < kTW; ++t)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) acc[t][tb] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int st, auto slot_tag) {
        constexpr int R = decltype(slot_tag)::value;
        const unsigned char *xb = stage_at(st);
        const float *sb = sums_at(st);
#pragma unroll
        for (int s = 0; s < kBKS; ++s) {
            bf16x8 B[kTW][4];
            float sc[kTW], cm[kTW];
#pragma unroll
            for (int t = 0; t < kTW; ++t) {
#pragma unroll
                for (int c = 0; c < 4; ++c) B[t][c] = codes_nat(wq[R][t][s], c);
                const uint32_t sw = wsc[R][t], mw = wmn[R][t];
                sc[t] = __uint_as_float(s ? (sw & 0xFFFF0000u) : (sw << 16));
                const float mv = __uint_as_float(s ? (mw & 0xFFFF0000u) : (mw << 16));
                cm[t] = fmaf(-128.f, sc[t], mv);
            }
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                bf16x8 Aop[4];
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    Aop[c] = *reinterpret_cast<const bf16x8 *>(xb + ((size_t)(s * 16 + g * 4 + c) * kBM + tb * 16 + n16) * 16);
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
    // One K block: the stage two blocks ahead is free once everyone has computed the block before this one; this
    // wave's chunks of block kb have landed once only the loads issued after them are outstanding (VMEM completes in
    // order); everyone's have after the barrier.
    // Barriers are s_barrier with explicit waits: a __syncthreads() fence would wait for every outstanding load,
    // the next blocks' included (the LDS DMA counts as an LDS write).
    auto step = [&](int kb, auto st_tag) {
        constexpr int ST = decltype(st_tag)::value;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // everyone is done with block kb - 1
        issue(kb + 2, (ST + 2) % kStages, std::integral_constant<int, (ST + 2) % kStages>{});
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(3 * kLoadsPerIssue - kChunks / kWaves) : "memory");
        sum_spans(ST);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        compute(ST, std::integral_constant<int, ST>{});
    };

    issue(0, 0, std::integral_constant<int, 0>{});
    issue(1, 1, std::integral_constant<int, 1>{});
    // unrolled by the stage count so that stages and slots are constants (a full unroll hoists every load and
    // spills)
    for (int kb = 0; kb < nkb; kb += kStages) {
        step(kb, std::integral_constant<int, 0>{});
        if (kb + 1 >= nkb) break;
        step(kb + 1, std::integral_constant<int, 1>{});
        if (kb + 2 >= nkb) break;
        step(kb + 2, std::integral_constant<int, 2>{});
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clamped loads past the end land before the block exits

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
    hipLaunchKernelGGL((gg_kernel<MODE, TY>), grid, dim3(kThreads), 0, stream, p);
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
    hipError_t e;
    switch (mode) {
    case qmm::SWIGLU:
        e = out_act == SX_ACT_F32 ? go<qmm::SWIGLU, float>(p, grid, stream) : go<qmm::SWIGLU, uint16_t>(p, grid, stream);
        break;
    case qmm::GATHER:
        e = out_act == SX_ACT_F32 ? go<qmm::GATHER, float>(p, grid, stream) : go<qmm::GATHER, uint16_t>(p, grid, stream);
        break;
    default:
        e = go<qmm::COMBINE, float>(p, grid, stream);
    }
    return e;
}

}  // namespace sx::gg
