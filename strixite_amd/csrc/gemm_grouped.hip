// Prefill-width grouped expert GEMM on the matrix cores: q4 experts (G = 128), BF16 activations, any bucket size.
//
// The verify kernel (qmm) stages every activation row of a unit over the whole K in LDS and passes the weights once
// per 16 rows; with hundreds of rows a bucket (kernels/moe_grouped.hpp:5-17: the prefill path) that re-streams each
// expert's weights per 16 rows. Here a block owns a 64-slot tile of one bucket (the workspace's wide tiles,
// moe_grouped.hip:63-81) times 256 weight rows (8 waves x 2 tiles of 16; SwiGLU: 128 features, gate and up), and
// walks K one span (128 codes, one quantization group) a step through a 4-stage pipeline of direct global->LDS
// loads (DMA): the block's activation rows (swizzled so that the MFMA operand reads are conflict-free) and each
// wave's weight codes (16 rows x 64 B a tile, in the MFMA B layout, as in qmm), scales and mins, three steps ahead.
// A code fragment feeds 4 token blocks of 16 slots each, and each weight tile is read once a 64-slot tile (the
// other tiles of the same bucket run next to it and find it in L2). Per span:
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
constexpr int kSpan = 128, kSpanBytes = 64;  // q4 codes / bytes a span (= one G = 128 group) = one K step
constexpr int kUnits = kSpan / 8;            // 16-byte units of a row a K step (16)
constexpr int kStages = 4;                   // K steps in LDS: three in flight while one is computed
constexpr int kTW = 2;                       // 16-row weight tiles a wave
constexpr int kXInstr = kBM * kUnits / 64 / kWaves;  // activation DMA instructions a wave a step (2)
constexpr int kLoadsOdd = kXInstr + kTW;        // activation + code DMA instructions a wave an odd step (4)
constexpr int kLoadsEven = kLoadsOdd + 2 * kTW;  // even steps add the scale and min words of two groups (8)
constexpr int kXBytes = kBM * kUnits * 16;             // 16 KB
constexpr int kWBytes = kWaves * kTW * 64 * 16;        // 16 KB: a wave's tiles, lane-ordered
constexpr int kSBytes = kWaves * kTW * 2 * 64 * 4;     // 8 KB: scale / min words, lane-ordered

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

__device__ __forceinline__ void dma16(const void *src, void *lds) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void *src, void *lds) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds, 4, 0, 0);
}

template <int MODE, typename TY>
__global__ void __launch_bounds__(kThreads) gg_kernel(Params p) {
    // One array a stage and kind, so that the wait-count pass tells a stage's DMA apart from the others'.
    __shared__ __attribute__((aligned(16))) unsigned char x0[kXBytes], x1[kXBytes], x2[kXBytes], x3[kXBytes];
    __shared__ __attribute__((aligned(16))) unsigned char w0[kWBytes], w1[kWBytes], w2[kWBytes], w3[kWBytes];
    // scale / min words (two groups each) load on even steps only; odd step k uses step k - 1's
    __shared__ __attribute__((aligned(16))) unsigned char c0[kSBytes], c2[kSBytes];
    __shared__ __attribute__((aligned(16))) float ss[kStages][kBM];
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
    const uint32_t *srow[kTW], *mrow[kTW];  // the word holding groups 2i, 2i + 1
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
    // Activation staging: a step is 16 instructions of 64 lanes x 16 B; instruction I covers rows 4I .. 4I + 3,
    // lane l = 16 (row % 4) + (chunk ^ row % 16), so each reads 4 x 256 contiguous bytes and the 16 rows an MFMA
    // operand read touches fall in 16 different bank groups. This wave issues I = 2 wave + j (rows 8 wave + 4 j +
    // lane / 16; past T: row T - 1 again, never stored).
    const uint16_t *xl[kXInstr];
#pragma unroll
    for (int j = 0; j < kXInstr; ++j) {
        const int r = 8 * wave + 4 * j + (lane >> 4);
        xl[j] = p.x + s_xrow[min(r, T - 1)] + (((lane & 15) ^ (r & 15)) * 8);
    }

    auto xs_at = [&](int st) -> unsigned char * { return st == 0 ? x0 : st == 1 ? x1 : st == 2 ? x2 : x3; };
    auto ws_at = [&](int st) -> unsigned char * { return st == 0 ? w0 : st == 1 ? w1 : st == 2 ? w2 : w3; };
    auto cs_at = [&](int st) -> unsigned char * { return st < 2 ? c0 : c2; };  // stages 0, 1 share c0; 2, 3 c2
    const int nk = (int)(K / kSpan);
    const int ntb = (T + 15) >> 4;  // 16-slot token blocks holding slots

    // K step k (clamped: past the end it re-loads the last step, never used), all by DMA into stage st: this wave's
    // two activation instructions, its two code tiles (16 rows x 64 B, lane-ordered as the B operand wants them),
    // and the scale / min words of its rows.
    auto issue = [&](int kstep, int st) {  // st = kstep % kStages: even stages carry the scale words
        const int k = min(kstep, nk - 1);
#pragma unroll
        for (int j = 0; j < kXInstr; ++j) dma16(xl[j] + (int64_t)k * kSpan, xs_at(st) + (2 * wave + j) * 1024);
#pragma unroll
        for (int t = 0; t < kTW; ++t) dma16(qrow[t] + (int64_t)k * kSpanBytes, ws_at(st) + (wave * kTW + t) * 1024);
        if ((st & 1) == 0) {
#pragma unroll
            for (int t = 0; t < kTW; ++t) {
                dma4(srow[t] + (k >> 1), cs_at(st) + ((wave * kTW + t) * 2 + 0) * 256);
                dma4(mrow[t] + (k >> 1), cs_at(st) + ((wave * kTW + t) * 2 + 1) * 256);
            }
        }
    };
    // Span sums: 8 threads a row, 2 units each (the swizzle only permutes a row's units), added across 8 lanes.
    auto sum_spans = [&](int st) {
        const int r = tid >> 3, part = tid & 7;
        const unsigned char *xb = xs_at(st) + ((r >> 2) * 64 + (r & 3) * 16 + part * 2) * 16;
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float v[8];
            qmm::detail::unpack8(*reinterpret_cast<const uint4 *>(xb + i * 16), v);
#pragma unroll
            for (int j = 0; j < 8; ++j) sum += v[j];
        }
        sum = qmm::detail::group_sum_c<8>(sum);
        if (part == 0) ss[st][r] = sum;
    };

    f32x4 acc[kTW][4];
#pragma unroll
    for (int t = 0; t < kTW; ++t)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) acc[t][tb] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Scale / min words of the current pair of steps: read from LDS on the even step and kept in registers for the
    // odd one (by then the pair-after-next is already landing in the same array).
    uint32_t swd[kTW], mwd[kTW];
    auto compute = [&](auto st_tag) {
        constexpr int st = decltype(st_tag)::value;
        const unsigned char *xb = xs_at(st), *wb = ws_at(st), *cb = cs_at(st);
        bf16x8 B[kTW][4];
        float sc[kTW], cm[kTW];
#pragma unroll
        for (int t = 0; t < kTW; ++t) {
            const uint4 w = *reinterpret_cast<const uint4 *>(wb + (wave * kTW + t) * 1024 + lane * 16);
#pragma unroll
            for (int c = 0; c < 4; ++c) B[t][c] = codes_nat(w, c);
            if constexpr ((st & 1) == 0) {
                swd[t] = *reinterpret_cast<const uint32_t *>(cb + ((wave * kTW + t) * 2 + 0) * 256 + lane * 4);
                mwd[t] = *reinterpret_cast<const uint32_t *>(cb + ((wave * kTW + t) * 2 + 1) * 256 + lane * 4);
            }
            sc[t] = __uint_as_float((st & 1) ? (swd[t] & 0xFFFF0000u) : (swd[t] << 16));
            const float mv = __uint_as_float((st & 1) ? (mwd[t] & 0xFFFF0000u) : (mwd[t] << 16));
            cm[t] = fmaf(-128.f, sc[t], mv);
        }
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            if (tb >= ntb) break;  // token blocks past the tile's slots (uniform)
            const int r = tb * 16 + n16;
            const unsigned char *xa = xb + ((r >> 2) * 64 + (r & 3) * 16) * 16;
            bf16x8 Aop[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) Aop[c] = *reinterpret_cast<const bf16x8 *>(xa + (((g * 4 + c) ^ n16) * 16));
            const float4 xv = *reinterpret_cast<const float4 *>(&ss[st][tb * 16 + 4 * g]);
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
    };
    // One K step. Barriers are s_barrier with explicit waits (a __syncthreads() fence would wait for every
    // outstanding DMA, the next steps' included). Step k's DMA of this wave has landed once only the three later
    // issues are outstanding (VMEM completes in order); everyone's has after the barrier.
    auto step = [&](int k, auto st_tag) {
        constexpr int ST = decltype(st_tag)::value;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // everyone is done with step k - 1
        issue(k + kStages - 1, (ST + kStages - 1) % kStages);
        constexpr int kNewer = (ST & 1) ? 2 * kLoadsEven + kLoadsOdd : 2 * kLoadsOdd + kLoadsEven;  // issues k+1..k+3
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kNewer) : "memory");
        sum_spans(ST);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        compute(st_tag);
    };

    static_assert(kStages % 2 == 0, "stage parity follows step parity");
#pragma unroll
    for (int s = 0; s < kStages - 1; ++s) issue(s, s);
    // unrolled by the stage count so that the stages are constants (a full unroll hoists every load and spills)
    for (int k = 0;; k += kStages) {
        if (k >= nk) break;
        step(k, std::integral_constant<int, 0>{});
        if (k + 1 >= nk) break;
        step(k + 1, std::integral_constant<int, 1>{});
        if (k + 2 >= nk) break;
        step(k + 2, std::integral_constant<int, 2>{});
        if (k + 3 >= nk) break;
        step(k + 3, std::integral_constant<int, 3>{});
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clamped DMA past the end lands before the block exits

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
    return bits == 4 && G == 128 && K % (2 * kSpan) == 0 && K >= 2 * kSpan && act == SX_ACT_BF16;
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
