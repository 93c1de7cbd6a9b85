// Dense dequantizing GEMV at decode / verify width (M <= 16 activation rows): y[M, N] = x[M, K] . deq(W)^T for q4
// (G = 128) and q8 (G = 64), one quantization group a 16-byte-a-lane span (kernels/linear_q4.hpp:26-30,
// kernels/linear_q8.hpp:13-14), for the served shapes (4-64 spans a row) in place of qmm's dense mode (a wave a
// 16-row tile over the whole K, many tiles a CU in flight at once). A block a CU takes an equal run of the 16-row
// tiles (to within one tile), and its 8 waves split K Q ways (Q = min(8, spans / 4)) and work on 8 / Q tiles at a
// time, so every wave of the grid issues the same loads: SPW spans a round (4 or 8 loads of 1 KB), one round in
// flight, and a CU reads one tile's rows at a time (measured faster than more tiles in flight a CU). The activation
// rows sit in LDS once per block (BF16 x: one plane; FP32 x: three exact BF16 planes) in the B operand's code order
// with their span sums; each span folds as acc += s * D + (m - off * s) * sum x with D from
// v_mfma_f32_16x16x32_bf16 on (off + code). The Q partial 16 x 16 tiles of a tile meet in LDS after a barrier (Q > 1),
// are summed in K order and stored by the Q waves that made them (a quarter-tile or less each).
#include "dense_ks.hpp"
#include "qmm_impl.hpp"

#include <atomic>

namespace sx::dks {
namespace {

using qmm::detail::bf16x8;
using qmm::detail::f32x4;

constexpr int kThreads = 512, kWaves = 8;
constexpr int kSpanBytes = 64;  // a row's span: 16 bytes a lane, 4 lanes
// One round of loads in flight a wave, and a slot's reload going out kLag slots after its unpack (2 of 4, 6 of 8):
// fewer requests in flight a CU measured faster (config 1 12.0 -> 8.6 us, the q8 LM head 139 -> 126 us).
constexpr int kRingKs = 1;
template <int SPW> constexpr int kLagKs = SPW == 8 ? 6 : 2;

// The BF16 word of span s in a window of 4 (uint2) or 8 (uint4) scales / mins.
__device__ __forceinline__ uint32_t win_word(const uint2 &w, int s) { return s < 2 ? w.x : w.y; }
__device__ __forceinline__ uint32_t win_word(const uint4 &w, int s) { return qmm::detail::dword(w, s >> 1); }

template <int BITS, int NPL, int SPW, typename TX, typename TY>
__global__ void __launch_bounds__(kThreads) dense_ks_kernel(Params p) {
    using F = qmm::detail::Fmt<BITS>;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    __shared__ __attribute__((aligned(16))) float red[2][kWaves][4][64];  // [round & 1][wave][v][lane]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = p.M, Q = p.Q, P = kWaves / Q;
    const int ip = wave / Q, kq = wave % Q;  // tile lane, K slice (spans SPW kq ..)
    const int64_t K = p.K, N = p.N, ldx = K + 8;
    const int nspan = (int)(K / F::kSpanCodes), chunks8 = (int)(K / 8), lg_chunks = __builtin_ctz((unsigned)chunks8);
    const int n16 = lane & 15, g = lane >> 4;
    uint16_t *xs = reinterpret_cast<uint16_t *>(smem);                      // [NPL][M][K + 8]
    float *xsum = reinterpret_cast<float *>(smem + (size_t)NPL * M * ldx * 2);  // [nspan][16]

    // this block's tiles [b0, b1), in rounds of P
    const int64_t T16 = (N + 15) / 16;
    const int b0 = (int)(blockIdx.x * T16 / gridDim.x), b1 = (int)((blockIdx.x + 1) * T16 / gridDim.x);
    const int groups = (b1 - b0 + P - 1) / P;

    // weight ring: round r = the slice kq of tile b0 + r P + ip (clamped into the run: a clamped round loads a
    // valid tile and stores nothing); the round's scales / mins as one window of SPW BF16 a row
    using Win = std::conditional_t<SPW == 4, uint2, uint4>;
    const int64_t rowbytes = K * BITS / 8, ngroups = nspan;
    uint4 ring[kRingKs][SPW];
    Win sw_n[kRingKs], mw_n[kRingKs];
    int ii = 0;
    const uint8_t *iq = p.q;
    const uint16_t *is_ = p.scale, *im = p.minv;
    auto iplace = [&]() {
        const int tile = min(b0 + ii * P + ip, b1 - 1);
        const int64_t n = (int64_t)tile * 16 + n16, row = n < N ? n : N - 1;
        iq = p.q + row * rowbytes + (int64_t)kq * SPW * kSpanBytes + g * 16;
        is_ = p.scale + row * ngroups + kq * SPW;
        im = p.minv + row * ngroups + kq * SPW;
    };
    auto advance_issue = [&]() {
        ++ii;
        iplace();
    };
    auto issue_window = [&](Win &sw, Win &mw) {
        sw = *reinterpret_cast<const Win *>(is_);
        mw = *reinterpret_cast<const Win *>(im);
    };
    auto issue_slot = [&](uint4 (&slot)[SPW], int s) {
        slot[s] = *reinterpret_cast<const uint4 *>(iq + (int64_t)s * kSpanBytes);
    };

    // 1. activation loads first (a chunk of 8 a thread a pass), then the first two rounds of weights, then the
    // staging into LDS: the staging waits for the activations only
    constexpr int kStage = 8;
    const int n_items_x = M * chunks8;
    const TX *x = static_cast<const TX *>(p.x);
    qmm::detail::Raw8<TX> raw[kStage];
    auto load_x = [&](int base) __attribute__((always_inline)) {
#pragma unroll
        for (int b = 0; b < kStage; ++b) {
            const int i = min(base + b * kThreads + tid, n_items_x - 1);
            raw[b] = qmm::detail::load_raw8<TX>(x + (int64_t)(i >> lg_chunks) * K + (int64_t)(i & (chunks8 - 1)) * 8);
        }
    };
    auto stage_x = [&](int base) __attribute__((always_inline)) {
#pragma unroll
        for (int b = 0; b < kStage; ++b) {
            const int i = base + b * kThreads + tid;
            if (i < n_items_x) {  // a span's chunks (16 q4 / 8 q8) are all in or all out
                const int r = i >> lg_chunks, c8 = i & (chunks8 - 1);
                uint4 planes[NPL];
                float sum;
                qmm::detail::chunk_planes<BITS, NPL, TX>(raw[b], planes, sum);
#pragma unroll
                for (int s = 0; s < NPL; ++s)
                    *reinterpret_cast<uint4 *>(xs + ((int64_t)s * M + r) * ldx + (int64_t)c8 * 8) = planes[s];
                constexpr int CPS = F::kSpanCodes / 8;  // chunks a span
                sum = qmm::detail::group_sum_c<CPS>(sum);
                if ((c8 & (CPS - 1)) == 0) xsum[(c8 / CPS) * 16 + r] = sum;
            }
        }
    };
    load_x(0);
    if (groups > 0) {
        __builtin_amdgcn_sched_barrier(0);
        iplace();
#pragma unroll
        for (int r = 0; r < kRingKs; ++r) {
            if (r > 0) advance_issue();  // unconditional (iplace clamps): a branch would copy the ring behind a full wait
            issue_window(sw_n[r], mw_n[r]);
#pragma unroll
            for (int s = 0; s < SPW; ++s) issue_slot(ring[r], s);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int base = 0;; base += kStage * kThreads) {
        stage_x(base);
        if (base + kStage * kThreads >= n_items_x) break;
        load_x(base + kStage * kThreads);
    }
    for (int i = tid; i < nspan * 16; i += kThreads)
        if ((i & 15) >= M) xsum[i] = 0.f;
    __syncthreads();
    if (groups <= 0) return;

    // 2. consume: A rows = activation rows (lane row n16, zeros past M), D rows 4g .. 4g + 3, columns = the tile's rows
    const bool a_on = n16 < M;
    const uint16_t *a_row = xs + (int64_t)(a_on ? n16 : 0) * ldx + g * (F::kSpanCodes / 4) + (int64_t)kq * SPW * F::kSpanCodes;
    const float *xsg = xsum + kq * SPW * 16 + 4 * g;
    // the D rows 4 g + vb .. whose results this wave stores (Q = 8: on half the lanes)
    const int VS = Q >= 4 ? 1 : 4 / Q;
    const int vb = Q == 8 ? kq >> 1 : kq * VS;
    const bool st_lane = Q != 8 || (g & 1) == (kq & 1);
    auto store = [&](int tile, int v, float val) __attribute__((always_inline)) {
        const int r = 4 * g + v;
        const int64_t n = (int64_t)tile * 16 + n16;
        if (r < M && n < N) store_act(static_cast<TY *>(p.y), (int64_t)r * N + n, val);
    };
    auto consume = [&](int gr, auto slot_tag) __attribute__((always_inline)) {
        constexpr int RS = decltype(slot_tag)::value;
        const Win sw = sw_n[RS], mw = mw_n[RS];
        if (gr + kRingKs < groups) advance_issue();
        issue_window(sw_n[RS], mw_n[RS]);
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < SPW; ++s) {
            bf16x8 bop[F::kMfmas];  // unpacked before the reload is issued: the slot's register is then free for it
#pragma unroll
            for (int t = 0; t < F::kMfmas; ++t) bop[t] = qmm::detail::codes_b<BITS>(ring[RS][s], t);
            if (s >= kLagKs<SPW>) issue_slot(ring[RS], s - kLagKs<SPW>);
            f32x4 D = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
                for (int t = 0; t < F::kMfmas; ++t) {
                    const bf16x8 av = a_on ? *reinterpret_cast<const bf16x8 *>(a_row + (int64_t)pl * M * ldx + s * F::kSpanCodes + t * 8)
                                           : bf16x8{};
                    D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bop[t], D, 0, 0, 0);
                }
            const float4 xv = *reinterpret_cast<const float4 *>(xsg + s * 16);
            const uint32_t swd = win_word(sw, s), mwd = win_word(mw, s);
            const float s_ = __uint_as_float((s & 1) ? (swd & 0xFFFF0000u) : (swd << 16));
            const float m_ = __uint_as_float((s & 1) ? (mwd & 0xFFFF0000u) : (mwd << 16));
            const float cm = fmaf(-F::kOff, s_, m_);
            acc[0] = fmaf(s_, D[0], fmaf(cm, xv.x, acc[0]));
            acc[1] = fmaf(s_, D[1], fmaf(cm, xv.y, acc[1]));
            acc[2] = fmaf(s_, D[2], fmaf(cm, xv.z, acc[2]));
            acc[3] = fmaf(s_, D[3], fmaf(cm, xv.w, acc[3]));
        }
#pragma unroll
        for (int s = SPW - kLagKs<SPW>; s < SPW; ++s) issue_slot(ring[RS], s);
        if (gr >= groups) return;  // the phantom round
        const int tile = b0 + gr * P + ip;
        if (Q == 1) {
            if (tile < b1)
#pragma unroll
                for (int v = 0; v < 4; ++v) store(tile, v, acc[v]);
            return;
        }
        float(&mine)[4][64] = red[gr & 1][wave];
#pragma unroll
        for (int v = 0; v < 4; ++v) mine[v][lane] = acc[v];
        // every wave's partial tile of this round is in LDS (the loads in flight stay in flight); the next write to
        // this half of red comes after the next round's barrier, when these reads are done
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (tile < b1 && st_lane) {
            for (int j = 0; j < VS; ++j) {
                float sum = 0.f;
                for (int qq = 0; qq < Q; ++qq) sum += red[gr & 1][ip * Q + qq][vb + j][lane];  // K order
                store(tile, vb + j, sum);
            }
        }
    };
    // Runs of two rounds, all issuing their loads (an odd count ends with a phantom round that re-loads the last one
    // and stops after its MFMAs): a consume whose loads were conditional would merge two versions of the ring
    // registers, and the copies at such a merge wait for every outstanding load.
    for (int gr = 0; gr < groups; gr += kRingKs)
        [&]<int... RS>(std::integer_sequence<int, RS...>) {
            (consume(gr + RS, std::integral_constant<int, RS>{}), ...);
        }(std::make_integer_sequence<int, kRingKs>{});
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the phantom round's loads land before the wave exits
}

template <int BITS, int NPL, int SPW, typename TX, typename TY>
hipError_t go(const Params &p, int cus, size_t lds, hipStream_t stream) {
    auto fn = dense_ks_kernel<BITS, NPL, SPW, TX, TY>;
    // the dynamic LDS limit, set once an instantiation (every launch asks for <= kLdsMax; setting it twice from two
    // threads is harmless)
    static std::atomic<bool> sized{false};
    if (!sized.load(std::memory_order_acquire)) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(fn),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsMax);
        if (e != hipSuccess) return e;
        sized.store(true, std::memory_order_release);
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)cus), dim3(kThreads), lds, stream, p);
    return hipGetLastError();
}

}  // namespace

size_t lds_bytes(int act, int64_t M, int64_t K, int bits) {
    const int npl = act == SX_ACT_F32 ? 3 : 1;
    const int64_t nspan = K / (bits == 4 ? 128 : 64);
    return (size_t)npl * M * (K + 8) * 2 + (size_t)nspan * 16 * 4;
}

bool eligible(int bits, int64_t G, int64_t N, int64_t K, int64_t M, int act, int out_act, int cus) {
    (void)N, (void)cus;  // any number of tiles: a block takes a run of them
    if (!((bits == 4 && G == 128) || (bits == 8 && G == 64))) return false;
    const int64_t span = bits == 4 ? 128 : 64;
    if (K % span != 0) return false;
    const int64_t nspan = K / span;
    if (!(nspan == 4 || nspan == 8 || nspan == 16 || nspan == 32 || nspan == 64)) return false;
    if (M < 1 || M > 16) return false;
    if (!((act == SX_ACT_BF16 && (out_act == SX_ACT_BF16 || out_act == SX_ACT_F32)) ||
          (act == SX_ACT_F32 && out_act == SX_ACT_F32)))
        return false;
    return lds_bytes(act, M, K, bits) <= kLdsMax;
}

hipError_t launch(int bits, int act, int out_act, const Params &p0, int cus, hipStream_t stream) {
    Params p = p0;
    const int64_t nspan = p.K / (bits == 4 ? 128 : 64);
    p.Q = (int)(nspan / 4 < kWaves ? nspan / 4 : kWaves);
    const int spw = (int)(nspan / p.Q);
    const size_t lds = lds_bytes(act, p.M, p.K, bits);
    auto by_spw = [&](auto bits_tag, auto npl_tag, auto tx, auto ty) {
        constexpr int B = decltype(bits_tag)::value, NPL = decltype(npl_tag)::value;
        using TX = decltype(tx);
        using TY = decltype(ty);
        return spw == 4 ? go<B, NPL, 4, TX, TY>(p, cus, lds, stream) : go<B, NPL, 8, TX, TY>(p, cus, lds, stream);
    };
    auto by_act = [&](auto bits_tag) {
        if (act == SX_ACT_F32) return by_spw(bits_tag, std::integral_constant<int, 3>{}, float{}, float{});
        if (out_act == SX_ACT_F32) return by_spw(bits_tag, std::integral_constant<int, 1>{}, uint16_t{}, float{});
        return by_spw(bits_tag, std::integral_constant<int, 1>{}, uint16_t{}, uint16_t{});
    };
    return bits == 4 ? by_act(std::integral_constant<int, 4>{}) : by_act(std::integral_constant<int, 8>{});
}

}  // namespace sx::dks
