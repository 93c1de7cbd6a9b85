// Dense dequantizing GEMV at decode / verify width (M <= 16 activation rows): y[M, N] = x[M, K] . deq(W)^T for q4
// (G = 128 or 64) and q8 (G = 64), one or two quantization groups a 16-byte-a-lane span (kernels/linear_q4.hpp:26-30,
// kernels/linear_q8.hpp:13-14), for the served shapes (4-64 spans a row) in place of qmm's dense mode (a wave a
// 16-row tile over the whole K, many tiles a CU in flight at once). A block a CU takes an equal share of the 16-row
// tiles (to within one tile; every G-th tile), and its 8 waves split K Q ways (Q = min(8, spans / 4)) and work on 8 / Q tiles at a
// time, so every wave of the grid issues the same loads: SPW spans a round (4 or 8 loads of 1 KB), one round in
// flight, and a CU reads one tile's rows at a time (measured faster than more tiles in flight a CU). The activation
// rows sit in LDS once per block (BF16 x: one plane; FP32 x: three exact BF16 planes) in the B operand's code order
// with their span sums; each span folds as acc += s * D + (m - off * s) * sum x with D from
// v_mfma_f32_16x16x32_bf16 on (off + code). The Q partial 16 x 16 tiles of a tile meet in LDS after a barrier (Q > 1),
// are summed in K order and stored by the Q waves that made them (a quarter-tile or less each).
// Each plane has a zero row after the M activation rows: the A-operand lanes past M read it, so every A read is an
// unconditional LDS load (a select of the read against zeros made each read wait for the one before it).
// q4 G = 64 (the MTP draft head) has two groups a span: a span's lanes 0-31 hold the first group's codes and lanes
// 32-63 the second's, so each MFMA runs twice, once with the other group's lanes reading the zero row instead of the
// activations (no ALU selects), and each group folds with its own scale, min and x sums.
// PICK (the MTP draft head, FP32 logits, M = 1): each thread keeps the running top-2 of the logits it stores (its
// indices ascend: its tiles do), and the blocks merge them at the end as pick::block_pick does, so the pick needs no
// launch and no second read of the logits of its own.
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

// The dword holding BF16 word s of a window of 4 (uint2), 8 (uint4) or 16 (Win16) scales / mins.
struct Win16 {
    uint4 a, b;
};
__device__ __forceinline__ uint32_t win_word(const uint2 &w, int s) { return s < 2 ? w.x : w.y; }
__device__ __forceinline__ uint32_t win_word(const uint4 &w, int s) { return qmm::detail::dword(w, s >> 1); }
__device__ __forceinline__ uint32_t win_word(const Win16 &w, int s) {
    return s < 8 ? qmm::detail::dword(w.a, s >> 1) : qmm::detail::dword(w.b, (s - 8) >> 1);
}
__device__ __forceinline__ float win_value(uint32_t dw, int s) {
    return __uint_as_float((s & 1) ? (dw & 0xFFFF0000u) : (dw << 16));
}

template <int BITS, int NPL, int SPW, int GS, typename TX, typename TY, bool PICK>
__global__ void __launch_bounds__(kThreads) dense_ks_kernel(Params p) {
    static_assert(GS == 1 || (GS == 2 && BITS == 4), "two groups a span: q4 G = 64");
    static_assert(!PICK || std::is_same_v<TY, float>, "the pick takes FP32 logits");
    __shared__ pick::Top2 pick_red[PICK ? kWaves : 1];
    __shared__ int pick_last;
    pick::Top2 pk = pick::top2_none();
    pick::ErrWords pk_errs{};
    if constexpr (PICK)
        pk_errs = pick::read_errs(threadIdx.x, p.pick.router_err, p.pick.expert_err, p.pick.attn_err, p.pick.emb_err);
    using F = qmm::detail::Fmt<BITS>;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    __shared__ __attribute__((aligned(16))) float red[2][kWaves][4][64];  // [round & 1][wave][v][lane]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Q is a power of two (1 .. 8): shifts and masks, not divisions
    const int M = p.M, Q = p.Q, lg_q = __builtin_ctz((unsigned)Q), P = kWaves >> lg_q;
    const int ip = wave >> lg_q, kq = wave & (Q - 1);  // tile lane, K slice (spans SPW kq ..)
    const int64_t K = p.K, N = p.N, ldx = K + 8;
    const int nspan = (int)(K / F::kSpanCodes), chunks8 = (int)(K / 8), lg_chunks = __builtin_ctz((unsigned)chunks8);
    const int n16 = lane & 15, g = lane >> 4;
    const int MP = M + 1;  // rows a plane (row M: zeros)
    uint16_t *xs = reinterpret_cast<uint16_t *>(smem);                       // [NPL][MP][K + 8]
    float *xsum = reinterpret_cast<float *>(smem + (size_t)NPL * MP * ldx * 2);  // [nspan * GS][16]

    // this block's tiles tile_of(j), j < ntile, in rounds of P: strided, blk + j G (the grid sweeps the rows
    // together: the q8 LM head 122 -> 119 us), else the run b0 + j (fewer tiles a block: config 2 q8 16.2 against
    // 17.3 us strided)
    // in 32-bit unsigned arithmetic (T16 * G < 2^32: the launch checks it): a 64-bit division by the grid size is a
    // long scalar sequence ahead of the first loads
    const unsigned T16 = (unsigned)((N + 15) / 16);
    const unsigned G = gridDim.x, blk = blockIdx.x;
    const bool strided = p.strided != 0;
    const int b0 = (int)(blk * T16 / G);
    const int ntile = strided ? (blk < T16 ? (int)((T16 - 1 - blk) / G + 1) : 0) : (int)((blk + 1) * T16 / G) - b0;
    const int groups = (ntile + P - 1) >> (3 - lg_q);
    auto tile_of = [&](int j) { return strided ? j * (int)G + (int)blk : b0 + j; };

    // weight ring: round r = the slice kq of tile tile_of(r P + ip) (clamped into the block's tiles: a clamped round
    // loads a valid tile and stores nothing); the round's scales / mins as one window of SPW BF16 a row
    using Win = std::conditional_t<SPW * GS == 4, uint2, std::conditional_t<SPW * GS == 8, uint4, Win16>>;
    const int64_t rowbytes = K * BITS / 8, ngroups = (int64_t)nspan * GS;
    uint4 ring[kRingKs][SPW];
    Win sw_n[kRingKs], mw_n[kRingKs];
    int ii = 0;
    const uint8_t *iq = p.q;
    const uint16_t *is_ = p.scale, *im = p.minv;
    auto iplace = [&]() {
        const int tile = tile_of(min(ii * P + ip, ntile - 1));
        const int64_t n = (int64_t)tile * 16 + n16, row = n < N ? n : N - 1;
        iq = p.q + row * rowbytes + (int64_t)kq * SPW * kSpanBytes + g * 16;
        is_ = p.scale + row * ngroups + kq * SPW * GS;
        im = p.minv + row * ngroups + kq * SPW * GS;
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
                    *reinterpret_cast<uint4 *>(xs + ((int64_t)s * MP + r) * ldx + (int64_t)c8 * 8) = planes[s];
                constexpr int CPG = F::kSpanCodes / 8 / GS;  // chunks a group
                sum = qmm::detail::group_sum_c<CPG>(sum);
                if ((c8 & (CPG - 1)) == 0) xsum[(c8 / CPG) * 16 + r] = sum;
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
    for (int i = tid; i < nspan * GS * 16; i += kThreads)
        if ((i & 15) >= M) xsum[i] = 0.f;
    for (int i = tid; i < NPL * (int)(ldx / 8); i += kThreads)  // the zero row of each plane
        *reinterpret_cast<uint4 *>(xs + ((int64_t)(i / (ldx / 8)) * MP + M) * ldx + (int64_t)(i % (ldx / 8)) * 8) =
            uint4{0u, 0u, 0u, 0u};
    __syncthreads();
    if (groups <= 0) {
        if constexpr (PICK) pick::block_pick<kWaves>(pk, p.pick, pk_errs, pick_red, &pick_last);
        return;
    }

    // 2. consume: A rows = activation rows (lane row n16, zeros past M), D rows 4g .. 4g + 3, columns = the tile's rows
    const bool a_on = n16 < M;
    const int64_t a_col = g * (F::kSpanCodes / 4) + (int64_t)kq * SPW * F::kSpanCodes;
    const uint16_t *a_zero = xs + (int64_t)M * ldx + a_col;
    const uint16_t *a_row = a_on ? xs + (int64_t)n16 * ldx + a_col : a_zero;
    // GS = 2: group 0's MFMAs read the activations on lanes 0-31 (its codes) and the zero row on lanes 32-63; group
    // 1's the other way round
    const uint16_t *a_g0 = g < 2 ? a_row : a_zero, *a_g1 = g < 2 ? a_zero : a_row;
    const float *xsg = xsum + kq * SPW * GS * 16 + 4 * g;
    // the D rows 4 g + vb .. whose results this wave stores (Q = 8: on half the lanes)
    const int VS = Q >= 4 ? 1 : 4 / Q;
    const int vb = Q == 8 ? kq >> 1 : kq * VS;
    const bool st_lane = Q != 8 || (g & 1) == (kq & 1);
    auto store = [&](int tile, int v, float val) __attribute__((always_inline)) {
        const int r = 4 * g + v;
        const int64_t n = (int64_t)tile * 16 + n16;
        if (r < M && n < N) {
            store_act(static_cast<TY *>(p.y), (int64_t)r * N + n, val);
            if constexpr (PICK)
                if (r == 0) pick::top2_take(pk, val, n);
        }
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
            f32x4 D[GS];
#pragma unroll
            for (int h = 0; h < GS; ++h) D[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
                for (int t = 0; t < F::kMfmas; ++t) {
                    const int64_t o = (int64_t)pl * MP * ldx + s * F::kSpanCodes + t * 8;
                    if constexpr (GS == 1) {
                        const bf16x8 av = *reinterpret_cast<const bf16x8 *>(a_row + o);
                        D[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bop[t], D[0], 0, 0, 0);
                    } else {
                        const bf16x8 a0 = *reinterpret_cast<const bf16x8 *>(a_g0 + o);
                        const bf16x8 a1 = *reinterpret_cast<const bf16x8 *>(a_g1 + o);
                        D[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bop[t], D[0], 0, 0, 0);
                        D[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bop[t], D[1], 0, 0, 0);
                    }
                }
#pragma unroll
            for (int h = 0; h < GS; ++h) {
                const int gi = s * GS + h;  // the group's index in the window
                const float4 xv = *reinterpret_cast<const float4 *>(xsg + gi * 16);
                const float s_ = win_value(win_word(sw, gi), gi), m_ = win_value(win_word(mw, gi), gi);
                const float cm = fmaf(-F::kOff, s_, m_);
                acc[0] = fmaf(s_, D[h][0], fmaf(cm, xv.x, acc[0]));
                acc[1] = fmaf(s_, D[h][1], fmaf(cm, xv.y, acc[1]));
                acc[2] = fmaf(s_, D[h][2], fmaf(cm, xv.z, acc[2]));
                acc[3] = fmaf(s_, D[h][3], fmaf(cm, xv.w, acc[3]));
            }
        }
#pragma unroll
        for (int s = SPW - kLagKs<SPW>; s < SPW; ++s) issue_slot(ring[RS], s);
        if (gr >= groups) return;  // the phantom round
        const int jt = gr * P + ip, tile = tile_of(jt);
        if (Q == 1) {
            if (jt < ntile)
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
        if (jt < ntile && st_lane) {
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
    if constexpr (PICK) pick::block_pick<kWaves>(pk, p.pick, pk_errs, pick_red, &pick_last);
}

template <int BITS, int NPL, int SPW, int GS, typename TX, typename TY, bool PICK = false>
hipError_t go(const Params &p, int cus, size_t lds, hipStream_t stream) {
    auto fn = dense_ks_kernel<BITS, NPL, SPW, GS, TX, TY, PICK>;
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

size_t lds_bytes(int act, int64_t M, int64_t K, int bits, int64_t G) {
    const int npl = act == SX_ACT_F32 ? 3 : 1;
    const int64_t span = bits == 4 ? 128 : 64, nspan = K / span, gs = span / G;
    return (size_t)npl * (M + 1) * (K + 8) * 2 + (size_t)nspan * gs * 16 * 4;
}

bool eligible(int bits, int64_t G, int64_t N, int64_t K, int64_t M, int act, int out_act, int cus) {
    // any number of tiles: a block takes a run of them (its range computed in 32 bits: tiles x blocks < 2^32)
    if (N < 1 || (N + 15) / 16 * (int64_t)(cus > 0 ? cus : 1) >= (int64_t(1) << 32)) return false;
    if (!((bits == 4 && (G == 128 || G == 64)) || (bits == 8 && G == 64))) return false;
    const int64_t span = bits == 4 ? 128 : 64;
    if (K % span != 0) return false;
    const int64_t nspan = K / span;
    if (!(nspan == 4 || nspan == 8 || nspan == 16 || nspan == 32 || nspan == 64)) return false;
    if (M < 1 || M > 16) return false;
    if (!((act == SX_ACT_BF16 && (out_act == SX_ACT_BF16 || out_act == SX_ACT_F32)) ||
          (act == SX_ACT_F32 && out_act == SX_ACT_F32)))
        return false;
    return lds_bytes(act, M, K, bits, G) <= kLdsMax;
}

hipError_t launch(int bits, int64_t G, int act, int out_act, const Params &p0, int cus, hipStream_t stream) {
    Params p = p0;
    const int64_t nspan = p.K / (bits == 4 ? 128 : 64);
    // 8 spans (8 KB) a wave a round when a block has at least two tiles for each round's 8 / Q tile lanes (the MTP
    // draft head: 49 against 51 us), else 4 spans a wave
    const int64_t tiles_per_block = ((p.N + 15) / 16 + cus - 1) / cus;
    const int64_t q8 = nspan / 8 < kWaves ? nspan / 8 : kWaves;
    if (nspan >= 8 && tiles_per_block >= 2 * (kWaves / q8)) p.Q = (int)q8;
    else p.Q = (int)(nspan / 4 < kWaves ? nspan / 4 : kWaves);
    const int spw = (int)(nspan / p.Q);
    p.strided = tiles_per_block >= 16 ? 1 : 0;
    const size_t lds = lds_bytes(act, p.M, p.K, bits, G);
    auto by_spw = [&](auto bits_tag, auto gs_tag, auto npl_tag, auto tx, auto ty) {
        constexpr int B = decltype(bits_tag)::value, GS = decltype(gs_tag)::value, NPL = decltype(npl_tag)::value;
        using TX = decltype(tx);
        using TY = decltype(ty);
        if (p.pick.ws != nullptr) {
            if constexpr (std::is_same_v<TY, float> && NPL == 1) {
                if (p.M != 1 || cus > pick::kMaxParts) return hipErrorInvalidValue;
                return spw == 4 ? go<B, NPL, 4, GS, TX, TY, true>(p, cus, lds, stream)
                                : go<B, NPL, 8, GS, TX, TY, true>(p, cus, lds, stream);
            } else {
                return hipErrorInvalidValue;  // the pick: BF16 x, FP32 logits
            }
        }
        return spw == 4 ? go<B, NPL, 4, GS, TX, TY>(p, cus, lds, stream) : go<B, NPL, 8, GS, TX, TY>(p, cus, lds, stream);
    };
    auto by_act = [&](auto bits_tag, auto gs_tag) {
        if (act == SX_ACT_F32) return by_spw(bits_tag, gs_tag, std::integral_constant<int, 3>{}, float{}, float{});
        if (out_act == SX_ACT_F32) return by_spw(bits_tag, gs_tag, std::integral_constant<int, 1>{}, uint16_t{}, float{});
        return by_spw(bits_tag, gs_tag, std::integral_constant<int, 1>{}, uint16_t{}, uint16_t{});
    };
    if (bits == 8) return by_act(std::integral_constant<int, 8>{}, std::integral_constant<int, 1>{});
    if (G == 64) return by_act(std::integral_constant<int, 4>{}, std::integral_constant<int, 2>{});
    return by_act(std::integral_constant<int, 4>{}, std::integral_constant<int, 1>{});
}

}  // namespace sx::dks
