// Verify-width MoE FFN in two launches after the router projection: the sequence runtime/qwen4exp.cpp:1139-1163
// runs below kGroupedMinTokens (moe_router, linear_q4_experts_gather_swiglu, linear_q4_experts_combine) with the
// same outputs, re-laid for one MI355X:
//
//   gate_up_kernel: every block routes all M tokens itself from the logits (routing::route_token, a wave a token;
//     M * k <= 64 slots, so this is a few microseconds and saves a launch plus the dependent workspace reads of a
//     separate grouping step), lists the distinct experts in id order with their token masks, stages all M
//     activation rows in LDS once, and takes an equal share of the (expert, 16-feature tile) items - equal per
//     wave to within one item, so every CU streams the same number of weight bytes. An item is one MFMA pass of
//     gate and up over all M tokens (the rows of a 16x16 MFMA tile cost the same filled or not); the epilogue
//     stores SwiGLU(gate, up) to the slots of the tokens routed to the expert. Block 0 also writes ids, coef and
//     the error words.
//   down_kernel: a block owns 16 output rows for all tokens, its 8 waves split the distinct experts, each expert's
//     tile is read once for all its tokens, and y[m] = sum_e coef[m, e] * (h[slot(m, e)] . W[e]) is summed per
//     wave in expert order, then across the waves in LDS in a fixed order: deterministic, no FP32 partials in
//     memory and no separate combine.
//
// Both stream their weight tiles like qmm_impl.hpp's fast path: a lane loads 16 code bytes a step (16 rows x one
// 64-byte span a wave) with the spans' scale / min windows, one round of loads in flight a wave (gate_up: 8 loads,
// down: 4; deeper rings measured slower: more requests in flight a CU lowered the HBM rate), and
// v_mfma_f32_16x16x32_bf16 on BF16 (128 + code) against the activations:
//   sum_k x * (code * s + m) = s * D + (m - 128 s) * sum_span x.
#include "qmm_impl.hpp"
#include "route_impl.hpp"
#include "verify_ffn.hpp"

namespace sx::vf {
namespace {

using qmm::detail::bf16x8;
using qmm::detail::f32x4;
using qmm::detail::kPrefetch;

constexpr int kThreads = 512, kWaves = 8;
constexpr int kLag = 2;  // a slot's reload goes out two slots after its unpack (fewer loads in flight: measured faster)
constexpr int kRing = 1;  // rounds of 8 loads in flight a wave (8 KB a wave, 64 KB a CU: measured faster than 2 or 3)
constexpr int kSpan = 128, kSpanBytes = 64;
constexpr int kLagDn = 2;  // down: a slot's reload two slots after its unpack
constexpr int kSpansDn = 4, kRingDn = 1;  // down: an item is 4 spans of a unit (4 loads a wave), one item in flight (2, 4 measured slower)
constexpr int kZeroBytes = qmm::detail::kZeroBytes;

struct Routes {                // one block's copy of the routing (LDS)
    int32_t ids[kMaxSlots];    // slot s = m * A + a
    float coef[kMaxSlots];
    int32_t u_exp[kMaxSlots];  // distinct valid experts, ascending
    uint32_t u_mask[kMaxSlots];  // their tokens (bit m)
    int U;
    uint64_t bad_slots;        // invalid slots: id outside [0, Ew) or repeated within its token
    int8_t slot_tab[kMaxSlots][kMaxTokens];  // [unit][token]: the token's slot of the unit's expert, or -1
};

// The distinct experts of the slots in id order with their token masks. bad_slots marks ids outside [0, Ew) and
// repeats of an id within a token (the routers never produce one; such a slot is treated as invalid: the later
// slot of the two). Wave 0 alone does it, from `id` = its lane's slot id (lane < S): the LDS operations of one wave
// take effect in program order, so no barrier is needed until the closing one. Lane t owns experts kPer t ..
// kPer t + kPer - 1: their token masks in four 16-byte reads, a wave prefix sum of the counts placing its units.
// emask: LDS [kMaxExperts], 16-byte aligned. Ends with an LDS-only block barrier.
__device__ void build_units(Routes &R, uint32_t *emask, int32_t id, int S, int A, int Ew) {
    constexpr int kPer = kMaxExperts / 64, kQuads = kPer / 4;
    static_assert(kPer % 4 == 0, "experts a lane: whole 16-byte words");
    static_assert(kMaxSlots * kMaxTokens == 64 * 16, "slot_tab: one 16-byte row a lane");
    const int t = threadIdx.x;
    if (t < 64) {
        uint4 *mine = reinterpret_cast<uint4 *>(emask) + t * kQuads;
#pragma unroll
        for (int q = 0; q < kQuads; ++q) mine[q] = uint4{0u, 0u, 0u, 0u};
        reinterpret_cast<int4 *>(&R.slot_tab[0][0])[t] = make_int4(-1, -1, -1, -1);
        const bool in = t < S;
        bool bad = in && !(id >= 0 && id < Ew);
        const uint32_t bit = in ? 1u << (t / A) : 0u;
        uint32_t old = 0u;
        if (in && !bad) old = atomicOr(&emask[id], bit);
        if (__ballot(old & bit)) {  // a repeat within a token: mark the later slots exactly
            for (int j = 1; j < A; ++j) {
                const int32_t o = __shfl(id, max(t - j, 0));
                bad |= in && t % A >= j && o == id;
            }
        }
        const uint64_t bad_mask = __ballot(bad);
        uint32_t mk[kPer];
#pragma unroll
        for (int q = 0; q < kQuads; ++q) {
            const uint4 w = mine[q];
            mk[4 * q] = w.x, mk[4 * q + 1] = w.y, mk[4 * q + 2] = w.z, mk[4 * q + 3] = w.w;
        }
        uint32_t c = 0u;
#pragma unroll
        for (int j = 0; j < kPer; ++j) c += mk[j] != 0u;
        const uint32_t incl = routing::wave_incl_scan_u32(c);
        int pos = (int)(incl - c);
#pragma unroll
        for (int j = 0; j < kPer; ++j)
            if (mk[j]) R.u_exp[pos] = kPer * t + j, R.u_mask[pos] = mk[j], emask[kPer * t + j] = (uint32_t)pos++;
        if (t == 63) R.U = (int)incl;
        if (t == 0) R.bad_slots = bad_mask;
        if (in && !bad) R.slot_tab[emask[id]][t / A] = (int8_t)t;
    }
    lds_barrier();  // the loads in flight (activations, weights) keep going
}

// ---------------------------------------------------------------------------------------------------------------
// gate_up + SwiGLU. A block takes an equal run of the (expert, 16-feature tile) items (to within one item of every
// other block); its 8 waves split K Q ways (Q = K / 512: four spans a wave) and take 8 / Q items a round, so every
// wave of the grid streams the same bytes: 8 loads a round (4 spans x gate, up), one round in flight. The Q partial
// tiles of an item are summed in LDS after a barrier (Q > 1), in K order, and the item's SwiGLU rows are stored by
// the Q waves that made them, a quarter-tile or less each. A wave's four spans of the M activation rows sit in its
// registers as MFMA A operands (code order) for the whole kernel, with their span sums. LDS (static): the partial
// tiles of two rounds, the routing.
template <int NV, int Q>
__global__ void __launch_bounds__(kThreads) gate_up_kernel(GateUpParams p) {
    constexpr int P = kWaves / Q;  // items a round
    __shared__ __attribute__((aligned(16))) float red[2][kWaves][2][4][64];  // [round & 1][wave][gate, up][v][lane]
    __shared__ Routes R;
    __shared__ __attribute__((aligned(16))) uint32_t emask[kMaxExperts];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ip = wave / Q, kq = wave % Q;  // item lane, K slice (spans 4 kq .. 4 kq + 3)
    const int M = p.M, A = p.A, S = M * A, Ew = p.Ew;
    const int64_t K = p.K;
    const int n16 = lane & 15, g = lane >> 4;

    // 1. this wave's logits (tokens wave and wave + 8, clamped: a redundant row past M), then its activations: A
    // operand (span so, MFMA t) of lane (n16, g) = x[n16][128 (4 kq + so) + 32 g + 8 t ..+ 7] in code order
    const float *row0 = p.logits + (int64_t)min(wave, M - 1) * p.ld, *row1 = p.logits + (int64_t)min(wave + kWaves, M - 1) * p.ld;
    float v0[NV], v1[NV];
    routing::load_logits<NV>([&](int e) { return row0[e]; }, p.E, v0);
    routing::load_logits<NV>([&](int e) { return row1[e]; }, p.E, v1);
    const float sl0 = p.shared_logit ? p.shared_logit[(int64_t)min(wave, M - 1) * p.shared_ld] : 0.f;
    const float sl1 = p.shared_logit ? p.shared_logit[(int64_t)min(wave + kWaves, M - 1) * p.shared_ld] : 0.f;
    uint4 xr[4][4];
    {
        const uint16_t *xrow = p.x + (int64_t)min(n16, M - 1) * K + (int64_t)kq * 4 * kSpan + g * 32;
#pragma unroll
        for (int so = 0; so < 4; ++so)
#pragma unroll
            for (int t = 0; t < 4; ++t) xr[so][t] = *reinterpret_cast<const uint4 *>(xrow + so * kSpan + t * 8);
    }

    // 2. routing, a wave a token (moe_router.hpp:11-23); only block 0 reports errors and writes ids / coef out
    const bool lead = blockIdx.x == 0;
    if (wave < M)
        routing::route_values<NV>(v0, p.E, p.k, p.shared_logit != nullptr, sl0, p.shared_id, wave, R.ids + wave * A,
                                  R.coef + wave * A, nullptr, lead ? p.router_err : nullptr);
    if (wave + kWaves < M)
        routing::route_values<NV>(v1, p.E, p.k, p.shared_logit != nullptr, sl1, p.shared_id, wave + kWaves,
                                  R.ids + (wave + kWaves) * A, R.coef + (wave + kWaves) * A, nullptr,
                                  lead ? p.router_err : nullptr);
    lds_barrier();
    build_units(R, emask, tid < S ? R.ids[tid] : 0, S, A, Ew);
    const int U = __builtin_amdgcn_readfirstlane(R.U);
    const int64_t Nrows = p.N / 2, rowbytes = K / 2, ngroups = K / kSpan;
    if (lead) {
        if (tid < S) p.ids[tid] = R.ids[tid], p.coef[tid] = R.coef[tid];
        uint64_t bad = R.bad_slots;  // invalid slots: error words (first slot wins) and NaN rows
        if (bad && tid == 0) {
            const int s = __builtin_ctzll(bad);
            flag_error(p.expert_err, (uint32_t)R.ids[s], (uint32_t)s);
        }
        while (bad) {
            const int s = __builtin_ctzll(bad);
            bad &= bad - 1;
            for (int64_t n = tid; n < Nrows; n += kThreads) p.h[s * Nrows + n] = (uint16_t)f32_to_bf16(qnan());
        }
    }

    // 3. this block's items [b0, b1) of U x T16 (expert-major), in rounds of P
    const int T16 = (int)((Nrows + 15) / 16);
    const int64_t F = (int64_t)U * T16;
    const int b0 = (int)(blockIdx.x * F / gridDim.x), b1 = (int)((blockIdx.x + 1) * F / gridDim.x);
    const int groups = (b1 - b0 + P - 1) / P;  // rounds (block-uniform)
    if (groups <= 0) return;

    // 4. weight ring: round r = the slice kq of item b0 + r P + ip (clamped into the run: a clamped round loads a
    // valid tile and stores nothing); gate and up alternate, scale / min windows of the 4 spans
    constexpr int NW = 2;
    const int64_t up_q = Nrows * rowbytes, up_g = Nrows * ngroups;
    uint4 ring[kRing][kPrefetch];
    uint2 sw_n[kRing][NW], mw_n[kRing][NW];
    int ii = 0;
    const uint8_t *iq = p.q;
    const uint16_t *is_ = p.scale, *im = p.minv;
    auto iplace = [&]() {
        const int item = min(b0 + ii * P + ip, b1 - 1);
        const int u = item / T16, tile = item - u * T16;
        const int64_t n = (int64_t)tile * 16 + n16, nn = n < Nrows ? n : Nrows - 1;
        const int64_t row = (int64_t)R.u_exp[u] * p.N + nn;
        iq = p.q + row * rowbytes + kq * 4 * kSpanBytes + g * 16;
        is_ = p.scale + row * ngroups + kq * 4;
        im = p.minv + row * ngroups + kq * 4;
    };
    auto advance_issue = [&]() {
        ++ii;
        iplace();
    };
    auto issue_window = [&](uint2 (&sw)[NW], uint2 (&mw)[NW]) {
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            sw[w] = *reinterpret_cast<const uint2 *>(is_ + (w ? up_g : 0));
            mw[w] = *reinterpret_cast<const uint2 *>(im + (w ? up_g : 0));
        }
    };
    auto issue_slot = [&](uint4 (&slot)[kPrefetch], int s) {
        const int span = s / NW, w = s % NW;
        slot[s] = *reinterpret_cast<const uint4 *>(iq + (w ? up_q : 0) + (int64_t)span * kSpanBytes);
    };
    __builtin_amdgcn_sched_barrier(0);
    iplace();
#pragma unroll
    for (int r = 0; r < kRing; ++r) {
        if (r > 0) advance_issue();  // unconditional (iplace clamps): a branch here would copy the ring behind a full wait
        issue_window(sw_n[r], mw_n[r]);
#pragma unroll
        for (int s = 0; s < kPrefetch; ++s) issue_slot(ring[r], s);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 5. the A operands (zero rows past M) and the span sums of the tokens of this lane's D rows 4 g + v
    bf16x8 aop[4][4];
    float xv[4][4];
#pragma unroll
    for (int so = 0; so < 4; ++so) {
        float sum = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint4 raw = n16 < M ? xr[so][t] : uint4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t d = qmm::detail::dword(raw, e);
                sum += __uint_as_float(d << 16) + __uint_as_float(d & 0xFFFF0000u);
            }
            aop[so][t] = __builtin_bit_cast(bf16x8, uint4{__builtin_amdgcn_perm(raw.z, raw.x, 0x05040100u),
                                                          __builtin_amdgcn_perm(raw.z, raw.x, 0x07060302u),
                                                          __builtin_amdgcn_perm(raw.w, raw.y, 0x05040100u),
                                                          __builtin_amdgcn_perm(raw.w, raw.y, 0x07060302u)});
        }
        sum += __shfl_xor(sum, 16);
        sum += __shfl_xor(sum, 32);
#pragma unroll
        for (int v = 0; v < 4; ++v) xv[so][v] = __shfl(sum, 4 * g + v);
    }

    // the D rows 4 g + vb .. 4 g + vb + VS - 1 whose SwiGLU this wave stores (Q = 8: on half the lanes)
    constexpr int VS = Q >= 4 ? 1 : 4 / Q;
    const int vb = Q == 8 ? kq >> 1 : kq * VS;
    const bool st_lane = Q != 8 || (g & 1) == (kq & 1);
    // Called by whole waves (the item is wave-uniform): the 16 lanes of a row (one g) hold the tile's 16 features
    // of token r, and their sum of the stored values is the slot's h_sums entry for the tile.
    auto epilogue = [&](int item, const float (&gate)[VS], const float (&up)[VS]) __attribute__((always_inline)) {
        const int u = item / T16, tile = item - u * T16;
        const uint32_t mask = R.u_mask[u];
        const int64_t n = (int64_t)tile * 16 + n16;
        const bool n_in = n < Nrows;
#pragma unroll
        for (int j = 0; j < VS; ++j) {
            const int r = 4 * g + vb + j;
            const bool on = st_lane && r < M && ((mask >> r) & 1u);  // uniform over the row of 16 lanes
            const float gv = as_bf16(gate[j]), uv = as_bf16(up[j]);
            const uint32_t hb = f32_to_bf16(as_bf16(silu(gv)) * uv);
            const int slot = on ? R.slot_tab[u][r] : 0;
            if (on && n_in) p.h[(int64_t)slot * Nrows + n] = (uint16_t)hb;
            if (p.h_sums) {
                const float ts = qmm::detail::group_sum_c<16>(n_in ? bf16_to_f32(hb) : 0.f);
                if (on && n16 == 0) p.h_sums[(int64_t)slot * T16 + tile] = ts;
            }
        }
    };

    // 6. consume: A rows = tokens (lane row n16), D rows 4g .. 4g + 3 = tokens, columns = the 16 features
    auto consume = [&](int gr, auto slot_tag) __attribute__((always_inline)) {
        constexpr int RS = decltype(slot_tag)::value;
        uint2 sw[NW], mw[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) sw[w] = sw_n[RS][w], mw[w] = mw_n[RS][w];
        if (gr + kRing < groups) advance_issue();
        issue_window(sw_n[RS], mw_n[RS]);
        float acc[NW][4] = {};
#pragma unroll
        for (int s = 0; s < kPrefetch; ++s) {
            const int w = s % NW, so = s / NW;
            bf16x8 bop[4];  // unpacked before the reload is issued: the slot's register is then free for it (a
                            // value still live there would make the loop rotate the ring behind a full wait)
#pragma unroll
            for (int t = 0; t < 4; ++t) bop[t] = qmm::detail::codes_b<4>(ring[RS][s], t);
            if (s >= kLag) issue_slot(ring[RS], s - kLag);
            f32x4 D = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; ++t) D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[so][t], bop[t], D, 0, 0, 0);
            const uint32_t swd = so < 2 ? sw[w].x : sw[w].y, mwd = so < 2 ? mw[w].x : mw[w].y;
            const float s_ = __uint_as_float((so & 1) ? (swd & 0xFFFF0000u) : (swd << 16));
            const float m_ = __uint_as_float((so & 1) ? (mwd & 0xFFFF0000u) : (mwd << 16));
            const float cm = fmaf(-128.f, s_, m_);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[w][v] = fmaf(s_, D[v], fmaf(cm, xv[so][v], acc[w][v]));
        }
#pragma unroll
        for (int s = kPrefetch - kLag; s < kPrefetch; ++s) issue_slot(ring[RS], s);
        if (gr >= groups) return;  // the phantom round
        const int item = b0 + gr * P + ip;
        if constexpr (Q == 1) {
            if (item < b1) epilogue(item, acc[0], acc[1]);
        } else {
            float(&mine)[2][4][64] = red[gr & 1][wave];
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int v = 0; v < 4; ++v) mine[w][v][lane] = acc[w][v];
            // every wave's partial tile of this round is in LDS (the loads in flight stay in flight); the next
            // write to this half of red comes after the next round's barrier, when these reads are done
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (item < b1) {
                float gate[VS] = {}, up[VS] = {};
#pragma unroll
                for (int qq = 0; qq < Q; ++qq) {  // K order
                    const float(&part)[2][4][64] = red[gr & 1][ip * Q + qq];
#pragma unroll
                    for (int j = 0; j < VS; ++j) gate[j] += part[0][vb + j][lane], up[j] += part[1][vb + j][lane];
                }
                epilogue(item, gate, up);
            }
        }
    };
    // Runs of kRing rounds, all issuing their loads (an odd count ends with a phantom round that re-loads the last
    // one and stops after its MFMAs): a consume whose loads were conditional would merge two versions of the ring
    // registers, and the copies at such a merge wait for every outstanding load.
    for (int gr = 0; gr < groups; gr += kRing)
        [&]<int... RS>(std::integer_sequence<int, RS...>) {
            (consume(gr + RS, std::integral_constant<int, RS>{}), ...);
        }(std::make_integer_sequence<int, kRing>{});
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the phantom round's loads land before the wave exits
}

// ---------------------------------------------------------------------------------------------------------------
// down + combine. LDS (static): the S slot rows of h [S][K + 8] BF16 (code order), span sums [S][K / 128], a zero
// block, the waves' partial sums [8][16 tokens][16 rows].
template <int NB, bool SUMS>
__global__ void __launch_bounds__(kThreads) down_kernel(DownParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t hs[kHsElems];
    __shared__ __attribute__((aligned(16))) float hsum[kMaxSlots * kMaxSpansDn];
    __shared__ __attribute__((aligned(16))) uint16_t zero_block[kZeroBytes / 2];
    __shared__ __attribute__((aligned(16))) float red[kWaves][16][16];
    __shared__ Routes R;
    __shared__ __attribute__((aligned(16))) uint32_t emask[kMaxExperts];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = p.M, A = p.A, S = M * A, Ew = p.Ew;
    const int64_t K = p.K, ldh = K + 8, N = p.N;
    const int nspan = (int)(K / kSpan), chunks8 = (int)(K / 8), lg_chunks = __builtin_ctz((unsigned)chunks8);
    const int n_items_x = S * chunks8;
    const int64_t n0 = (int64_t)blockIdx.x * 16;

    // the routing first, then the rows of h: the grouping waits for the ids only
    int32_t my_id;
    float my_coef;
    my_id = p.ids[min(lane, S - 1)], my_coef = p.coef[min(lane, S - 1)];  // every wave: no branch around loads
    constexpr int kSumLoads = SUMS ? (kMaxSlots * kMaxSpansDn + kThreads - 1) / kThreads : 0;
    float4 tsum[kSumLoads > 0 ? kSumLoads : 1][2];  // SUMS: the 8 tile sums of (slot, span) i = b * kThreads + tid
    if constexpr (SUMS) {
        const int tiles = (int)(K / 16);
#pragma unroll
        for (int b = 0; b < kSumLoads; ++b) {
            const int i = min(b * kThreads + tid, S * nspan - 1), r = i / nspan, sp = i - r * nspan;
            const float4 *src = reinterpret_cast<const float4 *>(p.h_sums + (int64_t)r * tiles + sp * 8);
            tsum[b][0] = src[0], tsum[b][1] = src[1];
        }
    }
    uint4 raw[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int i = min(b * kThreads + tid, n_items_x - 1);
        raw[b] = *reinterpret_cast<const uint4 *>(p.h + (int64_t)(i >> lg_chunks) * K + (int64_t)(i & (chunks8 - 1)) * 8);
    }
    R.ids[lane] = my_id, R.coef[lane] = my_coef;  // every wave the same values (unconditional: nothing sinks the loads)
    for (int i = tid; i < kZeroBytes / 4; i += kThreads) reinterpret_cast<uint32_t *>(zero_block)[i] = 0u;
    build_units(R, emask, my_id, S, A, Ew);  // its closing barrier also covers ids, coef and the zero block
    const int U = __builtin_amdgcn_readfirstlane(R.U);
    const uint64_t bad_slots = R.bad_slots;
    if (blockIdx.x == 0 && bad_slots && tid == 0) {
        const int s = __builtin_ctzll(bad_slots);
        flag_error(p.expert_err, (uint32_t)R.ids[s], (uint32_t)s);
    }

    const int64_t rowbytes = K / 2, ngroups = K / kSpan;
    const int n16 = lane & 15, g = lane >> 4;
    // items: (unit, chunk of 4 spans), unit-major; this wave's share [i0, i0 + groups), equal to within one item
    constexpr int SPG = kSpansDn;
    const int C = nspan / SPG, F = U * C;
    const int i0 = wave * F / kWaves, groups = (wave + 1) * F / kWaves - i0;
    uint4 ring[kRingDn][SPG];
    uint2 sw_n[kRingDn], mw_n[kRingDn];
    int ii = 0;
    const uint8_t *iq = p.q;
    const uint16_t *is_ = p.scale, *im = p.minv;
    auto iplace = [&]() {  // item i0 + ii, clamped into the items (or the first row when there are none)
        const int item = max(min(i0 + ii, F - 1), 0);
        const int u = item / C, c = item - u * C;
        const int64_t n = n0 + n16, nn = n < N ? n : N - 1;
        const int64_t row = (int64_t)(F > 0 ? R.u_exp[u] : 0) * N + nn;
        iq = p.q + row * rowbytes + c * SPG * kSpanBytes + g * 16;
        is_ = p.scale + row * ngroups + c * SPG;
        im = p.minv + row * ngroups + c * SPG;
    };
    auto advance_issue = [&]() {
        ++ii;
        iplace();
    };
    auto issue_window = [&](uint2 &sw, uint2 &mw) {
        sw = *reinterpret_cast<const uint2 *>(is_);
        mw = *reinterpret_cast<const uint2 *>(im);
    };
    auto issue_slot = [&](uint4 (&slot)[SPG], int s) {
        slot[s] = *reinterpret_cast<const uint4 *>(iq + (int64_t)s * kSpanBytes);
    };
    __builtin_amdgcn_sched_barrier(0);
    iplace();
#pragma unroll
    for (int r = 0; r < kRingDn; ++r) {
        if (r > 0) advance_issue();  // unconditional (iplace clamps): a branch here would copy the ring behind a full wait
        issue_window(sw_n[r], mw_n[r]);
#pragma unroll
        for (int s = 0; s < SPG; ++s) issue_slot(ring[r], s);
    }
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (SUMS) {  // h in code order; span sums = the 8 tile sums in tile order
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int i = b * kThreads + tid;
            if (i < n_items_x) {
                const int r = i >> lg_chunks, c8 = i & (chunks8 - 1);
                const uint4 w = raw[b];
                *reinterpret_cast<uint4 *>(hs + r * ldh + (int64_t)c8 * 8) =
                    uint4{__builtin_amdgcn_perm(w.z, w.x, 0x05040100u), __builtin_amdgcn_perm(w.z, w.x, 0x07060302u),
                          __builtin_amdgcn_perm(w.w, w.y, 0x05040100u), __builtin_amdgcn_perm(w.w, w.y, 0x07060302u)};
            }
        }
#pragma unroll
        for (int b = 0; b < kSumLoads; ++b) {
            const int i = b * kThreads + tid;
            if (i < S * nspan) {
                const float4 a = tsum[b][0], c = tsum[b][1];
                hsum[i] = ((((((a.x + a.y) + a.z) + a.w) + c.x) + c.y) + c.z) + c.w;
            }
        }
    } else {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int i = b * kThreads + tid;
            if (i < n_items_x) {
                const int r = i >> lg_chunks, c8 = i & (chunks8 - 1);
                uint4 planes[1];
                float sum;
                qmm::detail::chunk_planes<4, 1, uint16_t>(raw[b], planes, sum);
                *reinterpret_cast<uint4 *>(hs + r * ldh + (int64_t)c8 * 8) = planes[0];
                sum = qmm::detail::group_sum_c<16>(sum);
                if ((c8 & 15) == 0) hsum[r * nspan + (c8 >> 4)] = sum;
            }
        }
    }
    lds_barrier();  // the ring's weight loads stay in flight

    // consume: per item, A row n16 = token n16's slot of the unit's expert (or zeros); D rows 4g + v = tokens
    float yacc[4] = {0.f, 0.f, 0.f, 0.f};
    auto consume = [&](int gr, auto slot_tag) __attribute__((always_inline)) {
        constexpr int RS = decltype(slot_tag)::value;
        const uint2 sw = sw_n[RS], mw = mw_n[RS];
        if (gr + kRingDn < groups) advance_issue();
        issue_window(sw_n[RS], mw_n[RS]);
        const int item = max(min(i0 + gr, F - 1), 0);
        const int u = item / C, c0 = (item - u * C) * SPG;
        const int sa = R.slot_tab[u][n16];
        const uint16_t *ab = sa >= 0 ? hs + sa * ldh + g * 32 + c0 * kSpan : zero_block;
        const int a_step = sa >= 0 ? kSpan : 0;
        int sv[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) sv[v] = R.slot_tab[u][4 * g + v];
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            bf16x8 bop[4];  // unpacked before the reload is issued: the slot's register is then free for it (a
                            // value still live there would make the loop rotate the ring behind a full wait)
#pragma unroll
            for (int t = 0; t < 4; ++t) bop[t] = qmm::detail::codes_b<4>(ring[RS][s], t);
            if (s >= kLagDn) issue_slot(ring[RS], s - kLagDn);
            f32x4 D = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bf16x8 av = *reinterpret_cast<const bf16x8 *>(ab + s * a_step + t * 8);
                D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bop[t], D, 0, 0, 0);
            }
            const uint32_t swd = s < 2 ? sw.x : sw.y, mwd = s < 2 ? mw.x : mw.y;
            const float s_ = __uint_as_float((s & 1) ? (swd & 0xFFFF0000u) : (swd << 16));
            const float m_ = __uint_as_float((s & 1) ? (mwd & 0xFFFF0000u) : (mwd << 16));
            const float cm = fmaf(-128.f, s_, m_);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float xv = sv[v] >= 0 ? hsum[sv[v] * nspan + c0 + s] : 0.f;
                acc[v] = fmaf(s_, D[v], fmaf(cm, xv, acc[v]));
            }
        }
#pragma unroll
        for (int s = SPG - kLagDn; s < SPG; ++s) issue_slot(ring[RS], s);
        if (gr >= groups) return;  // a phantom item
#pragma unroll
        for (int v = 0; v < 4; ++v)
            if (sv[v] >= 0) yacc[v] = fmaf(R.coef[sv[v]], acc[v], yacc[v]);
    };
    // Runs of kRingDn items, all issuing their loads (a count short of a multiple ends with phantom items that
    // re-load the last one and stop after their MFMAs): a consume whose loads were conditional would merge two
    // versions of the ring registers, and the copies at such a merge wait for every outstanding load.
    for (int gr = 0; gr < groups; gr += kRingDn)
        [&]<int... RS>(std::integer_sequence<int, RS...>) {
            (consume(gr + RS, std::integral_constant<int, RS>{}), ...);
        }(std::make_integer_sequence<int, kRingDn>{});
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the phantom items' loads land before the wave exits

    // the waves' sums in wave order; tokens with an invalid slot get NaN rows (the combine's rule)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wave][4 * g + v][n16] = yacc[v];
    __syncthreads();
    if (tid < M * 16) {
        const int m = tid >> 4, c = tid & 15;
        const int64_t n = n0 + c;
        float y = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) y += red[w][m][c];
        bool bad = false;
        for (int a = 0; a < A; ++a) bad |= (bad_slots >> (m * A + a)) & 1ull;
        if (bad) y = qnan();
        if (n < N) {
            if (p.act == SX_ACT_F32) static_cast<float *>(p.y)[(int64_t)m * N + n] = y;
            else static_cast<uint16_t *>(p.y)[(int64_t)m * N + n] = (uint16_t)f32_to_bf16(y);
        }
    }
}

}  // namespace

hipError_t launch_gate_up(const GateUpParams &p, int cus, hipStream_t stream) {
    const int nv = p.E <= 256 ? 4 : p.E <= 512 ? 8 : 16;
    const int q = (int)(p.K / 512);  // K in {512, 1024, 2048, 4096}: four spans a wave
    const dim3 grid((unsigned)cus);
    auto go = [&](auto nv_tag, auto q_tag) {
        gate_up_kernel<decltype(nv_tag)::value, decltype(q_tag)::value><<<grid, kThreads, 0, stream>>>(p);
    };
    auto by_q = [&](auto nv_tag) {
        if (q == 1) go(nv_tag, std::integral_constant<int, 1>{});
        else if (q == 2) go(nv_tag, std::integral_constant<int, 2>{});
        else if (q == 4) go(nv_tag, std::integral_constant<int, 4>{});
        else go(nv_tag, std::integral_constant<int, 8>{});
    };
    if (nv == 4) by_q(std::integral_constant<int, 4>{});
    else if (nv == 8) by_q(std::integral_constant<int, 8>{});
    else by_q(std::integral_constant<int, 16>{});
    return hipGetLastError();
}

hipError_t launch_down(const DownParams &p, hipStream_t stream) {
    const int n_items = p.M * p.A * (int)(p.K / 8);
    const int nb = (n_items + kThreads - 1) / kThreads;
    const dim3 grid((unsigned)((p.N + 15) / 16));
    const bool sums = p.h_sums != nullptr;
    if (nb <= 4) sums ? down_kernel<4, true><<<grid, kThreads, 0, stream>>>(p) : down_kernel<4, false><<<grid, kThreads, 0, stream>>>(p);
    else if (nb <= 8) sums ? down_kernel<8, true><<<grid, kThreads, 0, stream>>>(p) : down_kernel<8, false><<<grid, kThreads, 0, stream>>>(p);
    else sums ? down_kernel<16, true><<<grid, kThreads, 0, stream>>>(p) : down_kernel<16, false><<<grid, kThreads, 0, stream>>>(p);
    return hipGetLastError();
}

}  // namespace sx::vf

using namespace sx;

namespace {

// The fused path's shape limits (all of them hold for the MTP verify layer: M <= 16, K = 4096, I = 1024).
int check_gate_up(const char *fn, int64_t M, int64_t A, int64_t E, int64_t k, int64_t Ew, const sx_qview *w, int act) {
    SX_CHECK(w != nullptr && w->q != nullptr && w->scale != nullptr && w->minv != nullptr, fn, " null weight view");
    SX_CHECK(act == SX_ACT_BF16, fn, " activations must be BF16 (got ", act, ")");
    SX_CHECK(M >= 1 && M <= vf::kMaxTokens && M * A <= vf::kMaxSlots, fn, " M = ", M, ", A = ", A, ": needs M <= ",
             vf::kMaxTokens, " and M * A <= ", vf::kMaxSlots);
    SX_CHECK(E >= 1 && k >= 1 && k <= E && Ew >= 1 && Ew <= vf::kMaxExperts, fn, " E = ", E, ", k = ", k, ", Ew = ", Ew);
    SX_CHECK(w->G == 128 && w->N % Ew == 0 && (w->N / Ew) % 2 == 0, fn, " gate_up view N = ", w->N, ", G = ", w->G,
             ": needs G = 128 and N a multiple of 2 Ew");
    const int64_t K = w->K;
    SX_CHECK(K == 512 || K == 1024 || K == 2048 || K == 4096, fn, " K = ", K, " does not fit the fused kernel");
    SX_CHECK(aligned(w->scale, 8) && aligned(w->minv, 8) && aligned(w->q, 16), fn, " weight arrays misaligned");
    return SX_OK;
}

int check_down(const char *fn, int64_t M, int64_t A, int64_t Ew, const sx_qview *w, int act) {
    SX_CHECK(w != nullptr && w->q != nullptr && w->scale != nullptr && w->minv != nullptr, fn, " null weight view");
    SX_CHECK(act == SX_ACT_BF16, fn, " activations must be BF16 (got ", act, ")");
    SX_CHECK(M >= 1 && M <= vf::kMaxTokens && A >= 1 && M * A <= vf::kMaxSlots, fn, " M = ", M, ", A = ", A,
             ": needs M <= ", vf::kMaxTokens, " and M * A <= ", vf::kMaxSlots);
    SX_CHECK(Ew >= 1 && Ew <= vf::kMaxExperts && w->N % Ew == 0, fn, " Ew = ", Ew, ", down view N = ", w->N);
    const int64_t K = w->K;
    SX_CHECK(w->G == 128 && (K == 1024 || K == 2048) && M * A * (K + 8) <= vf::kHsElems, fn, " K = ", K, ", G = ",
             w->G, " with M * A = ", M * A, " does not fit the fused kernel");
    SX_CHECK(aligned(w->scale, 16) && aligned(w->minv, 16) && aligned(w->q, 16), fn, " weight arrays misaligned");
    return SX_OK;
}

}  // namespace

extern "C" {

int sx_moe_verify_supported(int64_t M, int64_t A, int64_t E, int64_t k, int64_t Ew, const sx_qview *gate_up,
                            const sx_qview *down, int act) {
    if (int rc = check_gate_up("sx_moe_verify_supported", M, A, E, k, Ew, gate_up, act)) return rc;
    if (int rc = check_down("sx_moe_verify_supported", M, A, Ew, down, act)) return rc;
    SX_CHECK(down->K == gate_up->N / Ew / 2, "down K = ", down->K, " is not the gate_up I = ", gate_up->N / Ew / 2);
    return SX_OK;
}

int sx_moe_verify_gate_up(const void *x, int64_t M, const float *logits, int64_t ld, int64_t E, int64_t k,
                          const float *shared_logit, int64_t shared_ld, int32_t shared_id, const sx_qview *w, int64_t Ew,
                          int32_t *ids, float *coef, void *h, float *h_sums, int act, uint32_t *router_err,
                          uint32_t *expert_err, sx_stream stream) {
    const char *fn = "sx_moe_verify_gate_up";
    const int64_t A = k + (shared_logit ? 1 : 0);
    SX_CHECK(x != nullptr && logits != nullptr && ids != nullptr && coef != nullptr && h != nullptr &&
                 router_err != nullptr && expert_err != nullptr,
             fn, " null pointer");
    if (int rc = check_gate_up(fn, M, A, E, k, Ew, w, act)) return rc;
    SX_CHECK(ld >= E && (shared_logit == nullptr || shared_ld >= 1), fn, " ld = ", ld, ", shared_ld = ", shared_ld);
    SX_CHECK(aligned(x, 16) && aligned(h, 2), fn, " x must be 16-byte aligned");
    const int64_t I = w->N / Ew / 2;
    SX_CHECK(apart(h, M * A * I * 2, x, M * w->K * 2), fn, " h overlaps x");
    SX_CHECK(h_sums == nullptr || (aligned(h_sums, 16) && apart(h_sums, M * A * ((I + 15) / 16) * 4, h, M * A * I * 2)), fn,
             " h_sums must be 16-byte aligned and apart from h");
    vf::GateUpParams p{};
    p.x = static_cast<const uint16_t *>(x), p.M = (int)M, p.A = (int)A, p.k = (int)k, p.E = (int)E, p.Ew = (int)Ew;
    p.logits = logits, p.ld = ld, p.shared_logit = shared_logit, p.shared_ld = shared_ld, p.shared_id = shared_id;
    p.q = w->q, p.scale = w->scale, p.minv = w->minv, p.N = w->N / Ew, p.K = w->K;
    p.ids = ids, p.coef = coef, p.h = static_cast<uint16_t *>(h), p.h_sums = h_sums, p.router_err = router_err, p.expert_err = expert_err;
    SX_HIP(vf::launch_gate_up(p, device_cus(), stream_of(stream)), fn);
    return SX_OK;
}

int sx_moe_verify_down(const void *h, const float *h_sums, int64_t M, int64_t A, const int32_t *ids, const float *coef,
                       const sx_qview *w, int64_t Ew, void *y, int act, uint32_t *expert_err, sx_stream stream) {
    const char *fn = "sx_moe_verify_down";
    SX_CHECK(h != nullptr && ids != nullptr && coef != nullptr && y != nullptr && expert_err != nullptr, fn,
             " null pointer");
    if (int rc = check_down(fn, M, A, Ew, w, act)) return rc;
    SX_CHECK(aligned(h, 16) && aligned(h_sums, 16), fn, " h and h_sums must be 16-byte aligned");
    const int64_t N = w->N / Ew;
    SX_CHECK(apart(y, M * N * 2, h, M * A * w->K * 2), fn, " y overlaps h");
    vf::DownParams p{};
    p.h = static_cast<const uint16_t *>(h), p.h_sums = h_sums, p.M = (int)M, p.A = (int)A, p.Ew = (int)Ew, p.ids = ids, p.coef = coef;
    p.q = w->q, p.scale = w->scale, p.minv = w->minv, p.N = N, p.K = w->K, p.y = y, p.act = act;
    p.expert_err = expert_err;
    SX_HIP(vf::launch_down(p, stream_of(stream)), fn);
    return SX_OK;
}

}  // extern "C"
