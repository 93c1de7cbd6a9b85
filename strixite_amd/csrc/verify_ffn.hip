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

#include <atomic>
#include <mutex>
#include <unordered_map>

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
// A block's routing as gate_up hands it to down: the Routes bytes, copied 16 bytes a thread.
static_assert(sizeof(Routes) % 16 == 0 && sizeof(Routes) <= SX_VERIFY_PLAN_BYTES, "the plan holds a Routes");
constexpr int kPlanQuads = (int)(sizeof(Routes) / 16);
static_assert(kPlanQuads <= kThreads, "one 16-byte copy a thread");

// The distinct experts of the slots in id order with their token masks. bad_slots marks ids outside [0, Ew) and
// repeats of an id within a token (the routers never produce one; such a slot is treated as invalid: the later
// slot of the two). Wave 0 alone does it, from `id` = its lane's slot id (lane < S): the LDS operations of one wave
// take effect in program order, so no barrier is needed until the closing one. Every LDS access is conflict-free:
// the token-mask table is cleared and read a 64-expert row at a time (lane l: expert 64 q + l), each row's present
// experts form a ballot, and a unit's index is the count of present experts before it (the earlier rows' counts, a
// scalar running sum, plus the lane's rank in its row's ballot); only present experts write their unit.
// emask: LDS [kMaxExperts], 16-byte aligned. Ends with an LDS-only block barrier.
__device__ void build_units(Routes &R, uint32_t *emask, int32_t id, int S, int A, int Ew) {
    constexpr int kRows = kMaxExperts / 64;
    static_assert(kMaxSlots * kMaxTokens == 64 * 16, "slot_tab: one 16-byte row a lane");
    const int t = threadIdx.x;
    if (t < 64) {
#pragma unroll
        for (int q = 0; q < kRows / 4; ++q) reinterpret_cast<uint4 *>(emask)[q * 64 + t] = uint4{0u, 0u, 0u, 0u};
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
        uint32_t mk[kRows];
#pragma unroll
        for (int q = 0; q < kRows; ++q) mk[q] = emask[q * 64 + t];
        int base = 0;  // wave-uniform: units before row q
#pragma unroll
        for (int q = 0; q < kRows; ++q) {
            const uint64_t present = __ballot(mk[q] != 0u);
            if (mk[q] != 0u) {
                const int pos = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(present >> 32),
                                                                      __builtin_amdgcn_mbcnt_lo((uint32_t)present, 0u));
                R.u_exp[pos] = q * 64 + t, R.u_mask[pos] = mk[q], emask[q * 64 + t] = (uint32_t)pos;
            }
            base += __popcll(present);
        }
        if (t == 0) R.U = base, R.bad_slots = bad_mask;
        if (in && !bad) R.slot_tab[emask[id]][t / A] = (int8_t)t;
    }
    lds_barrier();  // the loads in flight (activations, weights) keep going
}

// ---------------------------------------------------------------------------------------------------------------
// Cross-block hand-offs of the one-launch layer (layer_kernel below). Its blocks pass the router logits, h and the
// h sums to each other through memory while the launch runs, across XCDs whose L2 caches are not coherent with each
// other: those values are written and read with agent-scope accesses (sc1: written through to, and read from, the
// level all XCDs share), and a block counts its contribution only after its own stores have completed.
__device__ __forceinline__ void store_agent(uint16_t *p, uint16_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_agent(const uint32_t *p) {
    return __hip_atomic_load(const_cast<uint32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_agent64(const uint64_t *p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes at byte offset off of an array of `bytes` bytes, agent scope (a buffer load with sc1).
__device__ __forceinline__ uint4 load16_agent(const void *base, uint32_t bytes, uint32_t off) {
    const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)off, 0, 16 /* sc1 */);
    return uint4{v[0], v[1], v[2], v[3]};
}

// The gate_up pool of a block: blocks 8j .. 8j + 7 (one on each XCD under the round-robin dispatch) share part
// j mod kQueues, so every part is served by the same mix of XCDs and the parts drain together.
__device__ __forceinline__ int queue_of(int block) { return (block >> 3) % kQueues; }
// The share of the gate_up items taken in fixed runs (the rest from the shared pool): kFixedNum / kFixedDen.
constexpr int kFixedNum = 4, kFixedDen = 5;

// One claim from a work counter by the calling lane. The zero offset comes from asm so the compiler cannot see
// that every lane names one address: it would otherwise merge the lanes' atomics into one and read its result out
// at once (readfirstlane), which waits for every load in flight; kept per lane, the wait lands where the result is
// used, at the end of the round.
__device__ __forceinline__ uint32_t claim_one(uint32_t *ctr) {
    uint32_t z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return atomicAdd(ctr + z, 1u);
}

// The one-launch layer's hand-off flags (LayerSync in verify_ffn.hpp): block b stores the launch's epoch into its
// slot of a phase once its part of that phase is complete (its own stores done), and a block that needs the phase
// complete waits until every slot holds the epoch. No counter is shared, so no block ever queues behind another's
// atomic; the host numbers the launches, so nothing needs resetting between them.
constexpr uint64_t kWaitTicks = 2000000;           // 20 ms of the 100 MHz s_memrealtime clock
constexpr uint32_t kWaitTimeoutCode = 0xFFFFFFFEu;  // expert_err word 1 after a wait gave up (word 2: the phase)

// Every thread's own stores are complete, then thread 0 publishes the block's flag.
__device__ __forceinline__ void block_publish(uint32_t *slot, uint32_t epoch) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(slot, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave 0 waits until flags[0 .. n) all hold epoch (n <= kMaxBlocks), or gives up after kWaitTicks and reports it;
// the block learns the outcome through `flag` (LDS) after an LDS-only barrier (the loads already in flight, such
// as the next weights, stay in flight). Every access after it comes after the wait.
__device__ bool block_wait(const uint32_t *flags, int n, uint32_t epoch, uint32_t phase, uint32_t *err, int *flag) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        int ok = 1;
        for (;;) {
            bool mine = true;
            for (int i = lane; i < n; i += 64) mine &= load_agent(flags + i) == epoch;
            if (__ballot(!mine) == 0) break;
            __builtin_amdgcn_s_sleep(1);
            if (__builtin_amdgcn_s_memrealtime() - t0 > kWaitTicks) {
                ok = 0;
                if (lane == 0) flag_error(err, kWaitTimeoutCode, phase);
                break;
            }
        }
        if (lane == 0) *flag = ok;
    }
    lds_barrier();
    return __builtin_amdgcn_readfirstlane(*flag) != 0;
}

// ---------------------------------------------------------------------------------------------------------------
// gate_up + SwiGLU. A block takes an equal run of the (expert, 16-feature tile) items (to within one item of every
// other block); its 8 waves split K Q ways (Q = K / 512: four spans a wave) and take 8 / Q items a round, so every
// wave of the grid streams the same bytes: 8 loads a round (4 spans x gate, up), one round in flight. The Q partial
// tiles of an item are summed in LDS after a barrier (Q > 1), in K order, and the item's SwiGLU rows are stored by
// the Q waves that made them, a quarter-tile or less each. A wave's four spans of the M activation rows sit in its
// registers as MFMA A operands (code order) for the whole kernel, with their span sums.
//
// FUSED (the one-launch layer): the logits come from the projection phase (agent-scope loads of the tagged pairs),
// h and its sums are stored at agent scope for the down phase of every block.
// DYN (the one-launch layer; gate_up with a sync buffer): a block streams S0 fixed items first (S0 = about 4/5 of an
// equal share, every G-th item: the grid sweeps the weights together, which streams faster than tiles claimed one
// by one and than a run of adjacent tiles a block), then items from the
// pool after all the runs, one round at a time from its part of the pool (kQueues parts, each shared by blocks on
// every XCD): its first two fixed, the rest claimed from the part's counter two rounds ahead. A block that streams
// faster takes more of the pool, so the blocks finish within about a round of each other however unevenly the
// memory system serves them.
struct GuLds {
    float red[2][kWaves][2][4][64];  // [round & 1][wave][gate, up][v][lane]
};

struct DnLds {
    alignas(16) uint16_t hs[kHsElems];
    alignas(16) float hsum[kMaxSlots * kMaxSpansDn];
    alignas(16) uint16_t zero_block[kZeroBytes / 2];
    alignas(16) float red[kWaves][16][16];
};

struct FusedSched {
    LayerSync *sync;
    uint32_t *queue;         // the counter of the block's part of the pool (this launch's set)
    int *rnd;                // LDS [4]: the claim (index into the part) of round gr, slot gr & 3
    const uint64_t *tagged;  // the projection's logits as (epoch << 32 | value bits) [M, ld]
    uint32_t epoch;
    uint64_t *trace;  // nullable: this block's stamp slots
    int *flag;        // LDS scratch of block_wait
};

template <int NV, int Q, bool FUSED, bool DYN = FUSED>
__device__ __forceinline__ void gate_up_body(const GateUpParams &p, GuLds &L, Routes &R, uint32_t *emask,
                                            const FusedSched &fs) {
    constexpr int P = kWaves / Q;  // items a round
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
    float sl0 = 0.f, sl1 = 0.f;
    if constexpr (FUSED) {
        // the logits as the projection phase published them: (epoch, value) pairs, re-read until every one this wave
        // needs carries this launch's epoch (or the wait gives up: error word, stale routing)
        const uint64_t *t0 = fs.tagged + (int64_t)min(wave, M - 1) * p.ld;
        const uint64_t *t1 = fs.tagged + (int64_t)min(wave + kWaves, M - 1) * p.ld;
        const int ecol = p.shared_logit ? p.E : p.E - 1;  // the shared gate's column, or a routed one again
        const uint64_t start = __builtin_amdgcn_s_memrealtime();
        int polls = 0;
        for (;;) {
            ++polls;
            bool fresh = true;
            uint64_t a[NV], c[NV];
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int e = min((int)(threadIdx.x & 63) + 64 * j, p.E - 1);
                a[j] = load_agent64(t0 + e), c[j] = load_agent64(t1 + e);
            }
            const uint64_t sa = load_agent64(t0 + ecol), sc = load_agent64(t1 + ecol);
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                fresh &= (uint32_t)(a[j] >> 32) == fs.epoch && (uint32_t)(c[j] >> 32) == fs.epoch;
                v0[j] = __uint_as_float((uint32_t)a[j]), v1[j] = __uint_as_float((uint32_t)c[j]);
            }
            fresh &= (uint32_t)(sa >> 32) == fs.epoch && (uint32_t)(sc >> 32) == fs.epoch;
            sl0 = __uint_as_float((uint32_t)sa), sl1 = __uint_as_float((uint32_t)sc);
            if (__ballot(!fresh) == 0) break;
            if (__builtin_amdgcn_s_memrealtime() - start > kWaitTicks) {
                if ((threadIdx.x & 63) == 0) flag_error(p.expert_err, kWaitTimeoutCode, 1);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (fs.trace && threadIdx.x == 0) fs.trace[2] = __builtin_amdgcn_s_memrealtime(), fs.trace[10] = polls;
    } else {
        routing::load_logits<NV>([&](int e) { return row0[e]; }, p.E, v0);
        routing::load_logits<NV>([&](int e) { return row1[e]; }, p.E, v1);
        sl0 = p.shared_logit ? p.shared_logit[(int64_t)min(wave, M - 1) * p.shared_ld] : 0.f;
        sl1 = p.shared_logit ? p.shared_logit[(int64_t)min(wave + kWaves, M - 1) * p.shared_ld] : 0.f;
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
    if constexpr (FUSED) {
        if (fs.trace && tid == 0) fs.trace[8] = __builtin_amdgcn_s_memrealtime();
    }
    // the activations only now: issued before the routing they queued ahead of the later waves' logits loads (the
    // waves of one compute unit share its load path), so the tokens routed by waves 4 .. 7 started about 0.9 us
    // late; they are first used after the weights' first round trip
    uint4 xr[4][4];
    {
        const uint16_t *xrow = p.x + (int64_t)min(n16, M - 1) * K + (int64_t)kq * 4 * kSpan + g * 32;
#pragma unroll
        for (int so = 0; so < 4; ++so)
#pragma unroll
            for (int t = 0; t < 4; ++t) xr[so][t] = *reinterpret_cast<const uint4 *>(xrow + so * kSpan + t * 8);
    }
    build_units(R, emask, tid < S ? R.ids[tid] : 0, S, A, Ew);
    if constexpr (FUSED) {
        if (fs.trace && tid == 0) fs.trace[9] = __builtin_amdgcn_s_memrealtime();
    }
    const int U = __builtin_amdgcn_readfirstlane(R.U);
    const int64_t Nrows = p.N / 2, rowbytes = K / 2, ngroups = K / kSpan;
    if (lead) {
        if (p.plan && tid < kPlanQuads) reinterpret_cast<uint4 *>(p.plan)[tid] = reinterpret_cast<const uint4 *>(&R)[tid];
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

    // 3. the items of U x T16 (expert-major). Static: this block's run [b0, b1) in rounds of P. DYN: rounds of one
    // item (Q = 8), rounds gr < S0 the items gr G + blk (the grid sweeps the items together), then items q0 + j of the block's part
    // [q0, q1) of the pool [G S0, F): j = r and nq + r for the first two (r: the block's rank among the nq blocks of
    // the part), then the claims in fs.rnd[gr & 3], from 2 nq on
    // 32-bit arithmetic (F = U T16 <= kMaxSlots I / 16): a 64-bit division by the grid size is a long software
    // sequence between the expert list and the first weight loads
    const int T16 = (int)((Nrows + 15) / 16);
    const int F = U * T16;
    const int G = (int)gridDim.x, blk = (int)blockIdx.x;
    const int S0 = DYN ? F * kFixedNum / kFixedDen / G : 0;
    const int PF = F - G * S0;  // the pool
    const int qj = queue_of(blk), grp = blk >> 3;
    const int q0 = G * S0 + qj * PF / kQueues, q1 = G * S0 + (qj + 1) * PF / kQueues;
    int nq = 0;
    for (int g2 = qj; DYN && g2 * 8 < G; g2 += kQueues) nq += min(8, G - 8 * g2);
    const int rank = 8 * (grp / kQueues) + (blk & 7);
    const int b0 = DYN ? 0 : (int)((unsigned)blk * F / G), b1 = DYN ? F : (int)((unsigned)(blk + 1) * F / G);
    const int groups = DYN ? 0 : (b1 - b0 + P - 1) / P;  // rounds (block-uniform; static)
    auto pool_item = [&](int gr) -> int {  // DYN, gr >= S0
        const int j = gr - S0;
        return j == 0 ? rank : j == 1 ? nq + rank : fs.rnd[gr & 3];
    };
    auto live = [&](int gr) -> bool {
        if constexpr (DYN) return gr < S0 || q0 + __builtin_amdgcn_readfirstlane(pool_item(gr)) < q1;
        else return gr < groups;
    };
    auto round_base = [&](int gr) -> int {
        if constexpr (DYN) return gr < S0 ? gr * G + blk : q0 + pool_item(gr);
        else return b0 + gr * P;
    };
    if (!live(0)) return;

    // 4. weight ring: round r = the slice kq of item round_base(r) + ip (clamped into the items: a clamped round
    // loads a valid tile and stores nothing); gate and up alternate, scale / min windows of the 4 spans
    constexpr int NW = 2;
    const int64_t up_q = Nrows * rowbytes, up_g = Nrows * ngroups;
    uint4 ring[kRing][kPrefetch];
    uint2 sw_n[kRing][NW], mw_n[kRing][NW];
    int ii = 0;
    const uint8_t *iq = p.q;
    const uint16_t *is_ = p.scale, *im = p.minv;
    auto iplace = [&]() {
        int item = round_base(ii) + ip;
        if constexpr (DYN) {  // a dead pool round (past the part; usually still inside F) loads the round before's item
            if (ii > 0 && ii >= S0 && item >= q1) item = round_base(ii - 1);  // again: an L2 hit, not an unused tile
        }
        item = min(item, b1 - 1);
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
    if constexpr (FUSED) {
        if (fs.trace && tid == 0) fs.trace[3] = __builtin_amdgcn_s_memrealtime();
    }

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
            if (on && n_in) {
                if constexpr (FUSED) store_agent(p.h + (int64_t)slot * Nrows + n, (uint16_t)hb);
                else p.h[(int64_t)slot * Nrows + n] = (uint16_t)hb;
            }
            if (p.h_sums) {
                const float ts = qmm::detail::group_sum_c<16>(n_in ? bf16_to_f32(hb) : 0.f);
                if (on && n16 == 0) {
                    if constexpr (FUSED) store_agent(p.h_sums + (int64_t)slot * T16 + tile, ts);
                    else p.h_sums[(int64_t)slot * T16 + tile] = ts;
                }
            }
        }
    };

    // 6. consume: A rows = tokens (lane row n16), D rows 4g .. 4g + 3 = tokens, columns = the 16 features
    auto consume = [&](int gr, auto slot_tag) __attribute__((always_inline)) {
        constexpr int RS = decltype(slot_tag)::value;
        // DYN: pool round gr + 2 >= S0 + 2, claimed while this one streams and published before the round's barrier.
        // Claimed whether or not the pool has run dry (a claim past the part's end is dead like every later one), and
        // the claim's value used only where it is published: a select on it here would wait for the atomic's return
        // (and every load issued before it) at once, holding the whole block up for a round trip to the counter.
        uint32_t claim_raw = 0u;
        if constexpr (DYN) {
            if (tid == 0 && gr >= S0) claim_raw = claim_one(fs.queue + qj * 32);
        }
        uint2 sw[NW], mw[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) sw[w] = sw_n[RS][w], mw[w] = mw_n[RS][w];
        if (DYN || gr + kRing < groups) advance_issue();
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
        if (!DYN && gr >= groups) return;  // the phantom round
        const int item = round_base(gr) + ip;
        if constexpr (Q == 1) {
            if (item < b1) epilogue(item, acc[0], acc[1]);
        } else {
            float(&mine)[2][4][64] = L.red[gr & 1][wave];
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int v = 0; v < 4; ++v) mine[w][v][lane] = acc[w][v];
            if constexpr (DYN) {
                if (tid == 0 && gr >= S0) fs.rnd[(gr + 2) & 3] = 2 * nq + (int)claim_raw;
            }
            // every wave's partial tile of this round is in LDS (the loads in flight stay in flight); the next
            // write to this half of red comes after the next round's barrier, when these reads are done
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (item < b1) {
                float gate[VS] = {}, up[VS] = {};
#pragma unroll
                for (int qq = 0; qq < Q; ++qq) {  // K order
                    const float(&part)[2][4][64] = L.red[gr & 1][ip * Q + qq];
#pragma unroll
                    for (int j = 0; j < VS; ++j) gate[j] += part[0][vb + j][lane], up[j] += part[1][vb + j][lane];
                }
                epilogue(item, gate, up);
            }
        }
    };
    if constexpr (DYN) {
        static_assert(!DYN || (Q == 8 && kRing == 1), "one item a round; the claims are published at the round's barrier");
        // a live round always issues the next one's loads (clamped when that one is dead): one path for the ring
        int gr = 0;
        for (;; ++gr) {
            consume(gr, std::integral_constant<int, 0>{});
            if (!live(gr + 1)) break;
        }
        if (fs.trace && tid == 0) fs.trace[11] = gr + 1;
    } else {
        // Runs of kRing rounds, all issuing their loads (an odd count ends with a phantom round that re-loads the
        // last one and stops after its MFMAs): a consume whose loads were conditional would merge two versions of
        // the ring registers, and the copies at such a merge wait for every outstanding load.
        for (int gr = 0; gr < groups; gr += kRing)
            [&]<int... RS>(std::integer_sequence<int, RS...>) {
                (consume(gr + RS, std::integral_constant<int, RS>{}), ...);
            }(std::make_integer_sequence<int, kRing>{});
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the phantom round's loads land before the wave moves on
}

// The pool counters of a launch: sync's set epoch & 1, one 128-byte line a part (block 0 zeroes the other set, which
// the next launch on this sync uses).
__device__ FusedSched make_sched(LayerSync *sync, uint32_t epoch, int *s_rnd, const uint64_t *tagged, uint64_t *trace,
                                 int *flag) {
    if (blockIdx.x == 0 && threadIdx.x < kQueues)
        __hip_atomic_store(&sync->queues[(epoch + 1) & 1][threadIdx.x][0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return FusedSched{sync, &sync->queues[epoch & 1][0][0], s_rnd, tagged, epoch, trace, flag};
}

// DYN: the items after the fixed runs come from the pool of p.sync (Q = 8).
template <int NV, int Q, bool DYN>
__global__ void __launch_bounds__(kThreads) gate_up_kernel(GateUpParams p) {
    __shared__ __attribute__((aligned(16))) GuLds L;
    __shared__ Routes R;
    __shared__ __attribute__((aligned(16))) uint32_t emask[kMaxExperts];
    __shared__ int s_flag, s_rnd[4];
    if constexpr (DYN)
        gate_up_body<NV, Q, false, true>(p, L, R, emask, make_sched(p.sync, p.epoch, s_rnd, nullptr, nullptr, &s_flag));
    else
        gate_up_body<NV, Q, false, false>(p, L, R, emask, FusedSched{});
}

// ---------------------------------------------------------------------------------------------------------------
// down + combine. A block owns 16 output rows for all tokens; LDS: the S slot rows of h [S][K + 8] BF16 (code
// order), span sums [S][K / 128], a zero block, the waves' partial sums [8][16 tokens][16 rows].
//
// Standalone (down_kernel): the routing and h come from memory (written by the gate_up launch). FUSED: the routing
// is the block's own (LDS, from the gate_up phase), h and its sums are staged once per block after the gate_up
// phase's counter is complete (agent-scope loads; this row block's first weight loads are already in flight), and
// the block may take several row blocks.
template <int NB, bool SUMS, bool FUSED>
__device__ __forceinline__ void down_body(const DownParams &p, DnLds &L, Routes &R, uint32_t *emask, int64_t n0,
                                          bool stage_h, const FusedSched &fs, bool &ok) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = p.M, A = p.A, S = M * A, Ew = p.Ew;
    const int64_t K = p.K, ldh = K + 8, N = p.N;
    const int nspan = (int)(K / kSpan), chunks8 = (int)(K / 8), lg_chunks = __builtin_ctz((unsigned)chunks8);
    const int n_items_x = S * chunks8;

    constexpr int kSumLoads = SUMS ? (kMaxSlots * kMaxSpansDn + kThreads - 1) / kThreads : 0;
    float4 tsum[kSumLoads > 0 ? kSumLoads : 1][2];  // SUMS: the 8 tile sums of (slot, span) i = b * kThreads + tid
    uint4 raw[NB];
    auto load_h = [&]() __attribute__((always_inline)) {
        const int tiles = (int)(K / 16);
        if constexpr (SUMS) {
#pragma unroll
            for (int b = 0; b < kSumLoads; ++b) {
                const int i = min(b * kThreads + tid, S * nspan - 1), r = i / nspan, sp = i - r * nspan;
                if constexpr (FUSED) {
                    const uint32_t off = (uint32_t)(((int64_t)r * tiles + sp * 8) * 4);
                    const uint4 a = load16_agent(p.h_sums, (uint32_t)(S * tiles * 4), off);
                    const uint4 c = load16_agent(p.h_sums, (uint32_t)(S * tiles * 4), off + 16);
                    tsum[b][0] = float4{__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z), __uint_as_float(a.w)};
                    tsum[b][1] = float4{__uint_as_float(c.x), __uint_as_float(c.y), __uint_as_float(c.z), __uint_as_float(c.w)};
                } else {
                    const float4 *src = reinterpret_cast<const float4 *>(p.h_sums + (int64_t)r * tiles + sp * 8);
                    tsum[b][0] = src[0], tsum[b][1] = src[1];
                }
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int i = min(b * kThreads + tid, n_items_x - 1);
            const int64_t e = (int64_t)(i >> lg_chunks) * K + (int64_t)(i & (chunks8 - 1)) * 8;
            if constexpr (FUSED) raw[b] = load16_agent(p.h, (uint32_t)(S * K * 2), (uint32_t)(e * 2));
            else raw[b] = *reinterpret_cast<const uint4 *>(p.h + e);
        }
    };
    if constexpr (!FUSED) {
        if (p.plan) {  // gate_up's routing as it stored it: one 16-byte load a thread, no rebuilding (h issued
                       // behind it: loading h after the first weight loads measured 0.8 us slower)
            const uint4 r = reinterpret_cast<const uint4 *>(p.plan)[min(tid, kPlanQuads - 1)];
            load_h();
            if (tid < kPlanQuads) reinterpret_cast<uint4 *>(&R)[tid] = r;
            for (int i = tid; i < kZeroBytes / 4; i += kThreads) reinterpret_cast<uint32_t *>(L.zero_block)[i] = 0u;
            lds_barrier();
        }
    }
    if constexpr (!FUSED) if (!p.plan) {
        // the routing first, then the rows of h: the grouping waits for the ids only
        const int32_t my_id = p.ids[min(lane, S - 1)];  // every wave: no branch around loads
        const float my_coef = p.coef[min(lane, S - 1)];
        load_h();
        R.ids[lane] = my_id, R.coef[lane] = my_coef;  // every wave the same values (unconditional: nothing sinks the loads)
        for (int i = tid; i < kZeroBytes / 4; i += kThreads) reinterpret_cast<uint32_t *>(L.zero_block)[i] = 0u;
        build_units(R, emask, my_id, S, A, Ew);  // its closing barrier also covers ids, coef and the zero block
    }
    const int U = __builtin_amdgcn_readfirstlane(R.U);
    const uint64_t bad_slots = R.bad_slots;
    if (!FUSED && blockIdx.x == 0 && bad_slots && tid == 0) {  // (FUSED: reported by the gate_up phase)
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

    if (!FUSED || stage_h) {
        if constexpr (FUSED) {  // h is complete once every block has published its gate_up part
            ok = block_wait(fs.sync->done_b, (int)gridDim.x, fs.epoch, 2, p.expert_err, fs.flag);
            if (fs.trace && tid == 0) fs.trace[5] = __builtin_amdgcn_s_memrealtime();
            load_h();
            for (int i = tid; i < kZeroBytes / 4; i += kThreads) reinterpret_cast<uint32_t *>(L.zero_block)[i] = 0u;
        }
        if constexpr (SUMS) {  // h in code order; span sums = the 8 tile sums in tile order
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int i = b * kThreads + tid;
                if (i < n_items_x) {
                    const int r = i >> lg_chunks, c8 = i & (chunks8 - 1);
                    const uint4 w = raw[b];
                    *reinterpret_cast<uint4 *>(L.hs + r * ldh + (int64_t)c8 * 8) =
                        uint4{__builtin_amdgcn_perm(w.z, w.x, 0x05040100u), __builtin_amdgcn_perm(w.z, w.x, 0x07060302u),
                              __builtin_amdgcn_perm(w.w, w.y, 0x05040100u), __builtin_amdgcn_perm(w.w, w.y, 0x07060302u)};
                }
            }
#pragma unroll
            for (int b = 0; b < kSumLoads; ++b) {
                const int i = b * kThreads + tid;
                if (i < S * nspan) {
                    const float4 a = tsum[b][0], c = tsum[b][1];
                    L.hsum[i] = ((((((a.x + a.y) + a.z) + a.w) + c.x) + c.y) + c.z) + c.w;
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
                    *reinterpret_cast<uint4 *>(L.hs + r * ldh + (int64_t)c8 * 8) = planes[0];
                    sum = qmm::detail::group_sum_c<16>(sum);
                    if ((c8 & 15) == 0) L.hsum[r * nspan + (c8 >> 4)] = sum;
                }
            }
        }
        lds_barrier();  // the ring's weight loads stay in flight
        if constexpr (FUSED) {
            if (fs.trace && tid == 0) fs.trace[6] = __builtin_amdgcn_s_memrealtime();
        }
    }

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
        const uint16_t *ab = sa >= 0 ? L.hs + sa * ldh + g * 32 + c0 * kSpan : L.zero_block;
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
                const float xv = sv[v] >= 0 ? L.hsum[sv[v] * nspan + c0 + s] : 0.f;
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
    for (int v = 0; v < 4; ++v) L.red[wave][4 * g + v][n16] = yacc[v];
    __syncthreads();
    if (tid < M * 16) {
        const int m = tid >> 4, c = tid & 15;
        const int64_t n = n0 + c;
        float y = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) y += L.red[w][m][c];
        bool bad = false;
        for (int a = 0; a < A; ++a) bad |= (bad_slots >> (m * A + a)) & 1ull;
        if (bad) y = qnan();
        if (n < N) {
            if (p.act == SX_ACT_F32) static_cast<float *>(p.y)[(int64_t)m * N + n] = y;
            else static_cast<uint16_t *>(p.y)[(int64_t)m * N + n] = (uint16_t)f32_to_bf16(y);
        }
    }
    if constexpr (FUSED) __syncthreads();  // red is rewritten by the next row block
}

template <int NB, bool SUMS>
__global__ void __launch_bounds__(kThreads) down_kernel(DownParams p) {
    __shared__ __attribute__((aligned(16))) DnLds L;
    __shared__ Routes R;
    __shared__ __attribute__((aligned(16))) uint32_t emask[kMaxExperts];
    bool ok = true;
    down_body<NB, SUMS, false>(p, L, R, emask, (int64_t)blockIdx.x * 16, true, FusedSched{}, ok);
}

// ---------------------------------------------------------------------------------------------------------------
// The router projection as the one-launch layer's first phase: block b projects weight rows [a R / PA, (a + 1) R / PA)
// for a = b, b + G, ... (at most kProjRows rows each); each thread owns 8-column chunks of those rows (every 512th),
// issues its weight and activation loads before any use, and the per-(row, token) sums meet in a wave sum and
// across the waves in LDS in a fixed order. Each logit goes to the output and, tagged with the launch's epoch as one
// 64-bit agent-scope store, to the pairs the routing of every block polls.
constexpr int kProjRows = 4;

struct ProjLds {
    float part[kWaves][kProjRows * kMaxTokens];
};

template <typename TW, int MT>
__device__ __forceinline__ void project_item(const LayerParams &lp, ProjLds &L, int r0, int nr) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int M = lp.gu.M;
    const int64_t K = lp.gu.K, K8 = K / 8;
    const TW *W = static_cast<const TW *>(lp.wr);
    float acc[kProjRows][MT];
#pragma unroll
    for (int r = 0; r < kProjRows; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[r][t] = 0.f;
    for (int64_t c = tid; c < K8; c += kThreads) {
        float wv[kProjRows][8];
#pragma unroll
        for (int r = 0; r < kProjRows; ++r) {
            const TW *wr = W + (int64_t)(r0 + min(r, nr - 1)) * K + c * 8;
            if constexpr (sizeof(TW) == 4) {
                const float4 a = reinterpret_cast<const float4 *>(wr)[0], b = reinterpret_cast<const float4 *>(wr)[1];
                wv[r][0] = a.x, wv[r][1] = a.y, wv[r][2] = a.z, wv[r][3] = a.w;
                wv[r][4] = b.x, wv[r][5] = b.y, wv[r][6] = b.z, wv[r][7] = b.w;
            } else {
                qmm::detail::unpack8(*reinterpret_cast<const uint4 *>(wr), wv[r]);
            }
        }
        uint4 xr[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) xr[t] = *reinterpret_cast<const uint4 *>(lp.gu.x + (int64_t)min(t, M - 1) * K + c * 8);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (t < M) {  // uniform
                float xv[8];
                qmm::detail::unpack8(xr[t], xv);
#pragma unroll
                for (int r = 0; r < kProjRows; ++r)
                    if (r < nr)  // uniform
#pragma unroll
                        for (int e = 0; e < 8; ++e) acc[r][t] = fmaf(xv[e], wv[r][e], acc[r][t]);
            }
        }
    }
    if constexpr (MT == 8 && kProjRows == 4) {
        // The wave's 32 sums (row r, token t: value 8 r + t) in 32 exchanges instead of a wave reduction each: every
        // step pairs lane l with l ^ o and halves the values a lane keeps (the half its bit of o picks), the other
        // half going to the partner; after o = 32 .. 2 a lane holds one value's sum over its pair of lanes, o = 1
        // completes it. Value v ends in the lanes l with bits 5..1 of l equal to v.
        const float *a = &acc[0][0];
        float hv[16];
        const bool h5 = (lane >> 5) & 1, h4 = (lane >> 4) & 1, h3 = (lane >> 3) & 1, h2 = (lane >> 2) & 1, h1 = (lane >> 1) & 1;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float send = h5 ? a[i] : a[16 + i], keep = h5 ? a[16 + i] : a[i];
            hv[i] = keep + __shfl_xor(send, 32);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float send = h4 ? hv[i] : hv[8 + i], keep = h4 ? hv[8 + i] : hv[i];
            hv[i] = keep + __shfl_xor(send, 16);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float send = h3 ? hv[i] : hv[4 + i], keep = h3 ? hv[4 + i] : hv[i];
            hv[i] = keep + __shfl_xor(send, 8);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float send = h2 ? hv[i] : hv[2 + i], keep = h2 ? hv[2 + i] : hv[i];
            hv[i] = keep + __shfl_xor(send, 4);
        }
        {
            const float send = h1 ? hv[0] : hv[1], keep = h1 ? hv[1] : hv[0];
            hv[0] = keep + __shfl_xor(send, 2);
        }
        hv[0] += __shfl_xor(hv[0], 1);
        const int v = (lane >> 1) & 31, r = v >> 3, t = v & 7;
        if ((lane & 1) == 0 && r < nr && t < M) L.part[wave][r * kMaxTokens + t] = hv[0];
    } else {
#pragma unroll
        for (int r = 0; r < kProjRows; ++r)
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                if (r < nr && t < M) {  // uniform
                    const float s = routing::wave_sum_f32(acc[r][t]);
                    if (lane == 0) L.part[wave][r * kMaxTokens + t] = s;
                }
            }
    }
    lds_barrier();
    if (tid < nr * kMaxTokens) {
        const int r = tid / kMaxTokens, t = tid % kMaxTokens;
        if (t < M) {
            float y = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) y += L.part[w][tid];
            const int64_t i = (int64_t)t * lp.ld + r0 + r;
            lp.logits[i] = y;
            __hip_atomic_store(lp.tagged + i, ((uint64_t)lp.epoch << 32) | __float_as_uint(y), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    lds_barrier();  // part is rewritten by the next item (an LDS-only barrier: the stores complete in the background)
}

// ---------------------------------------------------------------------------------------------------------------
// The whole verify-width MoE sublayer in one launch: router projection -> routing (each block its own copy) ->
// gate_up + SwiGLU -> down + combine, the phases handed over through per-block flags (LayerSync) rather than kernel
// boundaries: no phase waits for a launch, and the down phase's first weight loads go out while the last gate_up rounds
// finish. Each block's share of every phase is fixed (the shares of the two-launch kernels), so the launch relies on
// all its blocks being resident together (one 512-thread block a compute unit, as the launch sizes it); a wait that
// does not complete in 20 ms - another kernel holding compute units for that long - gives up with an error word
// instead of hanging.
union LayerPool {  // the phases' LDS, one after the other
    ProjLds proj;
    GuLds gu;
    DnLds dn;
};

template <int NV, int Q, int NB, typename TW, int MT>
__global__ void __launch_bounds__(kThreads) layer_kernel(LayerParams lp) {
    __shared__ __attribute__((aligned(16))) LayerPool pool;
    __shared__ Routes R;
    __shared__ __attribute__((aligned(16))) uint32_t emask[kMaxExperts];
    __shared__ int s_flag, s_rnd[4];
    LayerSync *sync = lp.sync;
    const int tid = threadIdx.x, G = (int)gridDim.x, b = (int)blockIdx.x;
    uint64_t *trace = lp.trace ? lp.trace + (int64_t)b * kTraceSlots : nullptr;
    auto stamp = [&](int i) {
        if (trace && tid == 0) trace[i] = __builtin_amdgcn_s_memrealtime();
    };
    stamp(0);
    const FusedSched fs = make_sched(sync, lp.epoch, s_rnd, lp.tagged, trace, &s_flag);

    // phase A: the router projection, rows [a R / PA, (a + 1) R / PA) for a = b, b + G, ... (at most kProjRows each)
    const int rows = lp.rows, PA = max(G, (rows + kProjRows - 1) / kProjRows);
    for (int a = b; a < PA; a += G) {
        // 32-bit unsigned (PA * rows < 2^21): a 64-bit division is a long scalar sequence ahead of the first loads
        const int r0 = (int)((unsigned)a * rows / PA), r1 = (int)((unsigned)(a + 1) * rows / PA);
        if (r1 > r0) project_item<TW, MT>(lp, pool.proj, r0, r1 - r0);
    }
    stamp(1);

    // phase B: routing (each routing wave polls the tagged logits it needs) + gate_up + SwiGLU
    bool ok = true;
    gate_up_body<NV, Q, true>(lp.gu, pool.gu, R, emask, fs);
    stamp(4);
    block_publish(&sync->done_b[b], lp.epoch);

    // phase C: down + combine, output rows [16 rb, 16 rb + 16) for rb = b, b + G, ...
    const int nrb = (int)((lp.dn.N + 15) / 16);
    for (int rb = b; rb < nrb && ok; rb += G) down_body<NB, true, true>(lp.dn, pool.dn, R, emask, (int64_t)rb * 16, rb == b, fs, ok);
    stamp(7);
}

}  // namespace

hipError_t launch_gate_up(const GateUpParams &p, int cus, hipStream_t stream) {
    const int nv = p.E <= 256 ? 4 : p.E <= 512 ? 8 : 16;
    const int q = (int)(p.K / 512);  // K in {512, 1024, 2048, 4096}: four spans a wave
    const dim3 grid((unsigned)cus);
    auto go = [&](auto nv_tag, auto q_tag) {
        constexpr int NV = decltype(nv_tag)::value, QQ = decltype(q_tag)::value;
        if constexpr (QQ == 8) {
            if (p.sync) {
                gate_up_kernel<NV, QQ, true><<<grid, kThreads, 0, stream>>>(p);
                return;
            }
        }
        gate_up_kernel<NV, QQ, false><<<grid, kThreads, 0, stream>>>(p);
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

hipError_t launch_layer(const LayerParams &p, bool wr_f32, int cus, hipStream_t stream) {
    const dim3 grid((unsigned)cus);
    auto go = [&](auto nv_tag, auto tw) {
        if (p.gu.M <= 8) layer_kernel<decltype(nv_tag)::value, 8, 16, decltype(tw), 8><<<grid, kThreads, 0, stream>>>(p);
        else layer_kernel<decltype(nv_tag)::value, 8, 16, decltype(tw), 16><<<grid, kThreads, 0, stream>>>(p);
    };
    auto by_w = [&](auto nv_tag) {
        if (wr_f32) go(nv_tag, float{});
        else go(nv_tag, uint16_t{});
    };
    if (p.gu.E <= 512) by_w(std::integral_constant<int, 8>{});
    else by_w(std::integral_constant<int, 16>{});
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
    SX_CHECK(E >= 1 && E <= vf::kMaxExperts && k >= 1 && k <= E && k <= 32 && Ew >= 1 && Ew <= vf::kMaxExperts, fn,
             " E = ", E, ", k = ", k, ", Ew = ", Ew, ": needs E, Ew <= ", vf::kMaxExperts, " and k <= min(E, 32)");
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

std::atomic<uint64_t *> g_layer_trace{nullptr};

// The launch numbers of the sync buffers: 1, 2, ... (never 0, the value of a freshly zeroed buffer). A launch that
// uses a buffer's pool takes the counter set of its number's parity and zeroes the other set for the next one, so the
// numbers of the launches that use a buffer must alternate in parity: a number is reserved before the launch and
// committed only once the launch went out (a failed launch, or one that does not use the pool, leaves it unused), and
// the wrap goes from 0xFFFFFFFF (odd) to 2, skipping 0.
std::mutex g_epoch_mu;
std::unordered_map<const void *, uint32_t> g_epochs;

uint32_t reserve_epoch(const void *sync) {
    std::lock_guard<std::mutex> lock(g_epoch_mu);
    const uint32_t last = g_epochs[sync];
    return last == 0xFFFFFFFFu ? 2u : last + 1;
}

void commit_epoch(const void *sync, uint32_t e) {
    std::lock_guard<std::mutex> lock(g_epoch_mu);
    g_epochs[sync] = e;
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
                          uint32_t *expert_err, void *sync, void *plan, sx_stream stream) {
    const char *fn = "sx_moe_verify_gate_up";
    const int64_t A = k + (shared_logit ? 1 : 0);
    SX_CHECK(x != nullptr && logits != nullptr && ids != nullptr && coef != nullptr && h != nullptr &&
                 router_err != nullptr && expert_err != nullptr,
             fn, " null pointer");
    if (int rc = check_gate_up(fn, M, A, E, k, Ew, w, act)) return rc;
    SX_CHECK(ld >= E && (shared_logit == nullptr || shared_ld >= 1), fn, " ld = ", ld, ", shared_ld = ", shared_ld);
    SX_CHECK(shared_logit == nullptr || (shared_id >= 0 && shared_id < Ew), fn, " shared_id = ", shared_id,
             ", expected the shared expert's row block in 0..", Ew - 1);
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
    SX_CHECK(plan == nullptr || aligned(plan, 16), fn, " plan must be 16-byte aligned");
    p.plan = plan;
    // The pool schedule exists for K = 4096 (eight K slices a block); other shapes split the items statically and
    // leave the buffer untouched.
    if (sync != nullptr && w->K == 4096) {
        SX_CHECK(aligned(sync, 16), fn, " sync must be 16-byte aligned");
        p.sync = static_cast<vf::LayerSync *>(sync);
        p.epoch = reserve_epoch(sync);
    }
    SX_HIP(vf::launch_gate_up(p, device_cus(), stream_of(stream)), fn);
    if (p.sync) commit_epoch(sync, p.epoch);
    return SX_OK;
}

int sx_moe_verify_down(const void *h, const float *h_sums, int64_t M, int64_t A, const int32_t *ids, const float *coef,
                       const sx_qview *w, int64_t Ew, void *y, int act, uint32_t *expert_err, const void *plan,
                       sx_stream stream) {
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
    SX_CHECK(plan == nullptr || aligned(plan, 16), fn, " plan must be 16-byte aligned");
    p.plan = plan;
    SX_HIP(vf::launch_down(p, stream_of(stream)), fn);
    return SX_OK;
}

int sx_moe_verify_layer_trace(uint64_t *buf) {
    g_layer_trace.store(buf);
    return SX_OK;
}

int sx_moe_verify_layer_sync_bytes(size_t *bytes) {
    SX_CHECK(bytes != nullptr, "null output");
    *bytes = sizeof(vf::LayerSync);
    return SX_OK;
}

int sx_moe_verify_layer(const void *x, int64_t M, const void *wr, int wr_act, int64_t rows, int64_t E, int64_t k,
                        int shared, int32_t shared_id, const sx_qview *gate_up, const sx_qview *down, int64_t Ew,
                        float *logits, int32_t *ids, float *coef, void *h, float *h_sums, void *y, int act,
                        uint32_t *router_err, uint32_t *expert_err, void *sync, sx_stream stream) {
    const char *fn = "sx_moe_verify_layer";
    SX_CHECK(x && wr && logits && ids && coef && h && h_sums && y && router_err && expert_err && sync, fn,
             " null pointer");
    const int64_t A = k + (shared ? 1 : 0);
    if (int rc = check_gate_up(fn, M, A, E, k, Ew, gate_up, act)) return rc;
    if (int rc = check_down(fn, M, A, Ew, down, act)) return rc;
    const int64_t K = gate_up->K, I = gate_up->N / Ew / 2, d = down->N / Ew;
    SX_CHECK(device_cus() <= vf::kMaxBlocks, fn, " more compute units than the sync buffer has slots");
    SX_CHECK(K == 4096 && E <= 1024, fn, " the one-launch layer takes d = 4096 and E <= 1024 (d = ", K, ", E = ", E,
             "); the two-launch FFN takes the others");
    SX_CHECK(down->K == I && d == K, fn, " down [", d, ", ", down->K, "] does not match gate_up's I = ", I,
             " and d = ", K);
    SX_CHECK(wr_act == SX_ACT_F32 || wr_act == SX_ACT_BF16, fn, " router weight dtype ", wr_act);
    SX_CHECK(!shared || (shared_id >= 0 && shared_id < Ew), fn, " shared_id = ", shared_id,
             ", expected the shared expert's row block in 0..", Ew - 1);
    SX_CHECK(rows >= E + (shared ? 1 : 0) && rows <= vf::kMaxRouterRows, fn, " router weight has ", rows, " rows for E = ", E,
             shared ? " plus the shared gate" : "");
    SX_CHECK(aligned(wr, 16) && aligned(x, 16) && aligned(h, 16) && aligned(h_sums, 16) && aligned(sync, 16), fn,
             " x, the router weight, h, h_sums and sync must be 16-byte aligned");
    SX_CHECK(apart(logits, M * rows * 4, x, M * K * 2) && apart(h, M * A * I * 2, x, M * K * 2) &&
                 apart(y, M * d * 2, h, M * A * I * 2) && apart(y, M * d * 2, x, M * K * 2),
             fn, " outputs overlap inputs");
    vf::LayerParams lp{};
    vf::GateUpParams &p = lp.gu;
    p.x = static_cast<const uint16_t *>(x), p.M = (int)M, p.A = (int)A, p.k = (int)k, p.E = (int)E, p.Ew = (int)Ew;
    p.logits = logits, p.ld = rows, p.shared_logit = shared ? logits + E : nullptr, p.shared_ld = rows;
    p.shared_id = shared_id;
    p.q = gate_up->q, p.scale = gate_up->scale, p.minv = gate_up->minv, p.N = gate_up->N / Ew, p.K = K;
    p.ids = ids, p.coef = coef, p.h = static_cast<uint16_t *>(h), p.h_sums = h_sums;
    p.router_err = router_err, p.expert_err = expert_err;
    vf::DownParams &q = lp.dn;
    q.h = p.h, q.h_sums = h_sums, q.M = (int)M, q.A = (int)A, q.Ew = (int)Ew, q.ids = ids, q.coef = coef;
    q.q = down->q, q.scale = down->scale, q.minv = down->minv, q.N = d, q.K = I, q.y = y, q.act = act;
    q.expert_err = expert_err;
    lp.wr = wr, lp.rows = (int)rows, lp.logits = logits, lp.ld = rows, lp.sync = static_cast<vf::LayerSync *>(sync);
    lp.trace = g_layer_trace.load();
    lp.tagged = lp.sync->tagged;
    lp.epoch = reserve_epoch(sync);
    SX_HIP(vf::launch_layer(lp, wr_act == SX_ACT_F32, device_cus(), stream_of(stream)), fn);
    commit_epoch(sync, lp.epoch);
    return SX_OK;
}

}  // extern "C"
