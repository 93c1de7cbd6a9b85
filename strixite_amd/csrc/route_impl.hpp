// Device pieces shared by the router and the grouping kernels: the 64-bit routing key, a wave's top-k routing of
// one token (kernels/moe_router.hpp:11-23), and the counting sort of slots into expert buckets by one block
// (the workspace layout of kernels/moe_grouped.hip:63-81).
#pragma once
#include "common.hpp"

#include <climits>

namespace sx::routing {

// Larger logit first, then lower index: value bits made monotone in the high word (-0 folded to +0, as a float
// compare treats them), ~index in the low word, so one unsigned compare orders (value desc, index asc).
__device__ __forceinline__ uint64_t route_key(float v, int idx) {
    const uint32_t b = v == 0.f ? 0u : __float_as_uint(v);
    const uint32_t hi = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)hi << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)idx);
}

// The logit a key was made from (a -0 logit comes back as +0, which no later use tells apart).
__device__ __forceinline__ float key_value(uint64_t key) {
    const uint32_t hi = (uint32_t)(key >> 32);
    return __uint_as_float((hi & 0x80000000u) ? (hi & 0x7FFFFFFFu) : ~hi);
}

// Wave-wide reductions of one 32-bit value, all in DPP (no LDS round trips): inside each row of 16 lanes quad
// [1,0,3,2], quad [2,3,0,1], half-row mirror and row mirror leave every lane with its row's result (max, min and
// sum need no particular pairing); then row_bcast:15 (rows 1, 3 take lane 15 of the row before) and row_bcast:31
// (rows 2, 3 take lane 31) leave the wave's result in lane 63, read out as a scalar. A row outside a broadcast's row
// mask receives `old`: the operation's identity.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWS, 0xF, false);
}

// `old` is the operation's identity (0 for max, ~0 for min), so the compiler folds each move into the max / min
// as one DPP instruction.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0xB1>(0u, v));
    v = max(v, dpp_u32<0x4E>(0u, v));
    v = max(v, dpp_u32<0x141>(0u, v));
    v = max(v, dpp_u32<0x140>(0u, v));
    v = max(v, dpp_u32<0x142, 0xA>(0u, v));
    v = max(v, dpp_u32<0x143, 0xC>(0u, v));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, dpp_u32<0xB1>(~0u, v));
    v = min(v, dpp_u32<0x4E>(~0u, v));
    v = min(v, dpp_u32<0x141>(~0u, v));
    v = min(v, dpp_u32<0x140>(~0u, v));
    v = min(v, dpp_u32<0x142, 0xA>(~0u, v));
    v = min(v, dpp_u32<0x143, 0xC>(~0u, v));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Inclusive prefix sum over the wave's lanes: row_shr 1, 2, 4, 8 scan each row of 16 (a lane with no source
// adds `old` = 0), then row_bcast:15 and row_bcast:31 carry the row totals into the rows after them.
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
    v += dpp_u32<0x111>(0u, v);
    v += dpp_u32<0x112>(0u, v);
    v += dpp_u32<0x114>(0u, v);
    v += dpp_u32<0x118>(0u, v);
    v += dpp_u32<0x142, 0xA>(0u, v);
    v += dpp_u32<0x143, 0xC>(0u, v);
    return v;
}

__device__ __forceinline__ float wave_sum_f32(float x) {
    auto add = [](float a, uint32_t b) { return a + __uint_as_float(b); };
    x = add(x, dpp_u32<0xB1>(0u, __float_as_uint(x)));
    x = add(x, dpp_u32<0x4E>(0u, __float_as_uint(x)));
    x = add(x, dpp_u32<0x141>(0u, __float_as_uint(x)));
    x = add(x, dpp_u32<0x140>(0u, __float_as_uint(x)));
    x = add(x, dpp_u32<0x142, 0xA>(0u, __float_as_uint(x)));
    x = add(x, dpp_u32<0x143, 0xC>(0u, __float_as_uint(x)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

// Sorts N (a power of two) keys descending in registers: a bitonic network with compile-time indices.
template <int N>
__device__ __forceinline__ void sort_desc(uint64_t (&a)[N]) {
#pragma unroll
    for (int size = 2; size <= N; size <<= 1)
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1)
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool desc = (i & size) == 0 || size == N;
                    const uint64_t x = a[i], y = a[j];
                    const bool sw = desc ? x < y : x > y;
                    a[i] = sw ? y : x, a[j] = sw ? x : y;
                }
            }
}

// Lane l's NV logits of one token (experts l, l + 64, ...; past E: expert E - 1 again, masked later). Every lane
// loads all NV, so the loads go out together and one wait covers them (a load under a per-lane condition becomes a
// branch with its own wait).
template <int NV, typename Load>
__device__ __forceinline__ void load_logits(Load load, int E, float (&v)[NV]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = load(min(lane + 64 * j, E - 1));
}

// route_token on logits already in registers (load_logits).
template <int NV>
__device__ void route_values(float (&v)[NV], int E, int k, bool has_shared, float sl, int32_t shared_id, int64_t m,
                             int32_t *id_row, float *coef_row, int32_t *lds_row, uint32_t *err) {
    const int lane = threadIdx.x & 63;
    const int A = k + (has_shared ? 1 : 0);
    int bad = INT_MAX;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = lane + 64 * j;
        v[j] = e < E ? v[j] : -INFINITY;
        if (e < E && !isfinite(v[j]) && e < bad) bad = e;
    }
    if (has_shared && !isfinite(sl) && E < bad) bad = E;
    if (__ballot(bad != INT_MAX)) bad = (int)wave_min_u32((uint32_t)bad);  // uniform; INT_MAX: no bad logit
    if (bad != INT_MAX) {  // kernels/moe_router.hpp:19-23
        if (lane == 0 && err) flag_error(err, (uint32_t)m, (uint32_t)bad);  // null err: a redundant copy of the routing
        for (int a = lane; a < A; a += 64) {
            id_row[a] = -1, coef_row[a] = qnan();
            if (lds_row) lds_row[a] = -1;
        }
        return;
    }
    // Padding past E never wins: its value key (0) is below every finite logit's.
    uint32_t hv[NV];  // value keys (the monotone bits)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = lane + 64 * j;
        hv[j] = e < E ? (uint32_t)(route_key(v[j], e) >> 32) : 0u;
    }
    float my_v = -INFINITY, top = 0.f;
    int my_i = -1;
    // T = the k-th largest of the 64 lane maxima (counted with multiplicity), bit by bit: k lanes hold an element
    // >= T, so every one of the top k is >= T. The candidates (>= T; usually a few more than k) go to lanes
    // 0 .. C-1, each takes its rank among them by (value desc, index asc), and a permute puts pick r in lane r.
    uint32_t lm = hv[0];
#pragma unroll
    for (int j = 1; j < NV; ++j) lm = max(lm, hv[j]);
    // Only the top 16 bits of T are searched (8 steps): a T with its low bits cleared is still <= the k-th largest
    // lane maximum, so the candidate set still holds the top k; it admits at most a few more (values within a
    // 2^-7 relative distance of the threshold).
    uint32_t T = 0u;
    for (int b = 30; b >= 16; b -= 2) {  // two bits a step: three independent counts
        const uint32_t t1 = T | (1u << b), t2 = T | (2u << b), t3 = T | (3u << b);
        const int c1 = __popcll(__ballot(lm >= t1)), c2 = __popcll(__ballot(lm >= t2)), c3 = __popcll(__ballot(lm >= t3));
        T = c3 >= k ? t3 : c2 >= k ? t2 : c1 >= k ? t1 : T;  // uniform
    }
    // the candidates' keys (value desc, index asc as one unsigned order) into this wave's LDS row, in (j, lane) order
    __shared__ __attribute__((aligned(16))) uint64_t route_cand[16][64];
    uint64_t *cand = route_cand[(threadIdx.x >> 6) & 15];
    int C = 0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const bool in = hv[j] >= T;
        const uint64_t bal = __ballot(in);
        const int pos = C + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        if (in && pos < 64) cand[pos] = ((uint64_t)hv[j] << 32) | (0xFFFFFFFFu - (uint32_t)(lane + 64 * j));
        C += __popcll(bal);
    }
    if (C <= 64) {
        // one wave's LDS accesses take effect in program order: the writes above precede these reads
        const uint64_t mine = lane < C ? cand[lane] : 0ull;
        int rank = 0;
        for (int c = 0; c < C; c += 8) {  // uniform; 16-byte broadcast reads, eight keys a step (past C: ignored)
#pragma unroll
            for (int u = 0; u < 8; u += 2) {
                const ulonglong2 o = *reinterpret_cast<const ulonglong2 *>(cand + c + u);
                rank += (c + u < C && o.x > mine) ? 1 : 0;
                rank += (c + u + 1 < C && o.y > mine) ? 1 : 0;
            }
        }
        if (lane >= C) rank = lane;  // ranks 0 .. C-1 of the candidates plus the other lanes: a permutation
        const uint32_t pv = (uint32_t)__builtin_amdgcn_ds_permute(rank * 4, (int)(uint32_t)(mine >> 32));
        const uint32_t px = 0xFFFFFFFFu - (uint32_t)__builtin_amdgcn_ds_permute(rank * 4, (int)(uint32_t)mine);
        top = key_value((uint64_t)__builtin_amdgcn_readfirstlane(pv) << 32);
        if (lane < k) my_v = key_value((uint64_t)pv << 32), my_i = (int)px;
    } else {
        // Many ties at the threshold: k rounds of the wave maximum over each lane's sorted keys, the lane owning the
        // winner popping its head (a tie between lanes goes to the lower index: a second reduction, only then).
        uint64_t keys[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int e = lane + 64 * j;
            keys[j] = e < E ? route_key(v[j], e) : 0;
        }
        sort_desc<NV>(keys);
        uint32_t hx[NV];  // expert index; padding: 0xFFFFFFFF
#pragma unroll
        for (int j = 0; j < NV; ++j) hv[j] = (uint32_t)(keys[j] >> 32), hx[j] = 0xFFFFFFFFu - (uint32_t)keys[j];
        for (int r = 0; r < k; ++r) {
            const uint32_t best = wave_max_u32(hv[0]);  // uniform
            const bool cand = hv[0] == best;
            const uint64_t cands = __ballot(cand);
            const uint32_t bi = __popcll(cands) == 1
                                    ? (uint32_t)__builtin_amdgcn_readlane((int)hx[0], __builtin_ctzll(cands))
                                    : wave_min_u32(cand ? hx[0] : 0xFFFFFFFFu);
            const float bv = key_value((uint64_t)best << 32);
            if (r == 0) top = bv;
            if (lane == r) my_v = bv, my_i = (int)bi;
            const bool pop = cand && hx[0] == bi;  // one lane: a lane's indices are distinct
#pragma unroll
            for (int j = 0; j + 1 < NV; ++j) hv[j] = pop ? hv[j + 1] : hv[j], hx[j] = pop ? hx[j + 1] : hx[j];
            hv[NV - 1] = pop ? 0u : hv[NV - 1];
            hx[NV - 1] = pop ? 0xFFFFFFFFu : hx[NV - 1];
        }
    }
    const float ex = lane < k ? expf(my_v - top) : 0.f;
    const float sum = wave_sum_f32(ex);
    if (lane < k) {
        id_row[lane] = my_i, coef_row[lane] = ex / sum;
        if (lds_row) lds_row[lane] = my_i;
    }
    if (has_shared && lane == 0) {
        id_row[k] = shared_id, coef_row[k] = 1.0f / (1.0f + expf(-sl));
        if (lds_row) lds_row[k] = shared_id;
    }
}

// Token m's routing by one wave: the E logits (load(e) -> float) stay in registers, lane l holding experts
// l, l + 64, ...; a threshold below which no top-k value lies (bit-by-bit search over the lane maxima), the few
// candidates above it ranked against each other (k rounds of a wave-wide maximum instead when more than 64 values
// reach the threshold); then the softmax over the k picks (coef = exp(l - l_max) / sum). A non-finite logit (or shared gate)
// fails the token: ids -1, coefficients NaN, err = {1, m, expert} (first wins). With has_shared, slot k is the
// shared expert with coefficient sigmoid(sl). lds_row (may be null) receives the ids too.
template <int NV, typename Load>
__device__ void route_token(Load load, int E, int k, bool has_shared, float sl, int32_t shared_id, int64_t m,
                            int32_t *id_row, float *coef_row, int32_t *lds_row, uint32_t *err) {
    float v[NV];
    load_logits<NV>(load, E, v);
    route_values<NV>(v, E, k, has_shared, sl, shared_id, m, id_row, coef_row, lds_row, err);
}

// Exclusive prefix sums of three per-thread counts over an NT-thread block: wave64 inclusive scans by shuffles,
// then the wave totals scanned by wave 0. wtot: LDS [NT / 64][3].
template <int NT>
__device__ void block_scan3(int (&v)[3], int (&excl)[3], int (&total)[3], int (*wtot)[3]) {
    constexpr int kW = NT / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc[3] = {v[0], v[1], v[2]};
#pragma unroll
    for (int off = 1; off < 64; off <<= 1)
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int o = __shfl_up(inc[j], off);
            if (lane >= off) inc[j] += o;
        }
    if (lane == 63)
#pragma unroll
        for (int j = 0; j < 3; ++j) wtot[wave][j] = inc[j];
    __syncthreads();
    if (wave == 0) {
        int w[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) w[j] = lane < kW ? wtot[lane][j] : 0;
#pragma unroll
        for (int off = 1; off < kW; off <<= 1)
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                const int o = __shfl_up(w[j], off);
                if (lane >= off) w[j] += o;
            }
        if (lane < kW)
#pragma unroll
            for (int j = 0; j < 3; ++j) wtot[lane][j] = w[j];  // inclusive wave prefix
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int before = wave ? wtot[wave - 1][j] : 0;
        excl[j] = before + inc[j] - v[j];
        total[j] = wtot[kW - 1][j];
    }
}

constexpr int kR = 16, kRW = 64;  // slots a tile (16-row MFMA tiles) and a wide tile

// Counting sort of S slots into E + 1 buckets (bucket E = invalid ids) by one NT-thread block, written in the
// workspace layout of kernels/moe_grouped.hip:63-81: header [n_tiles, S, E, n_wtiles], offsets [E + 2],
// slots [S], tile_bucket / tile_start [Tmax], wtile_bucket / wtile_start [WTmax]. Thread t owns a run of
// consecutive buckets. Slot order within a bucket follows the atomics; no output depends on it. The first
// invalid slot in slot order (an atomic minimum, independent of scheduling) goes to err = {1, id, slot}.
// LDS: cnt, cursor [E + 1], wtot [NT / 64][3], first_bad; optionally stage [stage_cap]: when S <= stage_cap the
// slots are placed in LDS and leave in order, a coalesced store for 64 of them (placed straight into the workspace,
// every slot is a store of its own to a scattered address: 20,480 slots took 18 us in one block, 10.7 staged).
template <int NT, typename IdAt>
__device__ void group_in_block(IdAt id_at, int S, int E, int Tmax, int WTmax, int32_t *ws, uint32_t *err, int *cnt,
                               int *cursor, int (*wtot)[3], int *first_bad, int *stage = nullptr, int stage_cap = 0) {
    const int t = threadIdx.x;
    for (int b = t; b <= E; b += NT) cnt[b] = 0;
    if (t == 0) *first_bad = INT_MAX;
    __syncthreads();
    // ids eight at a time, every load issued before the first use (a load per loop trip would wait each trip)
    constexpr int kIds = 8;
    for (int s0 = t; s0 < S; s0 += NT * kIds) {
        int32_t idv[kIds];
#pragma unroll
        for (int u = 0; u < kIds; ++u) idv[u] = id_at(min(s0 + u * NT, S - 1));
#pragma unroll
        for (int u = 0; u < kIds; ++u) {
            const int s = s0 + u * NT;
            if (s >= S) break;
            const int32_t id = idv[u];
            const bool bad = id < 0 || id >= E;
            atomicAdd(&cnt[bad ? E : id], 1);
            if (bad) atomicMin(first_bad, s);
        }
    }
    __syncthreads();
    if (t == 0 && *first_bad != INT_MAX) flag_error(err, (uint32_t)id_at(*first_bad), (uint32_t)*first_bad);
    const int per = (E + 1 + NT - 1) / NT;
    const int b0 = min(t * per, E + 1), b1 = min(b0 + per, E + 1);
    int v[3] = {0, 0, 0}, ex[3], tot[3];
    for (int b = b0; b < b1; ++b) {
        const int c = cnt[b];
        v[0] += c, v[1] += (c + kR - 1) / kR, v[2] += (c + kRW - 1) / kRW;
    }
    block_scan3<NT>(v, ex, tot, wtot);
    int32_t *offsets = ws + 4, *slots = offsets + E + 2, *tile_bucket = slots + S, *tile_start = tile_bucket + Tmax;
    int32_t *wtile_bucket = tile_start + Tmax, *wtile_start = wtile_bucket + WTmax;
    for (int b = b0; b < b1; ++b) {
        const int c = cnt[b], nt = (c + kR - 1) / kR, nw = (c + kRW - 1) / kRW;
        offsets[b] = ex[0];
        cursor[b] = ex[0];
        for (int i = 0; i < nt; ++i) tile_bucket[ex[1] + i] = b, tile_start[ex[1] + i] = ex[0] + i * kR;
        for (int i = 0; i < nw; ++i) wtile_bucket[ex[2] + i] = b, wtile_start[ex[2] + i] = ex[0] + i * kRW;
        ex[0] += c, ex[1] += nt, ex[2] += nw;
    }
    if (t == 0) {
        ws[0] = tot[1], ws[1] = S, ws[2] = E, ws[3] = tot[2];
        offsets[E + 1] = tot[0];
    }
    __syncthreads();
    const bool staged = S <= stage_cap;  // uniform
    int32_t *dst = staged ? stage : slots;
    for (int s0 = t; s0 < S; s0 += NT * kIds) {
        int32_t idv[kIds];
#pragma unroll
        for (int u = 0; u < kIds; ++u) idv[u] = id_at(min(s0 + u * NT, S - 1));
#pragma unroll
        for (int u = 0; u < kIds; ++u) {
            const int s = s0 + u * NT;
            if (s >= S) break;
            const int32_t id = idv[u];
            dst[atomicAdd(&cursor[(id < 0 || id >= E) ? E : id], 1)] = s;
        }
    }
    if (staged) {
        __syncthreads();
        for (int i = t; i < S; i += NT) slots[i] = stage[i];
    }
}

}  // namespace sx::routing
