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

// Wave-wide maximum of 64-bit keys, all in DPP (no LDS round trips): inside each row of 16 lanes quad [1,0,3,2],
// quad [2,3,0,1], half-row mirror and row mirror leave every lane with its row's maximum (max needs no particular
// pairing); then row_bcast:15 (rows 1, 3 take lane 15 of the row before) and row_bcast:31 (rows 2, 3 take lane 31)
// leave the wave's maximum in lane 63, read out as a scalar.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint64_t dpp_max(uint64_t k) {
    const int lo0 = (int)(uint32_t)k, hi0 = (int)(uint32_t)(k >> 32);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(lo0, lo0, CTRL, ROWS, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(hi0, hi0, CTRL, ROWS, 0xF, false);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    return o > k ? o : k;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
    k = dpp_max<0xB1>(k);        // quad_perm [1,0,3,2]
    k = dpp_max<0x4E>(k);        // quad_perm [2,3,0,1]
    k = dpp_max<0x141>(k);       // row_half_mirror
    k = dpp_max<0x140>(k);       // row_mirror
    k = dpp_max<0x142, 0xA>(k);  // row_bcast:15 into rows 1 and 3
    k = dpp_max<0x143, 0xC>(k);  // row_bcast:31 into rows 2 and 3
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
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

// Token m's routing by one wave: the E logits (load(e) -> float) stay in registers, lane l holding experts
// l, l + 64, ...; k rounds of a wave-wide key maximum, only the lane whose expert was picked rescanning its
// registers; then the softmax over the k picks (coef = exp(l - l_max) / sum). A non-finite logit (or shared gate)
// fails the token: ids -1, coefficients NaN, err = {1, m, expert} (first wins). With has_shared, slot k is the
// shared expert with coefficient sigmoid(sl). lds_row (may be null) receives the ids too.
template <int NV, typename Load>
__device__ void route_token(Load load, int E, int k, bool has_shared, float sl, int32_t shared_id, int64_t m,
                            int32_t *id_row, float *coef_row, int32_t *lds_row, uint32_t *err) {
    const int lane = threadIdx.x & 63;
    const int A = k + (has_shared ? 1 : 0);
    float v[NV];
    int bad = INT_MAX;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = lane + 64 * j;
        const float xv = e < E ? load(e) : -INFINITY;
        v[j] = xv;
        if (e < E && !isfinite(xv) && e < bad) bad = e;
    }
    if (has_shared && !isfinite(sl) && E < bad) bad = E;
    for (int off = 32; off > 0; off >>= 1) bad = min(bad, __shfl_xor(bad, off));
    if (bad != INT_MAX) {  // kernels/moe_router.hpp:19-23
        if (lane == 0) flag_error(err, (uint32_t)m, (uint32_t)bad);
        for (int a = lane; a < A; a += 64) {
            id_row[a] = -1, coef_row[a] = qnan();
            if (lds_row) lds_row[a] = -1;
        }
        return;
    }
    // Padding past E never wins: its key (0) is below every finite logit's. Each lane sorts its keys once; a round
    // takes the wave maximum of the lane heads and the lane that owned it pops its head.
    uint64_t keys[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = lane + 64 * j;
        keys[j] = e < E ? route_key(v[j], e) : 0;
    }
    sort_desc<NV>(keys);
    float my_v = -INFINITY, top = 0.f;
    int my_i = -1;
    for (int r = 0; r < k; ++r) {
        const uint64_t best = wave_max_u64(keys[0]);  // uniform
        const int bi = (int)(0xFFFFFFFFu - (uint32_t)best);
        const float bv = key_value(best);
        if (r == 0) top = bv;
        if (lane == r) my_v = bv, my_i = bi;
        const bool pop = keys[0] == best;  // one lane: keys are distinct
#pragma unroll
        for (int j = 0; j + 1 < NV; ++j) keys[j] = pop ? keys[j + 1] : keys[j];
        keys[NV - 1] = pop ? 0 : keys[NV - 1];
    }
    const float ex = lane < k ? expf(my_v - top) : 0.f;
    float sum = ex;
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    if (lane < k) {
        id_row[lane] = my_i, coef_row[lane] = ex / sum;
        if (lds_row) lds_row[lane] = my_i;
    }
    if (has_shared && lane == 0) {
        id_row[k] = shared_id, coef_row[k] = 1.0f / (1.0f + expf(-sl));
        if (lds_row) lds_row[k] = shared_id;
    }
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
// LDS: cnt, cursor [E + 1], wtot [NT / 64][3], first_bad.
template <int NT, typename IdAt>
__device__ void group_in_block(IdAt id_at, int S, int E, int Tmax, int WTmax, int32_t *ws, uint32_t *err, int *cnt,
                               int *cursor, int (*wtot)[3], int *first_bad) {
    const int t = threadIdx.x;
    for (int b = t; b <= E; b += NT) cnt[b] = 0;
    if (t == 0) *first_bad = INT_MAX;
    __syncthreads();
    for (int s = t; s < S; s += NT) {
        const int32_t id = id_at(s);
        const bool bad = id < 0 || id >= E;
        atomicAdd(&cnt[bad ? E : id], 1);
        if (bad) atomicMin(first_bad, s);
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
    for (int s = t; s < S; s += NT) {
        const int32_t id = id_at(s);
        slots[atomicAdd(&cursor[(id < 0 || id >= E) ? E : id], 1)] = s;
    }
}

}  // namespace sx::routing
