// The verify tail on gfx950: logits top-k (kernels/logits_topk.hpp:3-46), the MTP draft pick (kernels/mtp_pick.hpp:3-33)
// and draft acceptance on the device (serve/engine.cpp:592-610 with serve/sampler.cpp:183-248's draw).
#include "common.hpp"
#include "pick.hpp"

#include <climits>
#include <mutex>
#include <vector>

namespace sx {
namespace {

// ---------------- 64-bit candidate keys ----------------
// A candidate (value, id) as one key whose unsigned order is the candidates' order: value bits made monotone in the
// high word (-0 folded onto +0, so they tie as a float compare does), the id inverted in the low word (lower id
// first). 0 = no candidate (no real candidate maps there: only a NaN bit pattern would, and NaNs are left out).
__device__ __forceinline__ uint64_t cand_key(float v, int32_t id) {
    const uint32_t b = v == 0.f ? 0u : __float_as_uint(v);
    const uint32_t hi = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)hi << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)id);
}
__device__ __forceinline__ int32_t key_id(uint64_t k) { return (int32_t)(0xFFFFFFFFu - (uint32_t)k); }

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m), hi = __shfl_xor((uint32_t)(v >> 32), m);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl64(uint64_t v, int src) {
    const uint32_t lo = __shfl((uint32_t)v, src), hi = __shfl((uint32_t)(v >> 32), src);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t umax(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t umin(uint64_t a, uint64_t b) { return a < b ? a : b; }

// Bitonic sort of one key a lane across the wave, descending by lane (lane 0 = best): 21 compare-exchange stages.
__device__ uint64_t wave_sort_desc(uint64_t v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1)
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const uint64_t o = shfl_xor64(v, stride);
            const bool desc = (lane & size) == 0, lower = (lane & stride) == 0;
            v = (lower == desc) ? umax(v, o) : umin(v, o);
        }
    return v;
}

// Top 64 of two descending lane-sorted lists: max against the other list reversed is bitonic, then 6 merge stages.
__device__ uint64_t wave_merge_desc(uint64_t a, uint64_t b) {
    const int lane = threadIdx.x & 63;
    uint64_t c = umax(a, shfl64(b, 63 - lane));
#pragma unroll
    for (int stride = 32; stride > 0; stride >>= 1) {
        const uint64_t o = shfl_xor64(c, stride);
        c = (lane & stride) == 0 ? umax(c, o) : umin(c, o);
    }
    return c;
}

// The wave's best k (k <= 64) of the keys its lanes hold (P a lane), lane-sorted descending; lanes >= k hold 0.
// Threshold: the k-th best lane maximum - at least k keys reach it, so every key of the top k does. The keys that
// reach it (usually ~k: mostly the lane maxima) are compacted through LDS and sorted with one or a few bitonic passes.
template <int P>
__device__ __forceinline__ uint64_t wave_topk_sorted(const uint64_t (&key)[P], int k, uint64_t *scratch, int scratch_cap) {
    const int lane = threadIdx.x & 63;
    uint64_t head = 0;
#pragma unroll
    for (int p = 0; p < P; ++p) head = umax(head, key[p]);
    const uint64_t tau = shfl64(wave_sort_desc(head), k - 1);  // 0 if fewer than k lanes hold anything
    int cnt = 0;
#pragma unroll
    for (int p = 0; p < P; ++p) cnt += (key[p] != 0 && key[p] >= tau) ? 1 : 0;
    int incl = cnt;  // inclusive prefix of the counts across lanes
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
    }
    const int total = __shfl(incl, 63);
    uint64_t list = 0;
    if (total <= scratch_cap) {
        int at = incl - cnt;
#pragma unroll
        for (int p = 0; p < P; ++p)
            if (key[p] != 0 && key[p] >= tau) scratch[at++] = key[p];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        for (int b0 = 0; b0 < total; b0 += 64) {
            const uint64_t c = b0 + lane < total ? scratch[b0 + lane] : 0;
            const uint64_t s = wave_sort_desc(c);
            list = b0 == 0 ? s : wave_merge_desc(list, s);
        }
        __builtin_amdgcn_wave_barrier();
    } else {  // many keys at the threshold (heavy ties): merge column by column
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const uint64_t c = (key[p] != 0 && key[p] >= tau) ? key[p] : 0;
            if (__ballot(c != 0) == 0) continue;
            list = wave_merge_desc(list, wave_sort_desc(c));
        }
    }
    return lane < k ? list : 0;
}

constexpr int kTopkThreadsB = 256;  // threads of a top-k block

__device__ __forceinline__ uint32_t routing_wave_incl_scan(int v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(v, off);
        if (lane >= off) v += o;
    }
    return (uint32_t)v;
}
constexpr int kScratchB = 256;      // candidates a wave's region holds (keys)

// wave_topk_sorted's result by ranks instead of sorts: the threshold T is the value word of the k-th best lane
// maximum (a search two bits a step with ballots, over its top 16 bits: a T with its low bits cleared is still at
// most that maximum, and admits only keys within 2^-7 of it besides), so every top-k key has a value word >= T; the keys that reach it
// (a superset of the top k, ties at T included) go to the wave's LDS row by ballot positions, each takes its rank
// among them from broadcast reads (keys are unique: ids differ), and the best k land at their ranks. More than 128
// such keys (heavy ties at T) take the sorting path.
template <int P>
__device__ __forceinline__ uint64_t wave_topk(const uint64_t (&key)[P], int k, uint64_t *scratch, int scratch_cap) {
    const int lane = threadIdx.x & 63;
    uint64_t head = 0;
#pragma unroll
    for (int p = 0; p < P; ++p) head = umax(head, key[p]);
    const uint32_t hh = (uint32_t)(head >> 32);
    uint32_t T = 0u;
    for (int b = 30; b >= 16; b -= 2) {  // uniform
        const uint32_t t1 = T | (1u << b), t2 = T | (2u << b), t3 = T | (3u << b);
        const int c1 = __popcll(__ballot(hh >= t1)), c2 = __popcll(__ballot(hh >= t2)), c3 = __popcll(__ballot(hh >= t3));
        T = c3 >= k ? t3 : c2 >= k ? t2 : c1 >= k ? t1 : T;
    }
    int C = 0;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const bool in = key[p] != 0 && (uint32_t)(key[p] >> 32) >= T;
        const uint64_t bal = __ballot(in);
        const int pos = C + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        if (in && pos < scratch_cap) scratch[pos] = key[p];
        C += __popcll(bal);
    }
    if (C > 128 || C > scratch_cap) return wave_topk_sorted<P>(key, k, scratch, scratch_cap);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const uint64_t a0 = lane < C ? scratch[lane] : 0, a1 = lane + 64 < C ? scratch[lane + 64] : 0;
    int r0 = 0, r1 = 0;
    for (int c = 0; c < C; c += 4) {  // uniform
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint64_t o = scratch[min(c + u, C - 1)];
            const bool valid = c + u < C;
            r0 += (valid && o > a0) ? 1 : 0;
            r1 += (valid && o > a1) ? 1 : 0;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // every read above precedes the writes below
    if (lane < C && r0 < k) scratch[r0] = a0;
    if (lane + 64 < C && r1 < k) scratch[r1] = a1;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const uint64_t list = lane < min(k, C) ? scratch[lane] : 0;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // the row is free for the next use
    return list;
}

// LDS of block_topk.
struct BlockTopkLds {
    uint64_t cand[kTopkThreadsB * 2];  // candidates (keys that reach the threshold), any order
    uint32_t head[kTopkThreadsB];      // each thread's best value word
    uint64_t best[64];
    uint32_t T;
    int n;
};

// The block's best k (k <= 64) of the keys its threads hold (P a thread, kTopkThreadsB threads), sorted descending:
// lane l of every thread's wave returns key l of the list (0 past k or past the keys there are). The threshold T is
// the value word of the k-th best of the threads' own best keys, found by wave 0 two bits a step with ballots over
// its top 16 bits (a T with its low bits cleared is still at most that key, and admits only keys within 2^-7 of it
// besides): at least k keys reach it, so every key of the top k does. The keys that reach it (about k for continuous
// values) are compacted into LDS, and each is ranked against all of them by one thread with broadcast reads, eight
// keys in flight (keys are unique: ids differ); the one of rank r < k is the block's r-th best. No sort and no merge.
// More candidates than LDS holds (heavy ties at T) take the waves' own top-k lists, merged.
template <int P>
__device__ uint64_t block_topk(const uint64_t (&key)[P], int k, BlockTopkLds &L, uint64_t (*region)[kScratchB],
                               bool any_order = false) {
    constexpr int kCap = kTopkThreadsB * 2;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    uint64_t head = 0;
#pragma unroll
    for (int p = 0; p < P; ++p) head = umax(head, key[p]);
    L.head[t] = (uint32_t)(head >> 32);
    if (t == 0) L.n = 0;
    if (t < 64) L.best[t] = 0;
    __syncthreads();
    if (wave == 0) {
        constexpr int kH = kTopkThreadsB / 64;
        uint32_t h[kH];
#pragma unroll
        for (int j = 0; j < kH; ++j) h[j] = L.head[lane + 64 * j];
        uint32_t T = 0u;
        for (int b = 30; b >= 16; b -= 2) {  // uniform
            const uint32_t t1 = T | (1u << b), t2 = T | (2u << b), t3 = T | (3u << b);
            int c1 = 0, c2 = 0, c3 = 0;
#pragma unroll
            for (int j = 0; j < kH; ++j)
                c1 += __popcll(__ballot(h[j] >= t1)), c2 += __popcll(__ballot(h[j] >= t2)), c3 += __popcll(__ballot(h[j] >= t3));
            T = c3 >= k ? t3 : c2 >= k ? t2 : c1 >= k ? t1 : T;
        }
        if (lane == 0) L.T = T;
    }
    __syncthreads();
    const uint32_t T = L.T;
    int mine = 0;
#pragma unroll
    for (int p = 0; p < P; ++p) mine += (key[p] != 0 && (uint32_t)(key[p] >> 32) >= T) ? 1 : 0;
    const uint32_t incl = routing_wave_incl_scan(mine);
    int base = 0;
    if (lane == 63) base = atomicAdd(&L.n, (int)incl);
    base = __shfl(base, 63);
    int at = base + (int)incl - mine;
#pragma unroll
    for (int p = 0; p < P; ++p)
        if (key[p] != 0 && (uint32_t)(key[p] >> 32) >= T) {
            if (at < kCap) L.cand[at] = key[p];
            ++at;
        }
    __syncthreads();
    const int C = L.n;
    if (C > kCap) {  // uniform over the block: heavy ties at T
        const uint64_t w = wave_topk<P>(key, k, region[wave], kScratchB);
        __syncthreads();
        region[wave][lane] = w;
        __syncthreads();
        uint64_t list = region[0][lane];
#pragma unroll
        for (int v = 1; v < kTopkThreadsB / 64; ++v) {
            list = wave_merge_desc(list, region[v][lane]);
            list = lane < k ? list : 0;
        }
        __syncthreads();
        return list;
    }
    if (any_order && C <= 64) {  // a superset of the top k, unranked: the candidates themselves (uniform)
        const uint64_t r = lane < C ? L.cand[lane] : 0;
        __syncthreads();
        return r;
    }
    for (int i = t; i < C; i += kTopkThreadsB) {
        const uint64_t x = L.cand[i];
        int rank = 0;
        for (int c = 0; c < C; c += 8) {  // uniform; past C: ignored (reads stay inside cand)
            ulonglong2 o[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) o[u] = *reinterpret_cast<const ulonglong2 *>(L.cand + min(c + 2 * u, kCap - 2));
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                rank += (c + 2 * u < C && o[u].x > x) ? 1 : 0;
                rank += (c + 2 * u + 1 < C && o[u].y > x) ? 1 : 0;
            }
        }
        if (rank < k) L.best[rank] = x;
    }
    __syncthreads();
    const uint64_t r = lane < k ? L.best[lane] : 0;
    __syncthreads();  // L and the regions are free for the caller's next use
    return r;
}

// ---------------- logits top-k ----------------
// One level: workgroup g of row r reduces up to kGroup inputs - logits (level 1: ids = positions < n_valid, NaN
// flagged and left out, masked ids left out) or an earlier level's key lists - to its best k keys. Each wave takes a
// strided quarter (coalesced loads), finds its best k (wave_topk), and wave 0 merges the four lists.
constexpr int kTopkThreads = kTopkThreadsB;
constexpr int kPer = 16;                      // inputs a thread holds
constexpr int kGroup = kTopkThreads * kPer;   // inputs a workgroup reduces
constexpr int kScratch = kScratchB;           // compaction room a wave (keys)

template <bool kLogits, bool kMasked>
__global__ void __launch_bounds__(kTopkThreads)
    topk_level_kernel(const float *logits, int64_t ld, int n_valid, const uint64_t *in, int n_in, int groups, int k,
                      uint64_t *out_keys, sx_logit_cand *out_final, uint32_t *nan_level1, int groups1, uint32_t *nan,
                      const uint32_t *mask, int64_t mask_words) {
    __shared__ uint64_t scratch[kTopkThreads / 64][kScratch];
    __shared__ uint64_t lists[kTopkThreads / 64][64];
    __shared__ uint32_t s_nan;
    __shared__ BlockTopkLds s_btk;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, g = blockIdx.x;
    const int64_t r = blockIdx.y;
    if (t == 0) s_nan = 0;
    uint64_t key[kPer];
    uint32_t my_nan = 0;
    // every load unconditional (the index clamped into the row) so that all of them go out before the first wait;
    // a load under a per-lane condition becomes a branch that waits for it
    if constexpr (kLogits) {
        float xv[kPer];
        uint32_t mw[kPer];
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int j = min(g * kGroup + p * kTopkThreads + t, n_valid - 1);
            xv[p] = logits[r * ld + j];
            if constexpr (kMasked) mw[p] = mask[r * mask_words + (j >> 5)];
        }
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int j = g * kGroup + p * kTopkThreads + t;
            key[p] = 0;
            if (j < n_valid) {
                const float x = xv[p];
                const bool allowed = !kMasked || ((mw[p] >> (j & 31)) & 1u);
                if (x != x) my_nan = 1u;  // flagged whether the id is allowed or not
                else if (allowed) key[p] = cand_key(x, j);
            }
        }
    } else {
#pragma unroll
        for (int p = 0; p < kPer; ++p) key[p] = in[r * n_in + min(g * kGroup + p * kTopkThreads + t, n_in - 1)];
#pragma unroll
        for (int p = 0; p < kPer; ++p)
            if (g * kGroup + p * kTopkThreads + t >= n_in) key[p] = 0;
    }
    // the last level of several: the first level's NaN flags of the row, loaded now (64 at a time across wave 0),
    // used at the end
    bool f1 = false;
    if (!kLogits && groups == 1 && wave == 0)
        for (int c = lane; c < groups1; c += 64) f1 |= nan_level1[r * groups1 + c] != 0u;
    __syncthreads();
    if (my_nan) atomicOr(&s_nan, 1u);
    const uint64_t best = block_topk<kPer>(key, k, s_btk, scratch);
    if (wave != 0) return;
    if (groups > 1) {
        if (lane < k) out_keys[(r * groups + g) * k + lane] = best;
    } else if (lane < k) {  // the last level: candidates with their values from the keys (a zero read back from the
                            // row: the key folds -0 onto +0)
        sx_logit_cand c;
        if (best == 0) {
            c.v = -INFINITY, c.id = INT32_MAX;
        } else {
            const uint32_t hi = (uint32_t)(best >> 32);
            c.id = key_id(best);
            c.v = __uint_as_float((hi & 0x80000000u) ? (hi & 0x7FFFFFFFu) : ~hi);
            if (c.v == 0.f) c.v = logits[r * ld + c.id];
        }
        out_final[r * k + lane] = c;
    }
    if constexpr (kLogits) {
        if (lane == 0) {
            nan_level1[r * groups + g] = s_nan;
            if (groups == 1) nan[r] = s_nan;
        }
    } else if (groups == 1) {  // the first level's flags of the row
        const bool any = __ballot(f1) != 0;  // the whole wave votes
        if (lane == 0) nan[r] = any ? 1u : 0u;
    }
}

int64_t groups_of(int64_t n) { return (n + kGroup - 1) / kGroup; }

// ---------------- MTP draft pick ----------------
constexpr int kPickThreads = 1024;

using pick::top2_merge;
using pick::top2_take;
using pick::top2_xor;
using pick::Top2;

// VEC: 16-byte loads (n % 4 == 0, x 16-byte aligned), thread t taking elements 4j .. 4j + 3 for j = t, t + 1024, ...
// Either way a thread's indices ascend, and its loads go out in batches of kPickBatch before any is used (the index
// clamped into the row).
template <bool VEC>
__global__ void __launch_bounds__(kPickThreads)
    mtp_pick_kernel(const float *x, int64_t n, const uint32_t *router_err, const uint32_t *expert_err,
                    const uint32_t *attn_err, const unsigned long long *emb_err, sx_mtp_pick_t *out) {
    __shared__ Top2 part[kPickThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    Top2 p{-INFINITY, -INFINITY, INT_MAX, 0u};
    constexpr int kPickBatch = 16;
    if constexpr (VEC) {
        const int64_t n4 = n / 4;
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        for (int64_t base = tid; base < n4; base += (int64_t)kPickBatch * kPickThreads) {
            float4 v[kPickBatch];
#pragma unroll
            for (int b = 0; b < kPickBatch; ++b) {
                const int64_t j = base + (int64_t)b * kPickThreads;
                v[b] = x4[j < n4 ? j : n4 - 1];
            }
#pragma unroll
            for (int b = 0; b < kPickBatch; ++b) {
                const int64_t j = base + (int64_t)b * kPickThreads;
                if (j >= n4) break;
                top2_take(p, v[b].x, 4 * j), top2_take(p, v[b].y, 4 * j + 1);
                top2_take(p, v[b].z, 4 * j + 2), top2_take(p, v[b].w, 4 * j + 3);
            }
        }
    } else {
        for (int64_t base = tid; base < n; base += (int64_t)kPickBatch * kPickThreads) {
            float v[kPickBatch];
#pragma unroll
            for (int b = 0; b < kPickBatch; ++b) {
                const int64_t i = base + (int64_t)b * kPickThreads;
                v[b] = x[i < n ? i : n - 1];
            }
#pragma unroll
            for (int b = 0; b < kPickBatch; ++b) {
                const int64_t i = base + (int64_t)b * kPickThreads;
                if (i >= n) break;
                top2_take(p, v[b], i);
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) p = top2_merge(p, top2_xor(p, off));
    if (lane == 0) part[wave] = p;
    __syncthreads();
    if (wave != 0) return;
    p = lane < kPickThreads / 64 ? part[lane] : Top2{-INFINITY, -INFINITY, INT_MAX, 0u};
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) p = top2_merge(p, top2_xor(p, off));
    pick::write_pick(p, lane, pick::read_errs(lane, router_err, expert_err, attn_err, emb_err), out);
}

// The pick over many blocks (sx_mtp_pick_ws), one launch: block b reduces its run of the logits (its threads offer
// their indices in ascending order, as mtp_pick_kernel's do) and the block that finishes last merges the blocks'
// partials into the output (pick::block_pick); the merge does not depend on the split, so the output equals
// mtp_pick_kernel's bit for bit. A single block reads the whole row through one compute unit (the served 65,536
// logits: 12 us); 64 blocks read it at once.
constexpr int kPickWsBlocks = 64, kPickWsThreads = 256;

template <bool VEC>
__global__ void __launch_bounds__(kPickWsThreads) mtp_pick_ws_kernel(const float *x, int64_t n, pick::Args a) {
    __shared__ Top2 red[kPickWsThreads / 64];
    __shared__ int last;
    const int tid = threadIdx.x;
    Top2 p = pick::top2_none();
    const pick::ErrWords errs = pick::read_errs(tid, a.router_err, a.expert_err, a.attn_err, a.emb_err);
    // the block's run [lo, hi): whole float4s when VEC
    const int64_t per = VEC ? ((n / 4 + gridDim.x - 1) / gridDim.x) * 4 : (n + gridDim.x - 1) / gridDim.x;
    const int64_t lo = (int64_t)blockIdx.x * per, hi = lo + per < n ? lo + per : n;
    constexpr int kBatch = 4;
    if constexpr (VEC) {
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        const int64_t a4 = lo / 4, b4 = hi / 4;
        for (int64_t base = a4 + tid; base < b4; base += (int64_t)kBatch * kPickWsThreads) {
            float4 v[kBatch];
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int64_t j = base + (int64_t)b * kPickWsThreads;
                v[b] = x4[j < b4 ? j : b4 - 1];
            }
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int64_t j = base + (int64_t)b * kPickWsThreads;
                if (j >= b4) break;
                top2_take(p, v[b].x, 4 * j), top2_take(p, v[b].y, 4 * j + 1);
                top2_take(p, v[b].z, 4 * j + 2), top2_take(p, v[b].w, 4 * j + 3);
            }
        }
    } else {
        for (int64_t base = lo + tid; base < hi; base += (int64_t)kBatch * kPickWsThreads) {
            float v[kBatch];
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int64_t i = base + (int64_t)b * kPickWsThreads;
                v[b] = x[i < hi ? i : hi - 1];
            }
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int64_t i = base + (int64_t)b * kPickWsThreads;
                if (i >= hi) break;
                top2_take(p, v[b], i);
            }
        }
    }
    pick::block_pick<kPickWsThreads / 64>(p, a, errs, red, &last);
}

// ---------------- draft acceptance ----------------
// Lane 0 walks the rows in order, exactly as the engine's loop and the sampler's draw do on the host: the sums are
// sequential in double, the draw r = u * kept with u the host's generate_canonical<double, 53> for that row. The
// wave loads a row's candidates into LDS and computes their probabilities exp(v_i / T - v_0 / T) a lane each (the
// same double arithmetic, once each) before lane 0's sequential walk reads them; once lane 0 has their sum, the
// quotients p_i / sum the top-p walk adds are taken a lane each too (each quotient is the same division whoever
// makes it, so the walk's sums are unchanged).
// LDS of one acceptance walk.
struct AcceptLds {
    sx_logit_cand cs[64];
    double probs[64], quot[64], pre[64], sum;
    int go;
};

// Ordering among the lanes of one wave through LDS (the walk runs on one wave).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// The walk by one wave; cand(j, i) and nan_of(j) read row j's candidate i and NaN flag.
template <typename CandAt, typename NanAt>
__device__ void accept_walk(CandAt cand, NanAt nan_of, int kc, const int32_t *drafts, int k, const double *u,
                            double temperature, int top_k, double top_p, int64_t n_valid, int32_t *out, AcceptLds &L) {
    sx_logit_cand *cs = L.cs;
    double *probs = L.probs, *quot = L.quot;
    const int lane = threadIdx.x & 63;
    const int kk = (int)(top_k < n_valid ? top_k : n_valid);
    int status = 0, j = 0;
    for (;; ++j) {
        if (lane < kc) cs[lane] = cand(j, lane);
        const bool row_nan = nan_of(j) != 0u;
        wave_sync();
        const bool sampled = temperature != 0 && isfinite(cs[0].v);  // uniform
        if (sampled && lane < kk) probs[lane] = exp((double)cs[lane].v / temperature - (double)cs[0].v / temperature);
        wave_sync();
        // pre[i] = probs[0] + .. + probs[i], added in order: the sampler's total (pre[kk - 1]), its kept mass
        // (pre[keep - 1]) and its draw's running sums are all prefixes of this one sequence, so one sequential pass
        // gives every one of them bit for bit
        if (sampled) {
            if (lane == 0) {
                double acc = 0;
                for (int i = 0; i < kk; ++i) acc += probs[i], L.pre[i] = acc;
                L.sum = acc;
            }
            wave_sync();
        }
        if (sampled && top_p < 1) {
            if (lane < kk) quot[lane] = probs[lane] / L.sum;
            wave_sync();
        }
        if (lane == 0) {
            const sx_logit_cand *c = cs;
            int32_t v = -1;
            bool ok = !row_nan;
            // serve/sampler.cpp:192-201: real candidates (ids in range) first, then only padding; at least one real.
            bool padding = false;
            const int m = kc < 20 ? kc : 20;
            for (int i = 0; ok && i < m; ++i) {
                const bool pad = c[i].id == INT32_MAX && c[i].v == -INFINITY;
                ok = pad || (!padding && c[i].id >= 0 && c[i].id < n_valid);
                padding |= pad;
            }
            ok = ok && c[0].id != INT32_MAX;
            if (ok && temperature == 0) {
                v = c[0].id;
            } else if (ok) {
                ok = isfinite(c[0].v);
                if (ok) {
                    int keep = kk;
                    if (top_p < 1) {
                        double acc = 0;
                        for (int i = 0; i < kk; ++i) {
                            acc += quot[i];
                            if (acc >= top_p) {
                                keep = i + 1;
                                break;
                            }
                        }
                    }
                    const double kept = L.pre[keep - 1];  // probs[0] + .. + probs[keep - 1] in order
                    const double r = u[j] * kept;
                    v = c[keep - 1].id;
                    for (int i = 0; i < keep; ++i) {  // the draw's running sum after i + 1 terms is pre[i]
                        if (r < L.pre[i]) {
                            v = c[i].id;
                            break;
                        }
                    }
                }
            }
            bool go = false;
            if (!ok) {
                status = 1 + j;
            } else {
                out[2 + j] = v;
                go = !(j == k || v != drafts[j]);
            }
            L.go = go ? 1 : 0;
        }
        wave_sync();
        if (!L.go) break;
    }
    if (lane == 0) out[0] = j, out[1] = status;
}

__global__ void __launch_bounds__(64)
    mtp_accept_kernel(const sx_logit_cand *cands, const uint32_t *nan, int kc, const int32_t *drafts, int k,
                      const double *u, double temperature, int top_k, double top_p, int64_t n_valid, int32_t *out) {
    __shared__ AcceptLds L;
    accept_walk([&](int j, int i) { return cands[(int64_t)j * kc + i]; }, [&](int j) { return nan[j]; }, kc, drafts,
                k, u, temperature, top_k, top_p, n_valid, out, L);
}

// ---------------- logits top-k and acceptance in one launch ----------------
// The verify tail after the LM head. Block (g, r) takes the first level's group g of row r exactly as
// topk_level_kernel does and publishes its best k keys and its NaN flag at agent scope (the blocks run on different
// XCDs, whose L2 caches are not coherent with each other), then counts itself in the row's counter once those stores
// have completed. The row's last block reads the row's g1 k keys back (agent scope), reduces them to the final k the
// same way (a wave's best k of its strided share, four lists merged), writes the candidates and the row's NaN flag,
// and counts the row done; the last row's block walks the acceptance on one wave, from the candidates as the other
// blocks stored them. Counters: zero before the first launch, each set back to zero by the block that read it last.
constexpr int kMaxWalkRows = 16;  // the acceptance's rows: drafts (<= 15) + 1

struct TailArgs {
    const float *logits;
    int64_t ld;
    int n_valid, g1, k, rows;
    const uint32_t *mask;
    int64_t mask_words;
    uint64_t *keys;    // [rows][g1][64]: each first-level block's candidates (a superset of its top k; 0: none)
    uint32_t *nan1;    // [rows][g1]
    uint32_t *count;   // [rows + 1]
    sx_logit_cand *cands;
    uint32_t *nan;
    const int32_t *drafts;
    int nd;
    const double *u;
    double temperature;
    int top_k;
    double top_p;
    int32_t *out;
};

__device__ __forceinline__ void store_agent64(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_agent64(const uint64_t *p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_agent32(const uint32_t *p) {
    return __hip_atomic_load(const_cast<uint32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The candidate a final key stands for: padding (-inf, INT32_MAX) for 0, else the key's value and id (a zero is read
// back from the row: the key folds -0 onto +0).
__device__ __forceinline__ sx_logit_cand cand_of(uint64_t best, const float *row) {
    sx_logit_cand c;
    if (best == 0) {
        c.v = -INFINITY, c.id = INT32_MAX;
    } else {
        const uint32_t hi = (uint32_t)(best >> 32);
        c.id = key_id(best);
        c.v = __uint_as_float((hi & 0x80000000u) ? (hi & 0x7FFFFFFFu) : ~hi);
        if (c.v == 0.f) c.v = row[c.id];
    }
    return c;
}

template <bool kMasked>
__global__ void __launch_bounds__(kTopkThreads) topk_accept_kernel(TailArgs a) {
    __shared__ uint64_t scratch[kTopkThreads / 64][kScratch];
    __shared__ uint64_t lists[kTopkThreads / 64][64];
    __shared__ uint32_t s_nan;
    __shared__ int s_last;
    __shared__ BlockTopkLds s_btk;
    __shared__ AcceptLds acc_lds;
    __shared__ uint64_t walk_cands[kMaxWalkRows][64];
    __shared__ uint32_t walk_nan[64];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, g = blockIdx.x;
    const int64_t r = blockIdx.y;
    const int k = a.k;
    const float *row = a.logits + r * a.ld;
    if (t == 0) s_nan = 0;
    uint64_t key[kPer];
    uint32_t my_nan = 0;
    {
        float xv[kPer];
        uint32_t mw[kPer];
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int j = min(g * kGroup + p * kTopkThreads + t, a.n_valid - 1);
            xv[p] = row[j];
            if constexpr (kMasked) mw[p] = a.mask[r * a.mask_words + (j >> 5)];
        }
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int j = g * kGroup + p * kTopkThreads + t;
            key[p] = 0;
            if (j < a.n_valid) {
                const float x = xv[p];
                const bool allowed = !kMasked || ((mw[p] >> (j & 31)) & 1u);
                if (x != x) my_nan = 1u;
                else if (allowed) key[p] = cand_key(x, j);
            }
        }
    }
    __syncthreads();
    if (my_nan) atomicOr(&s_nan, 1u);
    const uint64_t best1 = block_topk<kPer>(key, k, s_btk, scratch, true);
    if (wave == 0) {
        store_agent64(a.keys + (r * a.g1 + g) * 64 + lane, best1);  // up to 64 keys: a superset of the block's top k
        if (lane == 0) __hip_atomic_store(a.nan1 + r * a.g1 + g, s_nan, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the wave's stores have reached the shared level
        if (lane == 0) {
            const uint32_t c = __hip_atomic_fetch_add(a.count + r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = c + 1u == (uint32_t)a.g1;
        }
    }
    __syncthreads();
    if (!s_last) return;

    // the row's last block: its g1 k keys (at most kGroup), every load out before the first use
    const int n = a.g1 * 64;
    const uint64_t *rk = a.keys + r * a.g1 * 64;
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
        const int i = p * kTopkThreads + t;
        key[p] = load_agent64(rk + min(i, n - 1));
    }
    bool f = false;
    if (wave == 0)
        for (int c = lane; c < a.g1; c += 64) f |= load_agent32(a.nan1 + r * a.g1 + c) != 0u;
#pragma unroll
    for (int p = 0; p < kPer; ++p)
        if (p * kTopkThreads + t >= n) key[p] = 0;
    const uint64_t best = block_topk<kPer>(key, k, s_btk, scratch);
    if (wave != 0) return;
    const bool any_nan = __ballot(f) != 0;
    if (lane < k) {
        const sx_logit_cand c = cand_of(best, row);
        store_agent64(reinterpret_cast<uint64_t *>(a.cands + r * k + lane),
                      ((uint64_t)(uint32_t)c.id << 32) | __float_as_uint(c.v));
    }
    if (lane == 0) __hip_atomic_store(a.nan + r, any_nan ? 1u : 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    int last_row = 0;
    if (lane == 0) {
        __hip_atomic_store(a.count + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t c = __hip_atomic_fetch_add(a.count + a.rows, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_row = c + 1u == (uint32_t)a.rows;
    }
    if (!__builtin_amdgcn_readfirstlane(last_row)) return;
    if (lane == 0) __hip_atomic_store(a.count + a.rows, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (a.out == nullptr) return;  // top-k only
    // every row's candidates and NaN flag the walk may read, in one round trip (the other rows' blocks stored them)
    const uint64_t *cw = reinterpret_cast<const uint64_t *>(a.cands);
    const int nr = a.nd + 1;  // <= kMaxWalkRows
    uint64_t pc[kMaxWalkRows];
#pragma unroll
    for (int j = 0; j < kMaxWalkRows; ++j) pc[j] = load_agent64(cw + (int64_t)min(j, nr - 1) * k + min(lane, k - 1));
    const uint32_t pn = load_agent32(a.nan + min(lane, nr - 1));
#pragma unroll
    for (int j = 0; j < kMaxWalkRows; ++j)
        if (j < nr) walk_cands[j][lane] = pc[j];
    walk_nan[lane] = pn;
    wave_sync();
    accept_walk(
        [&](int j, int i) {
            const uint64_t w = walk_cands[j][i];
            sx_logit_cand c;
            c.v = __uint_as_float((uint32_t)w), c.id = (int32_t)(uint32_t)(w >> 32);
            return c;
        },
        [&](int j) { return walk_nan[j]; }, k, a.drafts, a.nd, a.u, a.temperature, a.top_k, a.top_p, a.n_valid,
        a.out, acc_lds);
}

}  // namespace

// ---------------- fixed scratch of the allocation-free entry point ----------------
// sx_logits_topk_noalloc keeps its level candidates in this array instead of a caller's workspace: every device the
// library runs on holds its own copy until the process ends. Its device address comes from hipGetSymbolAddress, once
// per device with that device current; host code never passes the array's name to a kernel (on the host that name
// is only a stand-in, not a device address). Nothing in it needs clearing: each level writes every key and flag the
// next one reads. Calls on one device share it, so two that overlap in time (two streams) race.
static __device__ __align__(256) uint64_t scratch[SX_TOPK_SCRATCH_BYTES / 8];

int topk_scratch(void **ptr) {
    static std::mutex mu;
    static std::vector<void *> per_device;
    int dev = 0;
    SX_HIP(hipGetDevice(&dev), "(allocation-free top-k)");
    std::lock_guard<std::mutex> lock(mu);
    if ((int)per_device.size() <= dev) per_device.resize(dev + 1, nullptr);
    if (per_device[dev] == nullptr) {
        void *p = nullptr;
        SX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "(device ", dev, ")");
        per_device[dev] = p;
    }
    *ptr = per_device[dev];
    return SX_OK;
}


}  // namespace sx

using namespace sx;

extern "C" {

int sx_logits_topk_workspace_bytes(int64_t rows, int64_t n_valid, int64_t k, size_t *bytes) {
    SX_CHECK(bytes != nullptr, "null output");
    SX_CHECK(rows >= 1 && n_valid >= 1 && n_valid <= (1 << 24) && k >= 1 && k <= 64, "rows = ", rows, ", n_valid = ",
             n_valid, ", k = ", k, " (expected rows >= 1, n_valid 1..2^24, k 1..64)");
    const int64_t g1 = groups_of(n_valid);
    *bytes = 2 * (size_t)(rows * g1 * k) * 8 + (size_t)(rows * g1) * 4;
    return SX_OK;
}

int sx_logits_topk(const float *logits, int64_t rows, int64_t ld, int64_t n_valid, int64_t k, sx_logit_cand *out,
                   uint32_t *nan, void *workspace, size_t workspace_bytes, const uint32_t *mask, int64_t mask_words,
                   sx_stream stream) {
    SX_CHECK(logits && out && nan && workspace, "null pointer (logits=", (const void *)logits, ", out=", (void *)out,
             ", nan=", (void *)nan, ", workspace=", workspace, ")");
    SX_CHECK(rows >= 1 && rows <= 65535, "rows = ", rows, ", expected 1..65535");
    SX_CHECK(n_valid >= 1 && n_valid <= (1 << 24), "n_valid = ", n_valid, ", expected 1..2^24");
    SX_CHECK(k >= 1 && k <= 64, "k = ", k, ", expected 1..64");
    SX_CHECK(ld >= n_valid, "row stride ld = ", ld, " < n_valid = ", n_valid);
    size_t need = 0;
    if (int rc = sx_logits_topk_workspace_bytes(rows, n_valid, k, &need)) return rc;
    SX_CHECK(workspace_bytes >= need, "workspace ", workspace_bytes, " bytes, need ", need, " for ", rows, " rows of ",
             n_valid);
    SX_CHECK(aligned(workspace, 8), "workspace must be 8-byte aligned");
    if (mask != nullptr) {
        SX_CHECK(mask_words >= (n_valid + 31) / 32, "mask_words = ", mask_words, " per row covers ", mask_words * 32,
                 " ids, need ", (n_valid + 31) / 32, " words for n_valid = ", n_valid);
        SX_CHECK(aligned(mask, 4), "mask must be 4-byte aligned");
    } else {
        SX_CHECK(mask_words == 0, "mask_words = ", mask_words, " without a mask (pass 0 when mask is null)");
    }
    hipStream_t s = stream_of(stream);
    const int64_t g1 = groups_of(n_valid);
    auto *buf0 = static_cast<uint64_t *>(workspace);
    uint64_t *buf1 = buf0 + rows * g1 * k;
    auto *nan1 = reinterpret_cast<uint32_t *>(buf1 + rows * g1 * k);
    const dim3 grid1((unsigned)g1, (unsigned)rows);
    if (mask != nullptr)
        topk_level_kernel<true, true><<<grid1, kTopkThreads, 0, s>>>(logits, ld, (int)n_valid, nullptr, 0, (int)g1,
                                                                      (int)k, buf0, out, nan1, (int)g1, nan, mask,
                                                                      mask_words);
    else
        topk_level_kernel<true, false><<<grid1, kTopkThreads, 0, s>>>(logits, ld, (int)n_valid, nullptr, 0, (int)g1,
                                                                       (int)k, buf0, out, nan1, (int)g1, nan, nullptr, 0);
    SX_LAUNCHED("logits_topk level 1 rows=", rows, " n_valid=", n_valid);
    uint64_t *cur = buf0;
    for (int64_t groups = g1, level = 2; groups > 1; ++level) {
        const int64_t n_in = groups * k, next = groups_of(n_in);
        uint64_t *dst = cur == buf0 ? buf1 : buf0;
        topk_level_kernel<false, false><<<dim3((unsigned)next, (unsigned)rows), kTopkThreads, 0, s>>>(
            logits, ld, 0, cur, (int)n_in, (int)next, (int)k, dst, out, nan1, (int)g1, nan, nullptr, 0);
        SX_LAUNCHED("logits_topk level ", level, " rows=", rows, " candidates=", n_in);
        cur = dst, groups = next;
    }
    return SX_OK;
}

int sx_logits_topk_noalloc(const float *logits, int64_t rows, int64_t ld, int64_t n_valid, int64_t k,
                           sx_logit_cand *out, uint32_t *nan, const uint32_t *mask, int64_t mask_words,
                           sx_stream stream) {
    size_t need = 0;
    if (int rc = sx_logits_topk_workspace_bytes(rows, n_valid, k, &need)) return rc;
    SX_CHECK(need <= (size_t)SX_TOPK_SCRATCH_BYTES, "the level candidates of ", rows, " rows of ", n_valid,
             " logits at k = ", k, " need ", need, " bytes of scratch; the library's fixed scratch holds ",
             SX_TOPK_SCRATCH_BYTES, " (sx_logits_topk takes a workspace of any size)");
    void *ws = nullptr;
    if (int rc = topk_scratch(&ws)) return rc;
    return sx_logits_topk(logits, rows, ld, n_valid, k, out, nan, ws, need, mask, mask_words, stream);
}

int sx_mtp_pick(const float *logits, int64_t n, const uint32_t *router_err, const uint32_t *expert_err,
                const uint32_t *attn_err, const unsigned long long *emb_err, sx_mtp_pick_t *out, sx_stream stream) {
    SX_CHECK(logits && router_err && expert_err && attn_err && emb_err && out, "null pointer");
    SX_CHECK(n >= 1 && n <= INT_MAX, "n = ", n, " logits, expected 1..", INT_MAX);
    if (n % 4 == 0 && aligned(logits, 16))
        mtp_pick_kernel<true><<<1, kPickThreads, 0, stream_of(stream)>>>(logits, n, router_err, expert_err, attn_err,
                                                                        emb_err, out);
    else
        mtp_pick_kernel<false><<<1, kPickThreads, 0, stream_of(stream)>>>(logits, n, router_err, expert_err, attn_err,
                                                                         emb_err, out);
    SX_LAUNCHED("mtp_pick n=", n);
    return SX_OK;
}

int sx_mtp_pick_ws_bytes(int64_t n, size_t *bytes) {
    SX_CHECK(bytes != nullptr, "null output");
    SX_CHECK(n >= 1 && n <= INT_MAX, "n = ", n, " logits, expected 1..", INT_MAX);
    *bytes = sizeof(pick::Workspace);
    return SX_OK;
}

int sx_mtp_pick_ws(const float *logits, int64_t n, const uint32_t *router_err, const uint32_t *expert_err,
                   const uint32_t *attn_err, const unsigned long long *emb_err, sx_mtp_pick_t *out, void *workspace,
                   size_t workspace_bytes, sx_stream stream) {
    SX_CHECK(logits && router_err && expert_err && attn_err && emb_err && out && workspace, "null pointer");
    SX_CHECK(n >= 1 && n <= INT_MAX, "n = ", n, " logits, expected 1..", INT_MAX);
    SX_CHECK(workspace_bytes >= sizeof(pick::Workspace), "workspace ", workspace_bytes, " bytes, need ",
             sizeof(pick::Workspace));
    SX_CHECK(aligned(workspace, 16), "workspace must be 16-byte aligned");
    hipStream_t s = stream_of(stream);
    const pick::Args a{static_cast<pick::Workspace *>(workspace), router_err, expert_err, attn_err, emb_err, out};
    if (n % 4 == 0 && aligned(logits, 16))
        mtp_pick_ws_kernel<true><<<kPickWsBlocks, kPickWsThreads, 0, s>>>(logits, n, a);
    else
        mtp_pick_ws_kernel<false><<<kPickWsBlocks, kPickWsThreads, 0, s>>>(logits, n, a);
    SX_LAUNCHED("mtp_pick_ws n=", n);
    return SX_OK;
}

int sx_verify_tail_workspace_bytes(int64_t rows, int64_t n_valid, int64_t kc, size_t *bytes) {
    SX_CHECK(bytes != nullptr, "null output");
    SX_CHECK(rows >= 1 && rows <= 65535 && n_valid >= 1 && kc >= 1 && kc <= 64, "rows = ", rows, ", n_valid = ",
             n_valid, ", kc = ", kc);
    const int64_t g1 = groups_of(n_valid);
    SX_CHECK(g1 * 64 <= kGroup, "n_valid = ", n_valid, " leaves ", g1, " first-level groups a row; one launch "
             "reduces at most ", kGroup / 64);
    *bytes = (size_t)(rows * g1 * 64) * 8 + (size_t)(rows * g1) * 4 + (size_t)(rows + 1) * 4;
    return SX_OK;
}

int sx_verify_tail(const float *logits, int64_t rows, int64_t ld, int64_t n_valid, int64_t kc, sx_logit_cand *cands,
                   uint32_t *nan, const uint32_t *mask, int64_t mask_words, const int32_t *drafts, int64_t k,
                   const double *u, double temperature, int64_t top_k, double top_p, int32_t *out, void *workspace,
                   size_t workspace_bytes, sx_stream stream) {
    SX_CHECK(logits && cands && nan && workspace, "null pointer");
    SX_CHECK(ld >= n_valid, "row stride ld = ", ld, " < n_valid = ", n_valid);
    size_t need = 0;
    if (int rc = sx_verify_tail_workspace_bytes(rows, n_valid, kc, &need)) return rc;
    SX_CHECK(workspace_bytes >= need, "workspace ", workspace_bytes, " bytes, need ", need);
    SX_CHECK(aligned(workspace, 8) && aligned(cands, 8), "workspace and cands must be 8-byte aligned");
    if (mask != nullptr) {
        SX_CHECK(mask_words >= (n_valid + 31) / 32, "mask_words = ", mask_words, " per row covers ", mask_words * 32,
                 " ids, need ", (n_valid + 31) / 32, " words for n_valid = ", n_valid);
        SX_CHECK(aligned(mask, 4), "mask must be 4-byte aligned");
    } else {
        SX_CHECK(mask_words == 0, "mask_words = ", mask_words, " without a mask (pass 0 when mask is null)");
    }
    if (out != nullptr) {  // the acceptance's preconditions (sx_mtp_accept's)
        SX_CHECK(k >= 0 && k <= 15 && (k == 0 || drafts), "k = ", k, " drafts, expected 0..15 (drafts non-null)");
        SX_CHECK(rows >= k + 1, "rows = ", rows, ": one candidate row per draft plus the last");
        SX_CHECK(temperature >= 0 && temperature <= 100, "temperature ", temperature, ", expected 0..100");
        SX_CHECK(top_p > 0 && top_p <= 1, "top_p ", top_p, ", expected (0, 1]");
        SX_CHECK(kc >= (n_valid < 20 ? n_valid : 20), "kc = ", kc, " candidates, the sampler needs min(n_valid, 20)");
        if (temperature > 0) {
            SX_CHECK(u != nullptr, "sampled acceptance needs the host's uniform draws");
            SX_CHECK(top_k >= 1 && top_k <= kc, "top_k = ", top_k, " must be 1..", kc);
        }
    }
    const int64_t g1 = groups_of(n_valid);
    TailArgs a{};
    a.logits = logits, a.ld = ld, a.n_valid = (int)n_valid, a.g1 = (int)g1, a.k = (int)kc, a.rows = (int)rows;
    a.mask = mask, a.mask_words = mask_words;
    a.keys = static_cast<uint64_t *>(workspace);
    a.nan1 = reinterpret_cast<uint32_t *>(a.keys + rows * g1 * 64);
    a.count = a.nan1 + rows * g1;
    a.cands = cands, a.nan = nan;
    a.drafts = drafts, a.nd = (int)k, a.u = u, a.temperature = temperature, a.top_k = (int)top_k, a.top_p = top_p;
    a.out = out;
    const dim3 grid((unsigned)g1, (unsigned)rows);
    if (mask != nullptr) topk_accept_kernel<true><<<grid, kTopkThreads, 0, stream_of(stream)>>>(a);
    else topk_accept_kernel<false><<<grid, kTopkThreads, 0, stream_of(stream)>>>(a);
    SX_LAUNCHED("verify_tail rows=", rows, " n_valid=", n_valid);
    return SX_OK;
}

int sx_mtp_accept(const sx_logit_cand *cands, const uint32_t *nan, int64_t kc, const int32_t *drafts, int64_t k,
                  const double *u, double temperature, int64_t top_k, double top_p, int64_t n_valid, int32_t *out,
                  sx_stream stream) {
    SX_CHECK(cands && nan && out && (k == 0 || drafts), "null pointer");
    SX_CHECK(k >= 0 && k <= 15, "k = ", k, " drafts, expected 0..15 (mtp-draft's range)");
    SX_CHECK(kc >= 1 && kc <= 64, "kc = ", kc, " candidates a row, expected 1..64");
    SX_CHECK(n_valid >= 1, "n_valid = ", n_valid);
    SX_CHECK(temperature >= 0 && temperature <= 100, "temperature ", temperature, ", expected 0..100");
    SX_CHECK(top_p > 0 && top_p <= 1, "top_p ", top_p, ", expected (0, 1]");
    SX_CHECK(kc >= (n_valid < 20 ? n_valid : 20), "kc = ", kc, " candidates, the sampler needs min(n_valid, 20)");
    if (temperature > 0) {
        SX_CHECK(u != nullptr, "sampled acceptance needs the host's uniform draws");
        SX_CHECK(top_k >= 1 && top_k <= kc, "top_k = ", top_k, " must be 1..", kc,
                 " (the candidates a row; top_k off needs the whole row)");
    }
    mtp_accept_kernel<<<1, 64, 0, stream_of(stream)>>>(cands, nan, (int)kc, drafts, (int)k, u, temperature,
                                                       (int)top_k, top_p, n_valid, out);
    SX_LAUNCHED("mtp_accept k=", k);
    return SX_OK;
}

}  // extern "C"
