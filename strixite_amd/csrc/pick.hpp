// The MTP draft pick's reduction (kernels/mtp_pick.hpp:20-33): a running top-2 with a NaN flag, its merge, and the
// many-block form in which every block of a launch reduces its share and the last block to finish writes the pick.
// Used by the pick kernels (topk.hip) and by the dense GEMV's fused draft-head epilogue (dense_ks.hip).
#pragma once
#include "common.hpp"

#include <climits>

namespace sx::pick {

struct Top2 {
    float b1, b2;
    int i1;  // INT_MAX: nothing seen
    uint32_t nan;
};

__device__ __forceinline__ Top2 top2_none() { return Top2{-INFINITY, -INFINITY, INT_MAX, 0u}; }

// The larger best (the lower index of equal ones), the larger of the runners-up, either NaN flag: associative and
// commutative, so a pick does not depend on how its values were split or merged.
__device__ __forceinline__ Top2 top2_merge(const Top2 a, const Top2 b) {
    const bool a_none = a.i1 == INT_MAX, b_none = b.i1 == INT_MAX;
    const bool a_wins = b_none || (!a_none && (a.b1 > b.b1 || (a.b1 == b.b1 && a.i1 < b.i1)));
    // value selects without branches (branches and selects of whole operands put them in private memory)
    const float wb1 = a_wins ? a.b1 : b.b1, wb2 = a_wins ? a.b2 : b.b2, lb1 = a_wins ? b.b1 : a.b1;
    // the loser's best is at least its own runner-up; an empty side adds nothing
    return {wb1, (a_none || b_none) ? wb2 : fmaxf(wb2, lb1), a_wins ? a.i1 : b.i1, a.nan | b.nan};
}

__device__ __forceinline__ Top2 top2_xor(const Top2 &p, int off) {
    return {__shfl_xor(p.b1, off), __shfl_xor(p.b2, off), __shfl_xor(p.i1, off),
            (uint32_t)__shfl_xor((int)p.nan, off)};
}

// One value into a thread's running top-2 (indices offered in ascending order: the strict > keeps the lower index of
// equal values).
__device__ __forceinline__ void top2_take(Top2 &p, float v, int64_t i) {
    if (v != v) {
        p.nan = 1u;
        return;
    }
    if (p.i1 == INT_MAX || v > p.b1) p.b2 = p.b1, p.b1 = v, p.i1 = (int)i;
    else if (v > p.b2) p.b2 = v;
}

__device__ __forceinline__ Top2 wave_merge(Top2 p) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) p = top2_merge(p, top2_xor(p, off));
    return p;
}

// The forward's error words a pick carries, read by lanes 0-2 of a wave (lane 0 also the embedding's).
struct ErrWords {
    uint32_t r, e, a;
    unsigned long long emb;
};
__device__ __forceinline__ ErrWords read_errs(int lane, const uint32_t *router_err, const uint32_t *expert_err,
                                              const uint32_t *attn_err, const unsigned long long *emb_err) {
    ErrWords w{0u, 0u, 0u, 0ull};
    if (lane < 3) w.r = router_err[lane], w.e = expert_err[lane], w.a = attn_err[lane];
    if (lane == 0) w.emb = *emb_err;
    return w;
}

// The pick's 64 bytes from the merged top-2 and the error words (lanes 0-2 of one wave).
__device__ __forceinline__ void write_pick(const Top2 &p, int lane, const ErrWords &w, sx_mtp_pick_t *out) {
    if (lane == 0) {
        out->best = p.i1 == INT_MAX ? 0 : p.i1;  // every logit NaN: 0, flagged
        out->best_v = p.b1, out->second_v = p.b2, out->nan = p.nan;
        out->pad = 0;
        out->emb = w.emb;
    }
    if (lane < 3) out->err[lane] = w.r, out->err[3 + lane] = w.e, out->err[6 + lane] = w.a;
}

// The many-block pick's workspace: a partial a block, and the count of blocks done. The count starts at 0 (the
// workspace is zeroed before its first use) and the last block of each launch sets it back to 0.
constexpr int kMaxParts = 256;
struct Workspace {
    Top2 part[kMaxParts];
    uint32_t count;
    uint32_t pad[3];
};

struct Args {
    Workspace *ws;  // nullptr: no pick
    const uint32_t *router_err, *expert_err, *attn_err;
    const unsigned long long *emb_err;
    sx_mtp_pick_t *out;
};

// Every thread of the block calls this with its top-2 (WAVES waves, gridDim.x <= kMaxParts blocks, at a point every
// thread reaches), wave 0 with the error words (read_errs, loaded early: the last block does not wait for them). The
// block's partial goes out with agent-scope stores (written through to the level every XCD shares: the blocks run on
// different XCDs, whose L2 caches are not coherent with each other) and is counted only once those stores have
// completed; the block that counts last reads every partial with agent-scope loads, writes
// the pick and resets the count.
template <int WAVES>
__device__ void block_pick(Top2 p, const Args &a, const ErrWords &errs, Top2 *red /* LDS [WAVES] */,
                           int *last /* LDS */) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    p = wave_merge(p);
    if (lane == 0) red[wave] = p;
    __syncthreads();
    if (tid == 0) {
        Top2 q = red[0];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) q = top2_merge(q, red[w]);
        Top2 *dst = a.ws->part + blockIdx.x;
        __hip_atomic_store(&dst->b1, q.b1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&dst->b2, q.b2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&dst->i1, q.i1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&dst->nan, q.nan, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the partial has reached the shared level
        const uint32_t c = __hip_atomic_fetch_add(&a.ws->count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last = c + 1u == gridDim.x;
    }
    __syncthreads();
    if (!*last || wave != 0) return;
    // every partial's loads go out before any is used (one round trip)
    constexpr int kPer = kMaxParts / 64;
    Top2 q[kPer];
    const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(a.ws->part, (short)0, (int)sizeof(a.ws->part), 0x00020000);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int b = lane + 64 * j;
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (b < (int)gridDim.x ? b : 0) * (int)sizeof(Top2),
                                                             0, 16 /* sc1: agent scope */);
        q[j] = Top2{__uint_as_float(v[0]), __uint_as_float(v[1]), (int)v[2], v[3]};
        if (b >= (int)gridDim.x) q[j] = top2_none();
    }
    Top2 m = q[0];
#pragma unroll
    for (int j = 1; j < kPer; ++j) m = top2_merge(m, q[j]);
    m = wave_merge(m);
    write_pick(m, lane, errs, a.out);
    if (lane == 0) __hip_atomic_store(&a.ws->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace sx::pick
