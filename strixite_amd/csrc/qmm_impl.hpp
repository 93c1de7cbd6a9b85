// Skinny dequantizing GEMM on the matrix cores: the kernel template (see qmm.hpp for the scheme). Each qmm_mN.hip
// instantiates one mode, so the instantiations compile in parallel.
#pragma once
#include "qmm.hpp"

#include <type_traits>

namespace sx::qmm {
namespace detail {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kPrefetch = 8;  // steps (16-byte loads a lane) a group
constexpr int kRing = 1;      // groups in flight a wave (fast path)
constexpr int kStageLoads = 8;  // activation chunk loads in flight a thread while staging
constexpr int kZeroBytes = 2048;  // zero A operand for a group of idle-lane reads (8 q4 spans of BF16)

template <int BITS>
struct Fmt {
    static constexpr int kSpanCodes = BITS == 4 ? 128 : 64;
    static constexpr int kMfmas = BITS == 4 ? 4 : 2;  // MFMAs a span (8 codes a lane each)
    static constexpr float kOff = BITS == 4 ? 128.f : 0.f;
};

__device__ __forceinline__ uint32_t dword(const uint4 &w, int i) { return i == 0 ? w.x : i == 1 ? w.y : i == 2 ? w.z : w.w; }

template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of `lanes` (1, 2, 4, 8 or 16; uniform) lanes, every lane of a group getting the total.
// DPP butterflies inside a row: quad [1,0,3,2], quad [2,3,0,1], half-row mirror, row mirror (a mirror pairs two
// halves whose lanes already hold their half's sum, so it adds like an xor partner).
__device__ __forceinline__ float group_sum(float v, int lanes) {
    if (lanes >= 2) v = dpp_add<0xB1>(v);
    if (lanes >= 4) v = dpp_add<0x4E>(v);
    if (lanes >= 8) v = dpp_add<0x141>(v);
    if (lanes >= 16) v = dpp_add<0x140>(v);
    return v;
}

// (a & mask) | (b & ~mask) in one ALU operation (v_bitop3_b32, truth table 0xCA: S0 ? S1 : S2 bit by bit): the code
// nibbles under the BF16 exponent bits of 128. An intrinsic rather than inline asm, so the wait-count pass covers
// its operands (these often come straight from the code loads; it does not look at an asm statement's operands).
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) {
    return __builtin_amdgcn_bitop3_b32(mask, a, b, 0xCA);
}

// B operand of MFMA t from a lane's 16 code bytes. q4: dword t's nibbles j = 0..7 (code k0 + j) as BF16 128 + code in
// element order [0, 4, 1, 5, 2, 6, 3, 7] - one v_and_or (plus a shift) a pair. q8: dwords 2t, 2t+1 in byte order.
template <int BITS>
__device__ __forceinline__ bf16x8 codes_b(const uint4 &w, int t) {
    uint4 v;
    if constexpr (BITS == 4) {
        const uint32_t d = dword(w, t), d4 = d >> 4;
        v.x = bfi(0x000F000Fu, d, 0x43004300u);
        v.y = bfi(0x000F000Fu, d4, 0x43004300u);
        v.z = bfi(0x000F000Fu, d >> 8, 0x43004300u);
        v.w = bfi(0x000F000Fu, d >> 12, 0x43004300u);
    } else {
        const uint32_t d0 = dword(w, 2 * t), d1 = dword(w, 2 * t + 1);
        auto pair = [](uint32_t d, int b) {  // bytes b, b+1 -> BF16 pair (exact: <= 8 significant bits)
            const uint32_t lo = __float_as_uint((float)((d >> (8 * b)) & 0xFFu));
            const uint32_t hi = __float_as_uint((float)((d >> (8 * b + 8)) & 0xFFu));
            return (lo >> 16) | (hi & 0xFFFF0000u);
        };
        v.x = pair(d0, 0), v.y = pair(d0, 2), v.z = pair(d1, 0), v.w = pair(d1, 2);
    }
    return __builtin_bit_cast(bf16x8, v);
}

template <int LANES>
__device__ __forceinline__ float group_sum_c(float v) {
    if constexpr (LANES >= 2) v = dpp_add<0xB1>(v);
    if constexpr (LANES >= 4) v = dpp_add<0x4E>(v);
    if constexpr (LANES >= 8) v = dpp_add<0x141>(v);
    if constexpr (LANES >= 16) v = dpp_add<0x140>(v);
    return v;
}

// LDS position of code offset j (0..7) within an 8-code run, matching codes_b's element order.
template <int BITS>
__device__ __forceinline__ int lds_pos(int j) {
    if constexpr (BITS == 4) return (j & 3) * 2 + (j >> 2);  // inverse of [0, 4, 1, 5, 2, 6, 3, 7]
    else return j;
}

// FP32 -> NSPLIT BF16 terms whose sum is the value: hi = rne(x), mid = rne(x - hi), lo = rne(x - hi - mid)
// (exact differences: each step leaves <= 16 significant bits). One term for BF16 inputs.
template <int NSPLIT>
__device__ __forceinline__ void split(float x, uint16_t (&t)[NSPLIT]) {
    float r = x;
#pragma unroll
    for (int i = 0; i < NSPLIT; ++i) {
        const uint32_t b = f32_to_bf16(r);
        t[i] = (uint16_t)b;
        r = r - bf16_to_f32(b);
    }
}

// 8 activation elements as loaded (BF16: one 16-byte load; FP32: two), widened to FP32 when used.
struct F32x8 {
    float4 a, b;
};
template <typename TX>
using Raw8 = std::conditional_t<sizeof(TX) == 4, F32x8, uint4>;

template <typename TX>
__device__ __forceinline__ Raw8<TX> load_raw8(const TX *p) {
    if constexpr (sizeof(TX) == 4) return F32x8{reinterpret_cast<const float4 *>(p)[0], reinterpret_cast<const float4 *>(p)[1]};
    else return reinterpret_cast<const uint4 *>(p)[0];
}

__device__ __forceinline__ void unpack8(const F32x8 &u, float (&v)[8]) {
    v[0] = u.a.x, v[1] = u.a.y, v[2] = u.a.z, v[3] = u.a.w, v[4] = u.b.x, v[5] = u.b.y, v[6] = u.b.z, v[7] = u.b.w;
}
__device__ __forceinline__ void unpack8(const uint4 &u, float (&v)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t w = dword(u, i);
        v[2 * i] = __uint_as_float(w << 16), v[2 * i + 1] = __uint_as_float(w & 0xFFFF0000u);
    }
}

// One staged 8-element chunk: its NSPLIT BF16 planes in the B operand's code order and its FP32 sum. BF16 input
// needs no rounding: q4's order [0, 4, 1, 5, 2, 6, 3, 7] is four byte selects, q8's is the input order.
template <int BITS, int NSPLIT, typename TX>
__device__ __forceinline__ void chunk_planes(const Raw8<TX> &raw, uint4 (&out)[NSPLIT], float &sum) {
    float v[8];
    unpack8(raw, v);
    sum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += v[j];
    if constexpr (sizeof(TX) == 2 && NSPLIT == 1) {
        if constexpr (BITS == 4) {
            out[0] = uint4{__builtin_amdgcn_perm(raw.z, raw.x, 0x05040100u), __builtin_amdgcn_perm(raw.z, raw.x, 0x07060302u),
                           __builtin_amdgcn_perm(raw.w, raw.y, 0x05040100u), __builtin_amdgcn_perm(raw.w, raw.y, 0x07060302u)};
        } else {
            out[0] = raw;
        }
    } else {
        uint16_t planes[NSPLIT][8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint16_t t[NSPLIT];
            split<NSPLIT>(v[j], t);
#pragma unroll
            for (int s = 0; s < NSPLIT; ++s) planes[s][lds_pos<BITS>(j)] = t[s];
        }
#pragma unroll
        for (int s = 0; s < NSPLIT; ++s) out[s] = *reinterpret_cast<const uint4 *>(planes[s]);
    }
}

constexpr bool is_swiglu(int m) { return m == SWIGLU || m == SLOT_SWIGLU; }
constexpr bool is_slot(int m) { return m >= SLOT_GATHER; }

template <int BITS, int NSPLIT, int MODE, typename TX, typename TY>
__global__ void __launch_bounds__(kThreads) qmm_kernel(Params p) {
    using F = Fmt<BITS>;
    constexpr int NW = is_swiglu(MODE) ? 2 : 1;  // weight tiles a step: gate and up
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    __shared__ int64_t s_xrow[64], s_out[16], s_wrow[64];
    __shared__ float s_coef[64];
    __shared__ int s_T, s_R, s_bad;

    const int64_t K = p.K;
    const int G = p.G;
    const int nspan = (int)((K + F::kSpanCodes - 1) / F::kSpanCodes);  // the last span may hold 1-3 quarters
    const int qlast = (int)(K % F::kSpanCodes) / (F::kSpanCodes / 4);      // its quarters, 0 = all four
    const int run = G < F::kSpanCodes ? G : F::kSpanCodes;     // codes a partial sum covers
    const int nruns = (int)(K / run);
    const int ngs = F::kSpanCodes / run;                         // groups a span
    const int TP = 16 / ngs;                                     // activation rows a pass
    const int64_t ldx = K + 8;                                   // LDS row stride (BF16 elements)
    const int64_t rowbytes = BITS == 4 ? K / 2 : K;
    const int64_t ngroups = K / G;
    const int64_t Nrows = is_swiglu(MODE) ? p.N / 2 : p.N;      // output rows per expert
    const int unit = (int)(blockIdx.x / (unsigned)p.nchunks), chunk = (int)(blockIdx.x % (unsigned)p.nchunks);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps the loop control scalar

    // ---- the unit: its activation rows, output rows and expert. Wave 0 decodes it, lane r filling row r, so a
    // unit costs one or two dependent memory latencies rather than one a row. ----
    if (tid < 64) {
        const int l = tid;
        int T = 0, R = 0, bad = 0;
        if constexpr (MODE == DENSE) {
            const int64_t m0 = (int64_t)blockIdx.y * p.max_rows;
            T = (int)min((int64_t)p.max_rows, p.M - m0);
            if (l < T) s_xrow[l] = (m0 + l) * K, s_out[l] = (m0 + l) * p.N;
            if (l == 0) s_wrow[0] = 0;
            R = T;
        } else if constexpr (!is_slot(MODE)) {
            const int32_t *ws = p.ws;
            const int32_t n_tiles = ws[0], S = ws[1], E = ws[2];
            if (unit < n_tiles) {
                const int32_t *offsets = ws + 4, *slots = offsets + E + 2, *tile_bucket = slots + S;
                const int64_t Tmax = (int64_t)S / 16 + E + 2;
                const int32_t *tile_start = tile_bucket + Tmax;
                const int32_t bucket = tile_bucket[unit], st = tile_start[unit];
                T = min(16, offsets[bucket + 1] - st);
                if (l < T) {
                    const int64_t slot = slots[st + l];
                    s_xrow[l] = (MODE == COMBINE ? slot : slot / p.A) * K;
                    s_out[l] = slot * Nrows;
                }
                bad = bucket == E;
                if (l == 0) s_wrow[0] = (int64_t)bucket * p.N;
                R = T;
            }
        } else if constexpr (MODE != SLOT_COMBINE) {
            const int64_t slot = unit;
            const int32_t id = p.ids[slot];
            T = 1, R = 1;
            bad = !(id >= 0 && id < p.E);
            if (l == 0) {
                if (bad && chunk == 0) flag_error(p.err, (uint32_t)id, (uint32_t)slot);
                s_xrow[0] = (slot / p.A) * K, s_out[0] = slot * Nrows, s_wrow[0] = (int64_t)id * p.N;
            }
        } else {
            const int64_t m = unit;
            T = 1, R = (int)p.A;
            bool ok = true;
            int32_t id = 0;
            if (l < R) {
                id = p.ids[m * p.A + l];
                ok = id >= 0 && id < p.E;
                s_xrow[l] = (m * p.A + l) * K, s_wrow[l] = (int64_t)id * p.N, s_coef[l] = p.coef[m * p.A + l];
            }
            const uint64_t bad_lanes = __ballot(!ok);
            bad = bad_lanes != 0;
            // the first bad slot of the token is the one reported
            if (bad && chunk == 0 && l == __builtin_ctzll(bad_lanes)) flag_error(p.err, (uint32_t)id, (uint32_t)(m * p.A + l));
            if (l == 0) s_out[0] = m * p.N;
        }
        if (l == 0) s_T = T, s_R = R, s_bad = bad;
    }
    __syncthreads();
    const int T_all = __builtin_amdgcn_readfirstlane(s_T), R = __builtin_amdgcn_readfirstlane(s_R);
    if (T_all == 0) return;  // an over-provisioned grouped unit: uniform for the block
    const int tiles_total = (int)((Nrows + kTile - 1) / kTile);
    const int tile0 = chunk * p.tiles_per_chunk;
    const int tiles_here = min(p.tiles_per_chunk, tiles_total - tile0);
    if (tiles_here <= 0) return;

    if (__builtin_amdgcn_readfirstlane(s_bad)) {  // invalid expert id: NaN outputs, never an out-of-bounds weight read
        const int64_t rows = (int64_t)tiles_here * kTile;
        for (int64_t i = tid; i < rows * T_all; i += kThreads) {
            const int r = (int)(i / rows);
            const int64_t n = (int64_t)tile0 * kTile + i % rows;
            if (n >= Nrows) continue;
            if constexpr (MODE == COMBINE) static_cast<float *>(p.y)[s_out[r] + n] = qnan();
            else store_act(static_cast<TY *>(p.y), s_out[r] + n, qnan());
        }
        return;
    }

    const int cap = p.max_rows;                               // activation rows staged at once
    const int lds_rows = MODE == SLOT_COMBINE ? R : cap;      // LDS plane height
    const int nruns_pad = nspan * ngs;                        // run sums padded to whole spans (zeros past K)
    uint16_t *xs = reinterpret_cast<uint16_t *>(smem);
    float *xsum = reinterpret_cast<float *>(smem + (size_t)NSPLIT * lds_rows * ldx * 2);
    uint16_t *zero_block = reinterpret_cast<uint16_t *>(xsum + (size_t)(MODE == SLOT_COMBINE ? R : 1) * nruns_pad * 16);
    for (int i = tid; i < kZeroBytes / 4; i += kThreads) reinterpret_cast<float *>(zero_block)[i] = 0.f;  // A of idle lanes
    const int pad_entries = (nruns_pad - nruns) * 16;
    for (int i = tid; i < (MODE == SLOT_COMBINE ? R : 1) * pad_entries; i += kThreads)
        xsum[(size_t)(i / pad_entries) * nruns_pad * 16 + (size_t)nruns * 16 + i % pad_entries] = 0.f;
    const TX *x = static_cast<const TX *>(p.x);
    const int chunks8 = (int)(K / 8), lanes_per_run = run / 8;

    // ---- each wave: its tiles of the chunk, every activation pass, all spans (and SLOT_COMBINE's slots) ----
    // Steps run tile by tile; within a tile pass by pass, segment by segment (SLOT_COMBINE's slots), span by span,
    // and for SwiGLU gate then up for each span. Nothing reads a loaded value before its step comes up, so the loads
    // stay in flight across spans and tiles. Loop control is wave-uniform (scalar); row pointers change only at tile /
    // segment boundaries.
    const int n16 = lane & 15, g = lane >> 4;
    const int lg_ngs = ngs == 1 ? 0 : ngs == 2 ? 1 : 2;
    const int gam = (g << lg_ngs) >> 2;             // this lane-quarter's group within a span
    const int gshift = G > F::kSpanCodes ? 1 : 0;   // q8 G = 128: two spans a group
    const int nseg = MODE == SLOT_COMBINE ? R : 1;  // weight segments a tile (SLOT_COMBINE: one per slot)
    const int my_tiles = (tiles_here - wave + kWaves - 1) / kWaves;
    const uint16_t *xrow0 = xs + (size_t)g * (F::kSpanCodes / 4);
    const bool a_lane = (n16 / TP) == gam;  // this lane's A row belongs to its quarter's group
    const int64_t up_q = NW == 2 ? Nrows * rowbytes : 0, up_g = NW == 2 ? Nrows * ngroups : 0;
    int npass = (min(cap, T_all) + TP - 1) / TP;  // activation passes of the current batch

    // ---- fast path: a tile is a whole number of groups (kPrefetch steps), K a whole number of spans, and a span
    // inside one quantization group. A group never crosses a row, segment or pass, so its kPrefetch steps are
    // straight-line code with immediate span offsets. kRing groups are in flight: while group g is consumed, the code
    // loads of group g + kRing go out step by step into the registers g's steps free. A group's scales and mins
    // arrive as one contiguous window per row (8 or 16 bytes). (q4 K = 4096 / 1024, G = 128 and q8 K = 4096,
    // G = 64 / 128 all qualify.)
    constexpr int SPG = kPrefetch / NW;  // spans a group = quantization groups it covers (G is one span)
    const bool fast = qlast == 0 && ngs == 1 && gshift == 0 && ngroups % SPG == 0 && nspan % SPG == 0;
    uint4 ring[kRing][kPrefetch];
    uint4 sw_n[kRing][NW], mw_n[kRing][NW];
    int ic = 0, ia = 0, ip = 0, ii = 0;  // issue cursor: span, segment, pass, tile
    const uint8_t *iq;
    const uint16_t *is_, *im;
    auto iplace = [&]() {
        const int64_t n = (int64_t)(tile0 + wave + ii * kWaves) * kTile + n16;
        const int64_t nn = n < Nrows ? n : Nrows - 1;  // a partial last tile reads a valid row, stores nothing
        const int64_t row = (MODE == SLOT_COMBINE ? s_wrow[ia] : s_wrow[0]) + nn;
        iq = p.q + row * rowbytes + g * 16;
        is_ = p.scale + row * ngroups;
        im = p.minv + row * ngroups;
    };
    auto advance_issue = [&]() {
        if (ic + SPG < nspan) {
            ic += SPG;
            return;
        }
        ic = 0;
        if (++ia >= nseg) {
            ia = 0;
            if (++ip >= npass) ip = 0, ++ii;
        }
        iplace();
    };
    // the group at the issue cursor into ring slot r: one code load a step, one scale / min window per row
    auto issue_slot = [&](uint4 (&slot)[kPrefetch], int s) {
        const int span = ic + s / NW, w = s % NW;
        slot[s] = *reinterpret_cast<const uint4 *>(iq + (w ? up_q : 0) + (int64_t)span * kSpanBytes);
    };
    auto issue_window = [&](uint4 (&sw)[NW], uint4 (&mw)[NW]) {  // SPG BF16 scales and mins from group ic
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const uint16_t *sp_ = is_ + (w ? up_g : 0) + ic, *mp_ = im + (w ? up_g : 0) + ic;
            if constexpr (SPG == 8) {
                sw[w] = *reinterpret_cast<const uint4 *>(sp_);
                mw[w] = *reinterpret_cast<const uint4 *>(mp_);
            } else {
                const uint2 a = *reinterpret_cast<const uint2 *>(sp_), b = *reinterpret_cast<const uint2 *>(mp_);
                sw[w] = uint4{a.x, a.y, 0u, 0u}, mw[w] = uint4{b.x, b.y, 0u, 0u};
            }
        }
    };
    int groups = 0;  // groups of steps the wave consumes in the current batch
    auto prime = [&]() {
        ic = 0, ia = 0, ip = 0, ii = 0;
        iplace();
#pragma unroll
        for (int r = 0; r < kRing; ++r) {
            if (r > 0 && r < groups) advance_issue();  // past the last group a slot re-loads it (never used)
            issue_window(sw_n[r], mw_n[r]);
#pragma unroll
            for (int s = 0; s < kPrefetch; ++s) issue_slot(ring[r], s);
        }
    };

    // ---- staging the activation rows in LDS: NSPLIT BF16 planes in the B operand's code order, and run sums ----
    // Item i is the 8-element chunk c8 of staged row r. kThreads and chunks8 are multiples of lanes_per_run, so a
    // run's lanes are all in or all out of a round.
    auto item_src = [&](int i, int b0) {
        const int r = i / chunks8, c8 = i % chunks8;
        return x + s_xrow[MODE == SLOT_COMBINE ? r : b0 + r] + (int64_t)c8 * 8;
    };
    auto write_item = [&](const Raw8<TX> &raw, int i) {
        const int r = i / chunks8, c8 = i % chunks8;
        float v[8];
        unpack8(raw, v);
        uint16_t planes[NSPLIT][8];
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint16_t t[NSPLIT];
            split<NSPLIT>(v[j], t);
#pragma unroll
            for (int s = 0; s < NSPLIT; ++s) planes[s][lds_pos<BITS>(j)] = t[s];
            sum += v[j];
        }
#pragma unroll
        for (int s = 0; s < NSPLIT; ++s)
            *reinterpret_cast<uint4 *>(xs + ((size_t)s * lds_rows + r) * ldx + (int64_t)c8 * 8) =
                *reinterpret_cast<const uint4 *>(planes[s]);
        sum = group_sum(sum, lanes_per_run);
        if (c8 % lanes_per_run == 0) {
            const int rn = c8 / lanes_per_run;
            if constexpr (MODE == SLOT_COMBINE) xsum[((size_t)r * nruns_pad + rn) * 16] = sum;
            else xsum[(size_t)rn * 16 + r] = sum;
        }
    };
    // Rounds of kStageLoads chunks a thread, all of a round's loads issued before the first is used.
    auto stage = [&](int b0, int Rb) {
        const int n_items = Rb * chunks8;
        for (int i0 = 0; i0 < n_items; i0 += kThreads * kStageLoads) {
            Raw8<TX> raw[kStageLoads];
#pragma unroll
            for (int b = 0; b < kStageLoads; ++b) raw[b] = load_raw8(item_src(min(i0 + b * kThreads + tid, n_items - 1), b0));
#pragma unroll
            for (int b = 0; b < kStageLoads; ++b) {
                const int i = i0 + b * kThreads + tid;
                if (i >= n_items) break;
                write_item(raw[b], i);
            }
        }
    };

    constexpr int kStageMax = sizeof(TX) == 4 ? 4 : 12;  // chunks a thread the fast path stages in one round
    if (fast && T_all <= cap && (MODE == SLOT_COMBINE ? R : T_all) * chunks8 <= kThreads * kStageMax &&
        (chunks8 & (chunks8 - 1)) == 0) {
        // One batch, one staging round, straight-line: the activation loads go out first, then the weight loads of
        // the wave's first kRing groups, and the LDS writes wait for the activations only, so the weights' latency
        // and the staging overlap. (Loads complete in order; with no loop in between the waits are exact.)
        const int T = T_all, b0 = 0;
        npass = (T + TP - 1) / TP;
        const int total = my_tiles * npass * nseg * nspan * NW;
        groups = total / kPrefetch;
        const int n_items = (MODE == SLOT_COMBINE ? R : T) * chunks8;
        // Item i is chunk (i & (chunks8 - 1)) of staged row i >> lg_chunks (chunks8 is a power of two here).
        const int lg_chunks = __builtin_ctz((unsigned)chunks8);
        constexpr int kLanesRun = F::kSpanCodes / 8;  // lanes a run sum spans (a run is one span here)
        // NB chunk loads a thread (the fewest of 2, 4, 8, 12 that cover the rows), then the ring, then the LDS writes.
        // Each size is its own straight-line arm ending in the same ring loads, so every wait stays exact.
        auto stage_and_prime = [&](auto nb_tag) {
            constexpr int NB = decltype(nb_tag)::value;
            Raw8<TX> raw[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b) {  // past n_items: a repeat of the last chunk (one cache line), unused
                const int i = min(b * kThreads + tid, n_items - 1);
                raw[b] = load_raw8(x + s_xrow[i >> lg_chunks] + (int64_t)(i & (chunks8 - 1)) * 8);
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weight loads
            prime();  // unconditional (a wave without tiles reads a clamped, valid row): a branch here would make the
                      // activation waits below count the weight loads too
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int i = b * kThreads + tid;
                if (i < n_items) {  // a run's lanes are all in or all out (kThreads, chunks8 are multiples of kLanesRun)
                    const int r = i >> lg_chunks, c8 = i & (chunks8 - 1);
                    uint4 planes[NSPLIT];
                    float sum;
                    chunk_planes<BITS, NSPLIT, TX>(raw[b], planes, sum);
#pragma unroll
                    for (int sp = 0; sp < NSPLIT; ++sp)
                        *reinterpret_cast<uint4 *>(xs + ((size_t)sp * lds_rows + r) * ldx + (int64_t)c8 * 8) = planes[sp];
                    sum = group_sum_c<kLanesRun>(sum);
                    if ((c8 & (kLanesRun - 1)) == 0) {
                        const int rn = c8 / kLanesRun;
                        if constexpr (MODE == SLOT_COMBINE) xsum[((size_t)r * nruns_pad + rn) * 16] = sum;
                        else xsum[(size_t)rn * 16 + r] = sum;
                    }
                }
            }
        };
        const int nb = (n_items + kThreads - 1) / kThreads;  // uniform
        if (nb <= 2) stage_and_prime(std::integral_constant<int, 2>{});
        else if (nb <= 4) stage_and_prime(std::integral_constant<int, 4>{});
        else if (kStageMax > 4 && nb <= 8) stage_and_prime(std::integral_constant<int, (kStageMax > 4 ? 8 : 4)>{});
        else stage_and_prime(std::integral_constant<int, kStageMax>{});
        __syncthreads();
        if (my_tiles <= 0) return;
        int cc = 0, ca = 0, cp = 0, ci = 0;  // consume cursor
        f32x4 acc[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) acc[w] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto consume = [&](int gr, auto slot_tag) {
            constexpr int R = decltype(slot_tag)::value;
            uint4 sw[NW], mw[NW];
#pragma unroll
            for (int w = 0; w < NW; ++w) sw[w] = sw_n[R][w], mw[w] = mw_n[R][w];
            if (gr + kRing < groups) advance_issue();
            issue_window(sw_n[R], mw_n[R]);
            const int tok = cp * TP + n16 % TP;
            const bool a_on = a_lane && tok < T;
            const int xr = MODE == SLOT_COMBINE ? ca : tok;
            const uint16_t *xg = xrow0 + (size_t)xr * ldx + (int64_t)cc * F::kSpanCodes;
            const uint16_t *abase[NSPLIT];
#pragma unroll
            for (int sp = 0; sp < NSPLIT; ++sp) abase[sp] = a_on ? xg + (size_t)sp * lds_rows * ldx : zero_block;
            const float *xsg = MODE == SLOT_COMBINE ? xsum + ((size_t)ca * nruns_pad + cc) * 16
                                                    : xsum + (size_t)cc * 16 + cp * TP + ((4 * g) & (TP - 1));
            const float cf = MODE == SLOT_COMBINE ? s_coef[ca] : 1.f;
#pragma unroll
            for (int s = 0; s < kPrefetch; ++s) {
                const int w = s % NW, so = s / NW;  // gate / up; span offset within the group
                const int gw = so;                  // its group within the window
                const uint4 w_cur = ring[R][s];
                issue_slot(ring[R], s);
                f32x4 D = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < F::kMfmas; ++t) {
                    const bf16x8 bw = codes_b<BITS>(w_cur, t);
#pragma unroll
                    for (int sp = 0; sp < NSPLIT; ++sp) {
                        const bf16x8 av = *reinterpret_cast<const bf16x8 *>(abase[sp] + so * F::kSpanCodes + t * 8);
                        D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bw, D, 0, 0, 0);
                    }
                }
                const float4 xsv = *reinterpret_cast<const float4 *>(xsg + (size_t)so * 16);
                const float xv[4] = {xsv.x, xsv.y, xsv.z, xsv.w};
                const uint32_t swd = dword(sw[w], gw >> 1), mwd = dword(mw[w], gw >> 1);
                const float s_ = __uint_as_float((gw & 1) ? (swd & 0xFFFF0000u) : (swd << 16));
                const float m_ = __uint_as_float((gw & 1) ? (mwd & 0xFFFF0000u) : (mwd << 16));
                const float cm = fmaf(-F::kOff, s_, m_);
                if constexpr (MODE == SLOT_COMBINE) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[w][v] = fmaf(cf, fmaf(s_, D[v], cm * xv[v]), acc[w][v]);
                } else {
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[w][v] = fmaf(s_, D[v], fmaf(cm, xv[v], acc[w][v]));
                }
            }
            // consume cursor; at the end of a (tile, pass) the tile is stored
            if (cc + SPG < nspan) {
                cc += SPG;
                return;
            }
            cc = 0;
            if (++ca < nseg) return;
            ca = 0;
            const int64_t n = (int64_t)(tile0 + wave + ci * kWaves) * kTile + n16;
            if (n < Nrows) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int r = cp * TP + 4 * g + v;
                    if (r >= T) continue;
                    if constexpr (MODE == COMBINE) {
                        static_cast<float *>(p.y)[s_out[b0 + r] + n] = acc[0][v];
                    } else if constexpr (is_swiglu(MODE)) {
                        TY *h = static_cast<TY *>(p.y);
                        const float gv = as_stored(acc[0][v], h), uv = as_stored(acc[NW - 1][v], h);
                        store_act(h, s_out[b0 + r] + n, as_stored(silu(gv), h) * uv);
                    } else {
                        store_act(static_cast<TY *>(p.y), s_out[b0 + r] + n, acc[0][v]);
                    }
                }
            }
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) acc[w2] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (++cp >= npass) cp = 0, ++ci;
        };
        // The ring slot of group gr is gr % kRing: the loop takes kRing groups a trip so that slots are constants.
        for (int gr = 0; gr < groups; gr += kRing) {
            consume(gr, std::integral_constant<int, 0>{});
            if constexpr (kRing > 1) if (gr + 1 < groups) consume(gr + 1, std::integral_constant<int, (kRing > 1 ? 1 : 0)>{});
            if constexpr (kRing > 2) if (gr + 2 < groups) consume(gr + 2, std::integral_constant<int, (kRing > 2 ? 2 : 0)>{});
            if constexpr (kRing > 3) if (gr + 3 < groups) consume(gr + 3, std::integral_constant<int, (kRing > 3 ? 3 : 0)>{});
        }
        return;
    }

    // General path. Tokens of the unit in batches of `cap` (more than cap only for a grouped tile holding more slots
    // than the LDS takes at once: the batch re-reads the tile's weights).
    for (int b0 = 0; b0 < T_all; b0 += cap) {
    const int T = min(cap, T_all - b0);
    const int Rb = MODE == SLOT_COMBINE ? R : T;
    if (b0 > 0) __syncthreads();  // every wave is done with the previous batch's rows

    stage(b0, Rb);
    __syncthreads();
    npass = (T + TP - 1) / TP;
    if (my_tiles > 0) {
    const int per_tile = npass * nseg * nspan * NW;
    const int total = my_tiles * per_tile;

    // ---- general path: any K, any tile length; a step at a time ----
    // Issue cursor: step counters (uniform) and the lane's row pointers (gate row; the up row is Nrows below).
    int li = 0, lp = 0, la = 0, lc = 0, lw = 0, lf = 0;
    const uint8_t *lq = nullptr;
    const uint16_t *ls = nullptr, *lm = nullptr;
    auto place = [&]() {
        const int64_t n = (int64_t)(tile0 + wave + li * kWaves) * kTile + n16;
        const int64_t nn = n < Nrows ? n : Nrows - 1;  // a partial last tile reads a valid row and stores nothing
        const int64_t row = (MODE == SLOT_COMBINE ? s_wrow[la] : s_wrow[0]) + nn;
        lq = p.q + row * rowbytes;
        ls = p.scale + row * ngroups;
        lm = p.minv + row * ngroups;
    };
    place();
    auto lnext = [&]() {
        if (lf + 1 >= total) return;  // past the end: keep re-loading the last step (its data is never used)
        ++lf;
        if (NW == 2 && ++lw < 2) return;
        lw = 0;
        if (++lc < nspan) return;
        lc = 0;
        if (++la >= nseg) {
            la = 0;
            if (++lp >= npass) lp = 0, ++li;
        }
        place();
    };
    const int last_q = (int)rowbytes - 16, last_g = (int)ngroups - 1;
    uint4 wb[kPrefetch];
    uint32_t sb[kPrefetch], mb[kPrefetch];  // raw BF16 scale / min, widened only when consumed
    // A quarter past K (the last span of a K that is not a whole number of spans) re-reads the row's last 16 bytes
    // and group: its A operand and run sum are zero, so it adds nothing.
    auto issue = [&](int slot) {
        const int qo = min(lc * kSpanBytes + g * 16, last_q);
        const int gi = min(((lc << lg_ngs) + gam) >> gshift, last_g);
        const uint8_t *qp = lq + (lw ? up_q : 0);
        const int64_t go = lw ? up_g : 0;
        wb[slot] = *reinterpret_cast<const uint4 *>(qp + qo);
        sb[slot] = ls[go + gi];
        mb[slot] = lm[go + gi];
    };
#pragma unroll
    for (int s = 0; s < kPrefetch; ++s) issue(s), lnext();

    // Consume cursor.
    int ci = 0, cp = 0, ca = 0, cc = 0;
    f32x4 acc[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) acc[w] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int f0 = 0; f0 < total; f0 += kPrefetch) {
#pragma unroll
        for (int s = 0; s < kPrefetch; ++s) {
            const int w = NW == 2 ? (s & 1) : 0;  // per_tile and kPrefetch are even with NW = 2: f and s agree
            const bool live = f0 + s < total;     // wave-uniform; no early exit, so the loop unrolls fully
            const uint4 w_cur = wb[s];
            const uint32_t s_cur = sb[s], m_cur = mb[s];
            issue(s), lnext();
            if (live) {
            // A operand rows: lane row n16 is token pass*TP + n16 % TP of group n16 / TP; zero unless that group is
            // this lane-quarter's, the token exists and the quarter lies inside K.
            const bool q_ok = cc < nspan - 1 || qlast == 0 || g < qlast;
            const int tok = cp * TP + n16 % TP;
            const bool a_on = a_lane && tok < T && q_ok;
            const int xr = MODE == SLOT_COMBINE ? ca : tok;
            const uint16_t *xa = xrow0 + (size_t)xr * ldx + (int64_t)cc * F::kSpanCodes;
            f32x4 D = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < F::kMfmas; ++t) {
                const bf16x8 bw = codes_b<BITS>(w_cur, t);
#pragma unroll
                for (int sp = 0; sp < NSPLIT; ++sp) {
                    // lanes with nothing to feed read the zero block (no exec-masked load, no register clearing)
                    const uint16_t *src = a_on ? xa + (size_t)sp * lds_rows * ldx + t * 8 : zero_block + (t & 1) * 8;
                    const bf16x8 av = *reinterpret_cast<const bf16x8 *>(src);
                    D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bw, D, 0, 0, 0);
                }
            }
            // Span epilogue: acc += s * D + (min - off * s) * run sum, for this lane's 4 D rows. The run sums past K
            // are zero in LDS.
            const int rn = (cc << lg_ngs) + gam;
            float4 xsv;
            if constexpr (MODE == SLOT_COMBINE) xsv = *reinterpret_cast<const float4 *>(xsum + ((size_t)ca * nruns_pad + rn) * 16);
            else xsv = *reinterpret_cast<const float4 *>(xsum + (size_t)rn * 16 + cp * TP + ((4 * g) & (TP - 1)));
            const float xv[4] = {xsv.x, xsv.y, xsv.z, xsv.w};
            const float s_ = __uint_as_float(s_cur << 16), m_ = __uint_as_float(m_cur << 16);
            const float cm = fmaf(-F::kOff, s_, m_);
            if constexpr (MODE == SLOT_COMBINE) {
                const float cf = s_coef[ca];
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[w][v] = fmaf(cf, fmaf(s_, D[v], cm * xv[v]), acc[w][v]);
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[w][v] = fmaf(s_, D[v], fmaf(cm, xv[v], acc[w][v]));
            }

            // Advance; at the end of a (tile, pass): add the groups' lanes, store, reset.
            bool tile_end = false;
            if (w == NW - 1 && ++cc == nspan) {
                cc = 0;
                if (++ca == nseg) ca = 0, tile_end = true;
            }
            if (tile_end) {
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if (ngs >= 4) acc[w2][v] += __shfl_xor(acc[w2][v], 16);
                    if (ngs >= 2) acc[w2][v] += __shfl_xor(acc[w2][v], 32);
                }
            const int64_t n = (int64_t)(tile0 + wave + ci * kWaves) * kTile + n16;
            if ((g << lg_ngs) < 4 && n < Nrows) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int r = cp * TP + 4 * g + v;
                    if (r >= T) continue;
                    if constexpr (MODE == COMBINE) {
                        static_cast<float *>(p.y)[s_out[b0 + r] + n] = acc[0][v];
                    } else if constexpr (is_swiglu(MODE)) {
                        TY *h = static_cast<TY *>(p.y);
                        const float gv = as_stored(acc[0][v], h), uv = as_stored(acc[NW - 1][v], h);
                        store_act(h, s_out[b0 + r] + n, as_stored(silu(gv), h) * uv);
                    } else {
                        store_act(static_cast<TY *>(p.y), s_out[b0 + r] + n, acc[0][v]);
                    }
                }
            }
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) acc[w2] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (++cp >= npass) cp = 0, ++ci;
            }  // tile_end
            }  // live
        }
    }
    }  // my_tiles
    }  // token batches
}

template <int BITS, int MODE, typename TX, typename TY>
hipError_t go(const Params &p, dim3 grid, hipStream_t stream) {
    constexpr int NSPLIT = sizeof(TX) == 4 ? 3 : 1;
    const int rows = MODE == SLOT_COMBINE ? (int)p.A : p.max_rows;
    const size_t lds = lds_bytes(BITS, NSPLIT, p.K, p.G, rows, MODE == SLOT_COMBINE ? (int)p.A : 1);
    auto k = qmm_kernel<BITS, NSPLIT, MODE, TX, TY>;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k, grid, dim3(kThreads), lds, stream, p);
    return hipGetLastError();
}

template <int MODE>
hipError_t launch_mode(int bits, int ax, int ay, const Params &p, dim3 grid, hipStream_t s) {
    auto by_act = [&](auto bits_c) {
        constexpr int B = decltype(bits_c)::value;
        if (ax == SX_ACT_F32) return go<B, MODE, float, float>(p, grid, s);
        if (ay == SX_ACT_F32) return go<B, MODE, uint16_t, float>(p, grid, s);
        return go<B, MODE, uint16_t, uint16_t>(p, grid, s);
    };
    return bits == 4 ? by_act(std::integral_constant<int, 4>{}) : by_act(std::integral_constant<int, 8>{});
}

}  // namespace detail
}  // namespace sx::qmm
