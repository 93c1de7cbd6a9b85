// Skinny dequantizing GEMM on the matrix cores: the kernel template (see qmm.hpp for the scheme). Each qmm_mN.hip
// instantiates one mode, so the instantiations compile in parallel.
#pragma once
#include "qmm.hpp"

#include <type_traits>

namespace sx::qmm {
namespace detail {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kPrefetch = 8;  // spans whose loads are in flight per wave

template <int BITS>
struct Fmt {
    static constexpr int kSpanCodes = BITS == 4 ? 128 : 64;
    static constexpr int kMfmas = BITS == 4 ? 4 : 2;  // MFMAs a span (8 codes a lane each)
    static constexpr float kOff = BITS == 4 ? 128.f : 0.f;
};

__device__ __forceinline__ uint32_t dword(const uint4 &w, int i) { return i == 0 ? w.x : i == 1 ? w.y : i == 2 ? w.z : w.w; }

// B operand of MFMA t from a lane's 16 code bytes. q4: dword t's nibbles j = 0..7 (code k0 + j) as BF16 128 + code in
// element order [0, 4, 1, 5, 2, 6, 3, 7] - one v_and_or (plus a shift) a pair. q8: dwords 2t, 2t+1 in byte order.
template <int BITS>
__device__ __forceinline__ bf16x8 codes_b(const uint4 &w, int t) {
    uint4 v;
    if constexpr (BITS == 4) {
        const uint32_t d = dword(w, t);
        v.x = (d & 0x000F000Fu) | 0x43004300u;
        v.y = ((d >> 4) & 0x000F000Fu) | 0x43004300u;
        v.z = ((d >> 8) & 0x000F000Fu) | 0x43004300u;
        v.w = ((d >> 12) & 0x000F000Fu) | 0x43004300u;
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

template <typename TX>
__device__ __forceinline__ void load8(const TX *p, float (&v)[8]) {
    if constexpr (sizeof(TX) == 4) {
        const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else {
        const uint4 u = reinterpret_cast<const uint4 *>(p)[0];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w = dword(u, i);
            v[2 * i] = __uint_as_float(w << 16), v[2 * i + 1] = __uint_as_float(w & 0xFFFF0000u);
        }
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
    const int nspan = (int)(K / F::kSpanCodes);
    const int run = G < F::kSpanCodes ? G : F::kSpanCodes;     // codes a partial sum covers
    const int nruns = (int)(K / run);
    const int ngs = F::kSpanCodes / run;                         // groups a span
    const int TP = 16 / ngs;                                     // activation rows a pass
    const int64_t ldx = K + 8;                                   // LDS row stride (BF16 elements)
    const int64_t rowbytes = BITS == 4 ? K / 2 : K;
    const int64_t ngroups = K / G;
    const int64_t Nrows = is_swiglu(MODE) ? p.N / 2 : p.N;      // output rows per expert
    const int unit = (int)(blockIdx.x / (unsigned)p.nchunks), chunk = (int)(blockIdx.x % (unsigned)p.nchunks);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // ---- the unit: its activation rows, output rows and expert ----
    if (tid == 0) {
        int T = 0, R = 0, bad = 0;
        if constexpr (MODE == DENSE) {
            const int64_t m0 = (int64_t)blockIdx.y * p.max_rows;
            T = (int)min((int64_t)p.max_rows, p.M - m0);
            for (int r = 0; r < T; ++r) s_xrow[r] = (m0 + r) * K, s_out[r] = (m0 + r) * p.N;
            s_wrow[0] = 0;
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
                for (int r = 0; r < T; ++r) {
                    const int64_t slot = slots[st + r];
                    s_xrow[r] = (MODE == COMBINE ? slot : slot / p.A) * K;
                    s_out[r] = slot * Nrows;
                }
                bad = bucket == E;
                s_wrow[0] = (int64_t)bucket * p.N;
                R = T;
            }
        } else if constexpr (MODE != SLOT_COMBINE) {
            const int64_t slot = unit;
            const int32_t id = p.ids[slot];
            T = 1, R = 1;
            bad = !(id >= 0 && id < p.E);
            if (bad && chunk == 0) flag_error(p.err, (uint32_t)id, (uint32_t)slot);
            s_xrow[0] = (slot / p.A) * K, s_out[0] = slot * Nrows, s_wrow[0] = (int64_t)id * p.N;
        } else {
            const int64_t m = unit;
            T = 1, R = (int)p.A;
            for (int a = 0; a < R; ++a) {
                const int32_t id = p.ids[m * p.A + a];
                const bool ok = id >= 0 && id < p.E;
                if (!ok && !bad && chunk == 0) flag_error(p.err, (uint32_t)id, (uint32_t)(m * p.A + a));
                bad |= !ok;
                s_xrow[a] = (m * p.A + a) * K, s_wrow[a] = (int64_t)id * p.N, s_coef[a] = p.coef[m * p.A + a];
            }
            s_out[0] = m * p.N;
        }
        s_T = T, s_R = R, s_bad = bad;
    }
    __syncthreads();
    const int T_all = s_T, R = s_R;
    if (T_all == 0) return;  // an over-provisioned grouped unit: uniform for the block
    const int tiles_total = (int)((Nrows + kTile - 1) / kTile);
    const int tile0 = chunk * p.tiles_per_chunk;
    const int tiles_here = min(p.tiles_per_chunk, tiles_total - tile0);
    if (tiles_here <= 0) return;

    if (s_bad) {  // invalid expert id: NaN outputs, never an out-of-bounds weight read
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
    uint16_t *xs = reinterpret_cast<uint16_t *>(smem);
    float *xsum = reinterpret_cast<float *>(smem + (size_t)NSPLIT * lds_rows * ldx * 2);
    const TX *x = static_cast<const TX *>(p.x);
    const int chunks8 = (int)(K / 8), lanes_per_run = run / 8;

    // Tokens of the unit in batches of `cap` (more than cap only for a grouped tile holding more slots than the LDS
    // takes at once: the batch re-reads the tile's weights).
    for (int b0 = 0; b0 < T_all; b0 += cap) {
    const int T = min(cap, T_all - b0);
    const int Rb = MODE == SLOT_COMBINE ? R : T;
    if (b0 > 0) __syncthreads();  // every wave is done with the previous batch's rows

    // ---- stage the activation rows in LDS: NSPLIT BF16 planes in the B operand's code order, and run sums ----
    for (int i = tid; i < Rb * chunks8; i += kThreads) {  // kThreads and chunks8 are multiples of lanes_per_run
        const int r = i / chunks8, c8 = i % chunks8;
        float v[8];
        load8(x + s_xrow[MODE == SLOT_COMBINE ? r : b0 + r] + (int64_t)c8 * 8, v);
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
        for (int off = 1; off < lanes_per_run; off <<= 1) sum += __shfl_xor(sum, off);
        if (c8 % lanes_per_run == 0) {
            const int rn = c8 / lanes_per_run;
            if constexpr (MODE == SLOT_COMBINE) xsum[((size_t)r * nruns + rn) * 16] = sum;
            else xsum[(size_t)rn * 16 + r] = sum;
        }
    }
    __syncthreads();

    // ---- each wave: its tiles of the chunk, every activation pass, all spans (and SLOT_COMBINE's slots) ----
    const int n16 = lane & 15, g = lane >> 4;
    const int lg_ngs = ngs == 1 ? 0 : ngs == 2 ? 1 : 2;
    const int gam = (g << lg_ngs) >> 2;             // this lane-quarter's group within a span
    const int gshift = G > F::kSpanCodes ? 1 : 0;   // q8 G = 128: two spans a group
    const int nseg = MODE == SLOT_COMBINE ? R : 1;  // weight segments a tile (SLOT_COMBINE: one per slot)
    const int npass = (T + TP - 1) / TP;
    const int my_tiles = (tiles_here - wave + kWaves - 1) / kWaves;
    if (my_tiles > 0) {

    // A cursor over the wave's steps (tile i, pass, segment a, span c), span fastest; its row pointers follow it.
    struct Cursor {
        int i, pass, a, c;
        const uint8_t *qrow;
        const uint16_t *srow, *mrow;
        int64_t n;
    };
    auto place = [&](Cursor &u) {  // row pointers for (i, a)
        const int64_t tile = tile0 + wave + (int64_t)u.i * kWaves;
        u.n = tile * kTile + n16;
        const int64_t nn = u.n < Nrows ? u.n : Nrows - 1;  // partial last tile: a valid row, its result not stored
        const int64_t row = (MODE == SLOT_COMBINE ? s_wrow[u.a] : s_wrow[0]) + nn;
        u.qrow = p.q + row * rowbytes + g * 16;
        u.srow = p.scale + row * ngroups;
        u.mrow = p.minv + row * ngroups;
    };
    auto advance = [&](Cursor &u) {  // wave-uniform branches
        if (++u.c < nspan) return;
        u.c = 0;
        if (++u.a < nseg) return place(u);
        u.a = 0;
        if (++u.pass < npass) return place(u);
        u.pass = 0;
        ++u.i;
        place(u);
    };
    const int total = my_tiles * npass * nseg * nspan;
    uint4 wb[kPrefetch][NW];
    uint32_t sm[kPrefetch][NW];
    auto issue = [&](const Cursor &u, int slot) {
        const int gi = ((u.c << lg_ngs) + gam) >> gshift;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const int64_t up = w ? Nrows : 0;  // SwiGLU: the up row I rows below the gate row
            wb[slot][w] = *reinterpret_cast<const uint4 *>(u.qrow + up * rowbytes + (int64_t)u.c * kSpanBytes);
            sm[slot][w] = (uint32_t)u.srow[up * ngroups + gi] | ((uint32_t)u.mrow[up * ngroups + gi] << 16);
        }
    };

    Cursor ld{0, 0, 0, 0, nullptr, nullptr, nullptr, 0}, cu;
    place(ld);
    cu = ld;
#pragma unroll
    for (int s = 0; s < kPrefetch; ++s)
        if (s < total) issue(ld, s), advance(ld);

    f32x4 acc[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) acc[w] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int f0 = 0; f0 < total; f0 += kPrefetch) {
#pragma unroll
        for (int s = 0; s < kPrefetch; ++s) {
            if (f0 + s >= total) break;
            uint4 w_cur[NW];
            uint32_t sm_cur[NW];
#pragma unroll
            for (int w = 0; w < NW; ++w) w_cur[w] = wb[s][w], sm_cur[w] = sm[s][w];
            if (f0 + s + kPrefetch < total) issue(ld, s), advance(ld);

            // A operand rows: lane row n16 is token pass*TP + n16 % TP of group n16 / TP; zero unless that group is
            // this lane-quarter's and the token exists.
            const int tok = cu.pass * TP + n16 % TP;
            const bool a_on = (n16 / TP) == gam && tok < T;
            const int xr = MODE == SLOT_COMBINE ? cu.a : tok;
            const uint16_t *xa = xs + (size_t)xr * ldx + (int64_t)cu.c * F::kSpanCodes + g * (F::kSpanCodes / 4);
            f32x4 D[NW];
#pragma unroll
            for (int w = 0; w < NW; ++w) D[w] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < F::kMfmas; ++t) {
                bf16x8 bw[NW];
#pragma unroll
                for (int w = 0; w < NW; ++w) bw[w] = codes_b<BITS>(w_cur[w], t);
#pragma unroll
                for (int sp = 0; sp < NSPLIT; ++sp) {
                    bf16x8 av = {};
                    if (a_on) av = *reinterpret_cast<const bf16x8 *>(xa + (size_t)sp * lds_rows * ldx + t * 8);
#pragma unroll
                    for (int w = 0; w < NW; ++w) D[w] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bw[w], D[w], 0, 0, 0);
                }
            }
            // Span epilogue: acc += s * D + (min - off * s) * run sum, for this lane's 4 D rows.
            const int rn = (cu.c << lg_ngs) + gam;
            float4 xsv;
            if constexpr (MODE == SLOT_COMBINE) xsv = *reinterpret_cast<const float4 *>(xsum + ((size_t)cu.a * nruns + rn) * 16);
            else xsv = *reinterpret_cast<const float4 *>(xsum + (size_t)rn * 16 + cu.pass * TP + ((4 * g) & (TP - 1)));
            const float xv[4] = {xsv.x, xsv.y, xsv.z, xsv.w};
            const float cf = MODE == SLOT_COMBINE ? s_coef[cu.a] : 1.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const float s_ = bf16_to_f32(sm_cur[w] & 0xFFFFu), m_ = bf16_to_f32(sm_cur[w] >> 16);
                const float cm = m_ - F::kOff * s_;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float part = fmaf(s_, D[w][v], cm * xv[v]);
                    acc[w][v] = MODE == SLOT_COMBINE ? fmaf(cf, part, acc[w][v]) : acc[w][v] + part;
                }
            }

            // End of a (tile, pass): add the groups' lanes, store, reset.
            if (cu.a == nseg - 1 && cu.c == nspan - 1) {
#pragma unroll
                for (int w = 0; w < NW; ++w)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        if (ngs >= 4) acc[w][v] += __shfl_xor(acc[w][v], 16);
                        if (ngs >= 2) acc[w][v] += __shfl_xor(acc[w][v], 32);
                    }
                if ((g << lg_ngs) < 4 && cu.n < Nrows) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int r = cu.pass * TP + 4 * g + v;
                        if (r >= T) continue;
                        if constexpr (MODE == COMBINE) {
                            static_cast<float *>(p.y)[s_out[b0 + r] + cu.n] = acc[0][v];
                        } else if constexpr (is_swiglu(MODE)) {
                            TY *h = static_cast<TY *>(p.y);
                            const float gv = as_stored(acc[0][v], h), uv = as_stored(acc[1][v], h);
                            store_act(h, s_out[b0 + r] + cu.n, as_stored(silu(gv), h) * uv);
                        } else {
                            store_act(static_cast<TY *>(p.y), s_out[b0 + r] + cu.n, acc[0][v]);
                        }
                    }
                }
#pragma unroll
                for (int w = 0; w < NW; ++w) acc[w] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
            advance(cu);
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
