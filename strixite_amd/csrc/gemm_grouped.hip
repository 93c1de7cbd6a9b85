// Prefill-width grouped expert GEMM on the matrix cores: q4 experts (G = 128), BF16 activations, any bucket size.
//
// The verify kernel (qmm) stages every activation row of a unit over the whole K in LDS and passes the weights once
// per 16 rows; with hundreds of rows a bucket (kernels/moe_grouped.hpp:5-17: the prefill path) that re-streams each
// expert's weights per 16 rows. Here a block (4 waves, two blocks a CU) owns a 64-slot tile of one bucket (the
// workspace's wide tiles, moe_grouped.hip:63-81) times 256 weight rows; a wave owns all 64 slots times 64 rows (two
// 32-row tiles; SwiGLU: the gate and the up rows of 32 features) as 2 x 2 v_mfma_f32_32x32x16_bf16 tiles, so each
// activation fragment read from LDS feeds two MFMAs and each weight fragment two. K advances one span (128 codes =
// one quantization group) a step:
//   - the block's 64 activation rows of the span arrive by direct global->LDS loads (DMA) into a 4-stage ring, two
//     steps at a time two steps ahead (one block barrier every two steps), each row's sixteen 16-byte chunks
//     XOR-swizzled so that the MFMA operand reads are free of bank conflicts; the block sums each row's span;
//   - each lane loads its weight rows' codes (32 bytes a row a span) and scales straight into registers, two steps
//     ahead, and turns a dword of codes into the BF16 operand (128 + code) with four byte selects and AND-ORs;
//   - per span: acc[slot][row] += s[row] * D + (m[row] - 128 s[row]) * sum_span x[slot], with D = the span's
//     sum x * (128 + code) from the MFMAs, exact in FP32 (the identity qmm uses).
// MFMA k order: lane half h, MFMA kk, element e of a span <-> code h * 64 + kk * 8 + e (any order A and B share).
// Epilogues: SwiGLU (gate and up of the same features in one wave), plain gather, FP32 partials (combine).
#include "gemm_grouped.hpp"
#include "qmm_impl.hpp"

namespace sx::gg {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256, kWaves = 4;
constexpr int kBM = 64;                      // slots a block tile
constexpr int kSpan = 128, kSpanBytes = 64;  // q4 codes / bytes a span (= one G = 128 group) = one K step
constexpr int kStages = 4;                   // activation stages in LDS: three in flight while one is read
constexpr int kStageBytes = kBM * kSpan * 2;  // 16 KB
constexpr int kDmaPerWave = kStageBytes / 1024 / kWaves;  // 16-byte-a-lane DMA instructions a wave a step (4)
constexpr int kMaxGroups = 32;  // K <= 4096: the span sums of every step stay in LDS
constexpr int kSumStride = kMaxGroups + 4;  // floats a row (16-byte aligned, rows 4 banks apart)

// gg_kernel's K-step layout for q4 (G = 128) and q8 (G = 64) weights: one quantization group a K step (64 bytes of a
// weight row either way), the step's activation rows in 16-byte chunks, chunk c of row r in slot c ^ swz(r). The
// swizzle makes the 16 rows a quarter-wave's MFMA operand reads touch distinct banks (q4: 256-byte rows, 16 chunks;
// q8: 128-byte rows, two to the 256 bytes of the banks, so rows r and r + 1 share a swizzle and differ in half).
template <int BITS>
struct Lay {
    static constexpr int kSpan = BITS == 4 ? 128 : 64;  // codes a K step
    static constexpr int kChunks = kSpan / 8;             // 16-byte activation chunks a row a step
    static constexpr int kRowBytes = kSpan * 2;
    static constexpr int kStageBytes = kBM * kRowBytes;   // 16 KB / 8 KB
    static constexpr int kDmaPerWave = kStageBytes / 1024 / kWaves;  // 4 / 2
    static constexpr int kMaxGroups = 4096 / kSpan;        // K <= 4096
    static constexpr int kSumStride = kMaxGroups + 4;
    static constexpr int kKk = kSpan / 16;                 // MFMAs (k = 16) a step: 8 / 4
    static constexpr float kOff = BITS == 4 ? 128.f : 0.f;  // the operand is code + kOff
    static constexpr int kStageAlign = BITS == 4 ? 16 : 128;
    __device__ static int swz(int r) { return BITS == 4 ? (r & 15) : ((r >> 1) & 7); }
};

struct Params {
    const uint16_t *x;  // BF16 activations [tokens or slots, K]
    const uint8_t *q;
    const uint16_t *scale, *minv;
    void *y;
    const int32_t *ws;
    int64_t A, N, K;  // slots a token; rows an expert (SWIGLU: 2I); K
    int64_t E;
    int nrb;  // row blocks
    int64_t dense_M;  // > 0: a dense linear (GATHER) over dense_M token rows, tile u = tokens 64 u .. (no workspace)
    int vec_store;    // BF16 output, output rows a multiple of 8 and y 16-byte aligned: stores staged through LDS
};

// The 1-D grid in groups of 8 tiles x nrb row blocks, row-block-major inside a group: the row blocks of a tile get
// block ids of one residue mod 8 - the same XCD under the round-robin dispatch - close together, so the tile's
// activation rows come from HBM once and from that XCD's L2 for the other row blocks.
__device__ __forceinline__ int tile_of(unsigned id, int nrb) {
    const unsigned grp = id / (8u * nrb), r = id % (8u * nrb);
    return (int)(grp * 8 + r % 8);
}
__device__ __forceinline__ int rowblock_of(unsigned id, int nrb) { return (int)((id % (8u * nrb)) / 8); }

// (a & b) | c in one ALU operation, v_bitop3_b32 with truth table 0xEA (bit 4 S0 + 2 S1 + S2 of the table is the
// result for those input bits). Written as (a & b) | c the compiler splits it into an AND and an OR; as an intrinsic
// (not inline asm) its operands are ordinary uses, which the wait-count pass covers: an asm's are not, and an asm
// form of this on registers straight from the code loads gave run-to-run differences.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, b, c, 0xEA);
}

// Operand of 8 codes (one dword: the low nibble of byte b is code 2b) in natural order as BF16 128 + code: a byte
// select puts byte b of d (its low nibble wanted) and byte b of d >> 4 (the high nibble) in the two halves, one
// AND-OR masks the nibbles and sets the exponent: 9 ALU operations for 8 codes.
__device__ __forceinline__ bf16x8 codes_nat(uint32_t d) {
    const uint32_t hi = d >> 4, m = 0x000F000Fu, e = 0x43004300u;
    uint4 v;
    v.x = and_or(__builtin_amdgcn_perm(hi, d, 0x0C040C00u), m, e);
    v.y = and_or(__builtin_amdgcn_perm(hi, d, 0x0C050C01u), m, e);
    v.z = and_or(__builtin_amdgcn_perm(hi, d, 0x0C060C02u), m, e);
    v.w = and_or(__builtin_amdgcn_perm(hi, d, 0x0C070C03u), m, e);
    return __builtin_bit_cast(bf16x8, v);
}

// Operand of 8 q8 codes (two dwords, code order = byte order) as BF16: each byte to FP32 (exact) and the upper
// halves of two FP32 values into one dword.
__device__ __forceinline__ bf16x8 codes8(uint32_t d0, uint32_t d1) {
    auto pair = [](uint32_t d, int b) {
        const uint32_t lo = __float_as_uint((float)((d >> (8 * b)) & 0xFFu));
        const uint32_t hi = __float_as_uint((float)((d >> (8 * b + 8)) & 0xFFu));
        return __builtin_amdgcn_perm(hi, lo, 0x07060302u);
    };
    const uint4 v{pair(d0, 0), pair(d0, 2), pair(d1, 0), pair(d1, 2)};
    return __builtin_bit_cast(bf16x8, v);
}

// sum + the 8 BF16 values of a 16-byte chunk, in order, as four dot products with (1, 1): a v_dot2 adds a pair's two
// exact products to the running FP32 sum (4 ALU operations for the 16 of unpacking to FP32 and adding)
__device__ __forceinline__ float sum_chunk(const uint4 &c, float sum) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 one = __builtin_bit_cast(bf16x2, 0x3F803F80u);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, qmm::detail::dword(c, i)), one, sum, false);
    return sum;
}

__device__ __forceinline__ void dma16(const void *src, void *lds) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
}

template <int MODE, typename TY, int BITS>
__global__ void __launch_bounds__(kThreads, 2) gg_kernel(Params p) {
    using L = Lay<BITS>;
    constexpr int kSpan = L::kSpan, kStageBytes = L::kStageBytes, kDmaPerWave = L::kDmaPerWave,
                  kSumStride = L::kSumStride;
    // One array a stage, so that the wait-count pass tells a stage's DMA apart from the others'.
    __shared__ __attribute__((aligned(L::kStageAlign))) unsigned char x0[kStageBytes], x1[kStageBytes],
        x2[kStageBytes], x3[kStageBytes];
    __shared__ __attribute__((aligned(16))) float xsum[kBM * kSumStride];  // [slot][span]
    __shared__ int64_t s_xrow[kBM], s_out[kBM];
    __shared__ int s_T, s_bucket;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31, h = lane >> 5;  // MFMA row / column of the lane, its k half
    const int64_t K = p.K;
    const int E = (int)p.E;

    // ---- the 64-slot tile: bucket, slots (wave 0, lane r fills row r) ----
    if (tid < 64 && p.dense_M > 0) {  // a dense linear: one "bucket" (the weight), the tokens in order
        const int u = tile_of(blockIdx.x, p.nrb);
        const int64_t t0 = (int64_t)u * kBM;
        const int T = t0 < p.dense_M ? (int)min((int64_t)kBM, p.dense_M - t0) : 0;
        if (lane < T) s_xrow[lane] = (t0 + lane) * K, s_out[lane] = t0 + lane;
        if (lane == 0) s_T = T, s_bucket = 0;
    } else if (tid < 64) {
        const int32_t *ws = p.ws;
        const int32_t n_wt = ws[3], S = ws[1];
        int T = 0, bucket = -1;
        const int u = tile_of(blockIdx.x, p.nrb);
        if (u < n_wt) {
            const int32_t *offsets = ws + 4, *slots = offsets + E + 2;
            const int64_t Tmax = (int64_t)S / 16 + E + 2, WTmax = (int64_t)S / 64 + E + 2;
            const int32_t *wtile_bucket = slots + S + 2 * Tmax, *wtile_start = wtile_bucket + WTmax;
            bucket = wtile_bucket[u];
            const int32_t st = wtile_start[u];
            T = min(kBM, offsets[bucket + 1] - st);
            if (lane < T) {
                const int64_t slot = slots[st + lane];
                s_xrow[lane] = (MODE == qmm::COMBINE ? slot : slot / p.A) * K;
                s_out[lane] = slot;
            }
        }
        if (lane == 0) s_T = T, s_bucket = bucket;
    }
    __syncthreads();
    const int T = __builtin_amdgcn_readfirstlane(s_T), bucket = __builtin_amdgcn_readfirstlane(s_bucket);
    if (T == 0) return;  // past the tile count: uniform for the block
    const int64_t Nrows = MODE == qmm::SWIGLU ? p.N / 2 : p.N;  // output rows (features) an expert
    constexpr int kOutRows = MODE == qmm::SWIGLU ? kWaves * 32 : kWaves * 64;  // output rows a block
    const int64_t r0 = (int64_t)rowblock_of(blockIdx.x, p.nrb) * kOutRows;
    if (bucket == E) {  // invalid ids (reported by the grouping): NaN rows, never an out-of-range weight read
        for (int i = tid; i < T * kOutRows; i += kThreads) {
            const int r = i / kOutRows;
            const int64_t n = r0 + i % kOutRows;
            if (n >= Nrows) continue;
            if constexpr (MODE == qmm::COMBINE) static_cast<float *>(p.y)[s_out[r] * Nrows + n] = qnan();
            else store_act(static_cast<TY *>(p.y), s_out[r] * Nrows + n, qnan());
        }
        return;
    }
    if (tid >= T && tid < kBM) s_xrow[tid] = s_xrow[T - 1];  // rows past T: row T - 1 again, never stored
    __syncthreads();

    // ---- this lane's two weight rows (nb = 0, 1), clamped into the expert (stores are masked) ----
    const int64_t rowbytes = BITS == 4 ? K / 2 : K, ngroups = K / kSpan;
    const uint8_t *qrow[2];
    const uint16_t *srow[2], *mrow[2];
    int64_t feat[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        int64_t n;  // row within the expert
        if constexpr (MODE == qmm::SWIGLU) n = (nb == 0 ? 0 : Nrows) + r0 + wave * 32 + j;  // gate, up
        else n = r0 + wave * 64 + nb * 32 + j;
        feat[nb] = MODE == qmm::SWIGLU ? r0 + wave * 32 + j : n;
        const int64_t nn = min(n, (MODE == qmm::SWIGLU ? 2 * Nrows : Nrows) - 1);
        const int64_t row = (int64_t)bucket * p.N + nn;
        qrow[nb] = p.q + row * rowbytes + h * 32;
        srow[nb] = p.scale + row * ngroups;
        mrow[nb] = p.minv + row * ngroups;
    }
    // Activation DMA: instruction I covers kDmaRows tile rows from kDmaRows I; lane l writes row kDmaRows I +
    // l / kChunks, chunk (l % kChunks) ^ swz(row), so slot s of a row holds chunk s ^ swz(row) (q4: 16 instructions
    // of 4 rows; q8: 8 of 8). This wave issues I = kDmaPerWave wave + i.
    constexpr int kChunks = L::kChunks, kDmaRows = 64 / kChunks;
    const uint16_t *xl[kDmaPerWave];
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
        const int r = kDmaRows * (kDmaPerWave * wave + i) + lane / kChunks;
        xl[i] = p.x + s_xrow[r] + (((lane % kChunks) ^ L::swz(r)) * 8);
    }
    auto xs_at = [&](int st) -> unsigned char * { return st == 0 ? x0 : st == 1 ? x1 : st == 2 ? x2 : x3; };
    const int nk = (int)(K / kSpan);
    const bool two_tb = T > 32;  // the second 32-slot half holds slots (uniform)

    // K step k (clamped: past the end it re-loads the last step, never used) into stage st
    // (a tile of at most 32 slots leaves rows 32..63 alone: waves 2 and 3, which cover them, load nothing)
    const bool dma_on = two_tb || wave < 2;  // wave-uniform
    auto issue_x = [&](int kstep, int st) __attribute__((always_inline)) {
        const int k = min(kstep, nk - 1);
        if (!dma_on) return;
#pragma unroll
        for (int i = 0; i < kDmaPerWave; ++i)
            dma16(xl[i] + (int64_t)k * kSpan, xs_at(st) + (kDmaPerWave * wave + i) * 1024);
    };
    // the lane's codes (2 rows x 2 x 16 bytes) and scales / mins of step k, into a ring slot
    uint4 cw[2][2][2];     // [ring slot][nb][half of the lane's 32 bytes]
    // the scales of 4 steps a row as one 8-byte window (fewer cache lines a step than one 2-byte load a step); the
    // mins are used once, at the end
    uint2 wcur[2], wnxt[2];
    auto issue_codes = [&](int kstep, uint4 (&w)[2][2], int half) {
        const int k = min(kstep, nk - 1);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
            w[nb][half] = *reinterpret_cast<const uint4 *>(qrow[nb] + (int64_t)k * kSpanBytes + half * 16);
    };
    auto issue_window = [&](int kstep, uint2 (&w)[2]) {  // steps kstep .. kstep + 3 (clamped: nk % 4 == 0)
        const int k = min(kstep, nk - 4);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) w[nb] = *reinterpret_cast<const uint2 *>(srow[nb] + k);
    };
    // the span sums of stage st's 64 rows (K step grp): 4 threads a row, 4 chunks each. The reads are inline asm
    // ending in lgkmcnt(0): the compiler does not track an asm output as a pending LDS load, so the asm waits for
    // its own reads (lgkmcnt counts LDS operations; nothing else is outstanding on it here)
    auto sum_rows = [&](int st, int grp) __attribute__((always_inline)) {
        const int r = tid >> 2, qd = tid & 3;
        if (!dma_on) return;  // rows 32..63 of a tile of at most 32 slots
        if constexpr (BITS == 8) {
            // chunks 2 qd, 2 qd + 1 in chunk order: slots (2 qd) ^ swz(r) and that ^ 1 (the row is 128-byte aligned)
            const uint32_t at = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const unsigned char *)(
                xs_at(st) + r * 128 + (((2 * qd) ^ L::swz(r)) * 16));
            uint4 raw[2];
            uint32_t tmp;
            asm volatile("ds_read_b128 %0, %3\n\t"
                         "v_xor_b32 %2, 16, %3\n\tds_read_b128 %1, %2\n\ts_waitcnt lgkmcnt(0)"
                         : "=&v"(raw[0]), "=&v"(raw[1]), "=&v"(tmp)
                         : "v"(at));
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < 2; ++i) sum = sum_chunk(raw[i], sum);
            sum = qmm::detail::group_sum_c<4>(sum);
            if (qd == 0 && grp < nk) xsum[r * kSumStride + grp] = sum;
            return;
        }
        // chunks 4 qd .. 4 qd + 3 of the row in chunk order (chunk c sits in slot c ^ (r & 15)), so that a slot's
        // sum does not depend on its position in the tile
        const uint32_t grp0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const unsigned char *)(
            xs_at(st) + r * 256 + ((qd ^ ((r & 15) >> 2)) * 64));
        const uint32_t at = grp0 + ((uint32_t)(r & 3) << 4);  // chunk 4 qd + i at at ^ 16 i (grp0 is 64-byte aligned)
        // read in asm: the wait-count pass would otherwise hold these reads for every DMA in flight (it cannot
        // tell this stage from the one just issued); the step's barrier already covers this stage's DMA. One
        // scratch register forms the other three addresses (a read has taken its address once it has issued).
        uint4 raw[4];
        uint32_t tmp;
        asm volatile("ds_read_b128 %0, %5\n\t"
                     "v_xor_b32 %4, 16, %5\n\tds_read_b128 %1, %4\n\t"
                     "v_xor_b32 %4, 32, %5\n\tds_read_b128 %2, %4\n\t"
                     "v_xor_b32 %4, 48, %5\n\tds_read_b128 %3, %4\n\ts_waitcnt lgkmcnt(0)"
                     : "=&v"(raw[0]), "=&v"(raw[1]), "=&v"(raw[2]), "=&v"(raw[3]), "=&v"(tmp)
                     : "v"(at));
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) sum = sum_chunk(raw[i], sum);
        sum = qmm::detail::group_sum_c<4>(sum);
        if (qd == 0 && grp < nk) xsum[r * kSumStride + grp] = sum;
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[tb][nb] = f32x16{};

    // one K step on stage st with ring slot RS; the ring slot is re-loaded (step k + 2) as its codes are used
    auto compute = [&](int k, int st, auto rs_tag, auto two_tag) __attribute__((always_inline)) {
        constexpr int RS = decltype(rs_tag)::value;
        constexpr bool TWO = decltype(two_tag)::value;  // the second 32-slot half holds slots
        const unsigned char *xb = xs_at(st);
        f32x16 D[2][2];
        // activation fragments one MFMA step ahead (their LDS latency hides behind the step before)
        bf16x8 aop[2][2];  // [buffer][tb]
        auto load_a = [&](int kk, bf16x8 (&a)[2]) __attribute__((always_inline)) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                if (tb == 1 && !TWO) continue;
                const int row = tb * 32 + j;
                a[tb] = *reinterpret_cast<const bf16x8 *>(xb + row * L::kRowBytes +
                                                          (((h * (kChunks / 2) + kk) ^ L::swz(row)) * 16));
            }
        };
        load_a(0, aop[0]);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
            for (int kq = 0; kq < L::kKk / 2; ++kq) {
                const int kk = half * (L::kKk / 2) + kq;
                if (kk < L::kKk - 1) load_a(kk + 1, aop[(kk + 1) & 1]);
                bf16x8 bop[2];
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    const uint4 &c = cw[RS][nb][half];
                    if constexpr (BITS == 4) bop[nb] = codes_nat(qmm::detail::dword(c, kq));
                    else bop[nb] = codes8(qmm::detail::dword(c, 2 * kq), qmm::detail::dword(c, 2 * kq + 1));
                }
#pragma unroll
                for (int tb = 0; tb < 2; ++tb) {
                    if (tb == 1 && !TWO) continue;
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb)
                        D[tb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aop[kk & 1][tb], bop[nb],
                                                                            kk == 0 ? f32x16{} : D[tb][nb], 0, 0, 0);
                }
            }
            issue_codes(k + 2, cw[RS], half);  // this half's codes are in the operands
        }
        // fold the span: s * D (the (m - 128 s) * sum x term of every span is added once, at the end); a lane's
        // value v is slot 8 (v / 4) + 4 h + v % 4 of its tile
        float s_[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const uint32_t wd = (st & 2) ? wcur[nb].y : wcur[nb].x;
            s_[nb] = __uint_as_float((st & 1) ? (wd & 0xFFFF0000u) : (wd << 16));
        }
        if (st == 3) {  // the next window becomes current (loaded four steps ago); the one after is issued
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) wcur[nb] = wnxt[nb];
            issue_window(k + 5, wnxt);
        }
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            if (tb == 1 && !TWO) continue;
#pragma unroll
            for (int v = 0; v < 16; ++v)
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) acc[tb][nb][v] = fmaf(s_[nb], D[tb][nb][v], acc[tb][nb][v]);
        }
    };

    // One K step k (stage k % 4, ring slot k % 2; both constants in the unrolled loop); one barrier every two steps
    // (s_barrier with an explicit wait: a __syncthreads() fence would wait for every outstanding load). At the top of
    // an even step k: every wave is done with steps k - 2 and k - 1 (stages (k + 2) % 4 and (k + 3) % 4 are free and
    // take the DMA of steps k + 2 and k + 3 now), and the DMA of steps k and k + 1 (issued at the top of step k - 2)
    // has landed in every wave and is visible. Each step sums its own stage; the sums meet the end after one more
    // barrier. (A barrier a step, with the DMA three steps ahead, measured 2-3 % slower.)
    // How the wait count is derived (vmcnt counts a wave's vector memory operations and they complete in issue order):
    //   after its DMA pair (kDmaPerWave each, first in the even step) a wave issues, up to the next even step, the
    //   codes of two steps (2 after each half's MFMAs, in `compute`: 8) and at most one scale window pair (steps j
    //   with j % 4 == 3 issue one: 2), kBetween = 10 loads. With at most kBetween outstanding at the top of step k,
    //   the pair issued at the top of step k - 2 has landed; what may still be out are register loads, which the
    //   compiler waits for before their first use. A wave with no DMA (!dma_on) has no pair to wait for; the same
    //   count only waits for older register loads. The DMA of other waves is covered by their own wait before the
    //   same barrier.
    // A change to what a step issues, or to the order, changes these counts: re-derive them, and run the
    // grouped kernels twice on the same inputs (the parity tests do) - a load landing after its use shows up as
    // run-to-run differences.
    constexpr int kBetween = 10;
    auto step = [&](int k, auto st_tag, auto rs_tag, auto two_tag) __attribute__((always_inline)) {
        constexpr int ST = decltype(st_tag)::value;
        if constexpr (ST % 2 == 0) {
            asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(kBetween) : "memory");
            issue_x(k + 2, (ST + 2) % kStages);
            issue_x(k + 3, (ST + 3) % kStages);
            __builtin_amdgcn_sched_barrier(0);
        }
        sum_rows(ST, k);
        compute(k, ST, rs_tag, two_tag);
    };

    // prologue: steps 0 and 1 of activations and of weights; vmcnt(0): all landed in this wave, and the barrier makes
    // every wave's DMA visible
    issue_x(0, 0), issue_x(1, 1);
    issue_codes(0, cw[0], 0), issue_codes(0, cw[0], 1), issue_window(0, wcur);
    issue_codes(1, cw[1], 0), issue_codes(1, cw[1], 1), issue_window(4, wnxt);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    // unrolled by the stage count (a multiple of the ring depth) so that stages and ring slots are constants; one
    // copy for tiles of more than 32 slots and one for the rest (no branch inside the K loop)
    auto run = [&](auto two_tag) __attribute__((always_inline)) {
        for (int k = 0;; k += kStages) {
            if (k >= nk) break;
            step(k, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, two_tag);
            if (k + 1 >= nk) break;
            step(k + 1, std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{}, two_tag);
            if (k + 2 >= nk) break;
            step(k + 2, std::integral_constant<int, 2>{}, std::integral_constant<int, 0>{}, two_tag);
            if (k + 3 >= nk) break;
            step(k + 3, std::integral_constant<int, 3>{}, std::integral_constant<int, 1>{}, two_tag);
        }
    };
    if (two_tb) run(std::true_type{});
    else run(std::false_type{});
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // every wave's span sums are in LDS
    // The scales and mins of the lane's spans for the end below, every load issued before the first use and before
    // the drain (their latency overlaps it): 4-byte loads (two spans each; a row's scales start 8-byte aligned, as
    // ngroups % 4 == 0 and the view is 4-byte aligned), clamped into the row, the spans past nk zeroed below (nk % 4
    // == 0, so a pair is wholly in or out).
    constexpr int kPasses = L::kMaxGroups / 16;  // 16 spans a pass
    uint32_t sm[kPasses][2][2][4];  // [pass][nb][scale, min][pair]
#pragma unroll
    for (int g = 0; g < kPasses; ++g)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int at = min(g * 16 + h * 8 + 2 * i, nk - 2);
                sm[g][nb][0][i] = *reinterpret_cast<const uint32_t *>(srow[nb] + at);
                sm[g][nb][1][i] = *reinterpret_cast<const uint32_t *>(mrow[nb] + at);
            }
    // vmcnt(0): the clamped loads past the end (steps nk .. nk + 2, never used) land before the block exits - a DMA
    // still in flight at exit would write into LDS that the next block on this compute unit may own
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // ---- sum over the spans of (m - 128 s)[row] * sum x[slot], on the MFMA: 16 spans an instruction, both operands
    // split into three BF16 terms (t0 = rne(v), t1 = rne(v - t0), t2 = rne(v - t0 - t1): 24 significant bits, as
    // the FP32 fold this replaces; the term largely cancels s * 128 * sum x inside s * D, so 16 bits would not do).
    // The six products down to 2^-16 of the whole; the rest (below 2^-24) are dropped. Every wave's span sums are in
    // LDS: the barrier after the K loop. ----
    auto split3 = [](const float (&v)[8], bf16x8 (&t)[3]) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const __bf16 a = (__bf16)v[e];
            const float r1 = v[e] - (float)a;
            const __bf16 b = (__bf16)r1;
            t[0][e] = a, t[1][e] = b, t[2][e] = (__bf16)(r1 - (float)b);
        }
    };
#pragma unroll
    for (int g = 0; g < kPasses; ++g) {
        const int g0 = g * 16;
        if (g0 >= nk) break;
        const int gl = g0 + h * 8;  // this lane's 8 spans
        bf16x8 bt[2][3];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            float cmv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t sw = sm[g][nb][0][e / 2], mw = sm[g][nb][1][e / 2];
                const float sv = __uint_as_float((e & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
                const float mv = __uint_as_float((e & 1) ? (mw & 0xFFFF0000u) : (mw << 16));
                cmv[e] = gl + e < nk ? fmaf(-L::kOff, sv, mv) : 0.f;
            }
            split3(cmv, bt[nb]);
        }
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            if (tb == 1 && !two_tb) continue;
            float xv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) xv[e] = gl + e < nk ? xsum[(tb * 32 + j) * kSumStride + gl + e] : 0.f;
            bf16x8 at[3];
            split3(xv, at);
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
                for (int pa = 0; pa < 3; ++pa)
#pragma unroll
                    for (int pb = 0; pb < 3 - pa; ++pb)  // (0,0) (0,1) (0,2) (1,0) (1,1) (2,0)
                        acc[tb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(at[pa], bt[nb][pb], acc[tb][nb], 0, 0, 0);
            }
        }
    }

    // ---- stores: tile (tb, nb), lane value v = slot tb * 32 + 8 (v / 4) + 4 h + v % 4, row j of the tile ----
    if constexpr (sizeof(TY) == 2 && MODE != qmm::COMBINE) {
        if (p.vec_store) {
            // BF16 output through LDS: the wave's 64 slots x kF features go to its own stage array (every wave is
            // past its K loop and has drained its DMA - vmcnt(0) above - once all pass this barrier), then out
            // as 16-byte stores of 8 features: a quarter (SwiGLU: an eighth) of the store instructions of one
            // 2-byte store a value, with no per-value address arithmetic
            constexpr int kF = MODE == qmm::SWIGLU ? 32 : 64, kRowB = kF * 2, kChunksRow = kF / 8;
            static_assert(kBM * kRowB <= L::kStageBytes, "a wave's staged outputs fit its stage array");
            asm volatile("s_barrier" ::: "memory");
            unsigned char *stg = xs_at(wave);
            TY *hy = static_cast<TY *>(p.y);
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                if (tb == 1 && !two_tb) break;  // rows 32..63 hold no slot (uniform)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = tb * 32 + 8 * (v / 4) + 4 * h + v % 4;
                    if constexpr (MODE == qmm::SWIGLU) {
                        const float gv = as_stored(acc[tb][0][v], hy), uv = as_stored(acc[tb][1][v], hy);
                        *reinterpret_cast<uint16_t *>(stg + r * kRowB + j * 2) =
                            (uint16_t)f32_to_bf16(as_stored(silu(gv), hy) * uv);
                    } else {
#pragma unroll
                        for (int nb = 0; nb < 2; ++nb)
                            *reinterpret_cast<uint16_t *>(stg + r * kRowB + (nb * 32 + j) * 2) =
                                (uint16_t)f32_to_bf16(acc[tb][nb][v]);
                    }
                }
            }
            const int64_t fbase = r0 + wave * kF;  // the wave's first output row (feature)
#pragma unroll
            for (int i = 0; i < kBM * kChunksRow / 64; ++i) {
                const int c = lane + 64 * i, r = c / kChunksRow, cc = c % kChunksRow;
                const int64_t f = fbase + cc * 8;  // Nrows % 8 == 0: a chunk is wholly in or out
                const uint4 val = *reinterpret_cast<const uint4 *>(stg + r * kRowB + cc * 16);
                if (r < T && f < Nrows) *reinterpret_cast<uint4 *>(hy + s_out[r] * Nrows + f) = val;
            }
            return;
        }
    }
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = tb * 32 + 8 * (v / 4) + 4 * h + v % 4;
            if (r >= T) continue;
            const int64_t o = s_out[r] * Nrows;
            if constexpr (MODE == qmm::SWIGLU) {
                if (feat[0] < Nrows) {
                    TY *hy = static_cast<TY *>(p.y);
                    const float gv = as_stored(acc[tb][0][v], hy), uv = as_stored(acc[tb][1][v], hy);
                    store_act(hy, o + feat[0], as_stored(silu(gv), hy) * uv);
                }
            } else {
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    if (feat[nb] >= Nrows) continue;
                    if constexpr (MODE == qmm::COMBINE) static_cast<float *>(p.y)[o + feat[nb]] = acc[tb][nb][v];
                    else store_act(static_cast<TY *>(p.y), o + feat[nb], acc[tb][nb][v]);
                }
            }
        }
}

// ---------------- down at prefill width: the tile's activations resident ----------------
// COMBINE with K <= 1024 (the experts' down projection, K = I). gg_kernel pays, for every 256 weight rows, the tile's
// set-up, the activation DMA of every K step, the pipeline's fill and a barrier a step, and at K = 1024 a block has
// only 8 K steps to spread them over. Here a block of 16 waves stages its 64-slot tile's activations over the whole
// K in LDS once (128 KB at K = 1024, in gg_kernel's K-step layout, with gg_kernel's span sums) and then streams chunk
// after chunk of 512 weight rows against them, a wave 32 rows x the 64 slots (2 v_mfma_f32_32x32x16_bf16 tiles a
// step): the K loop only reads LDS, so it has no barrier, and four waves a SIMD (a wave's registers fit in 128)
// hide each other's latencies. The codes and scales of the step two ahead (across chunk ends) and each chunk's
// scales and mins for the final fold are ordinary loads the compiler waits for. A block takes the chunks
// [part * n / kPdSplits, (part + 1) * n / kPdSplits) of its tile, handed out to its waves a 32-row slice at a time
// from an LDS counter (statically, a wave a chunk's slice, the four waves of a SIMD ended far apart: 486 -> 474 us for
// config 4's down + combine).
constexpr int kPdThreads = 1024, kPdWaves = 16, kPdMaxSteps = 8;
constexpr int kPdChunkRows = kPdWaves * 32;
constexpr int kPdSumStride = kPdMaxSteps + 4;  // floats a row of the span sums
constexpr int kPdSplits = 2;                   // blocks a tile

// The step's fold happens in the step: an empty asm that takes the 16 sums as operands (otherwise the compiler moves
// every step's fold to the chunk's end and keeps all the steps' MFMA results alive, far more than the registers hold).
__device__ __forceinline__ void pin16(f32x16 &a) {
    asm volatile("" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7]),
                 "+v"(a[8]), "+v"(a[9]), "+v"(a[10]), "+v"(a[11]), "+v"(a[12]), "+v"(a[13]), "+v"(a[14]), "+v"(a[15]));
}

template <int NK, bool TWO>
__device__ __forceinline__ void pd_run(const Params &p, const unsigned char *xs, const float *xsum,
                                       const int64_t *s_out, int T, int bucket, int c0, int c1, int *slice_ctr) {
    using Win = std::conditional_t<NK == 8, uint4, uint2>;  // a row's NK BF16 scales (or mins)
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int j = lane & 31, h = lane >> 5;
    const int64_t N = p.N, rowbytes = p.K / 2;
    // slice s: rows 32 (s % kPdWaves) .. + 31 of chunk c0 + s / kPdWaves; a wave takes slice `wave` first, then the
    // next one from the block's counter (the waves of a SIMD do not progress at one rate: handed out statically,
    // the block's last waves ended long after its first). The lane's weight row of slice s (past the end: the last
    // slice again, loaded and never used), clamped into the expert:
    const int nsl = (c1 - c0) * kPdWaves;
    auto feat_of = [&](int s) -> int64_t {
        s = min(s, nsl - 1);
        return (int64_t)(c0 + s / kPdWaves) * kPdChunkRows + (s % kPdWaves) * 32 + j;
    };
    auto row_of = [&](int s) -> int64_t {
        const int64_t n = feat_of(s);
        return (int64_t)bucket * N + (n < N ? n : N - 1);
    };
    uint4 cw[2][2];     // [ring slot][half]: the step's 32 bytes of codes
    uint32_t sc[2];     // [ring slot]: its scale
    auto issue = [&](int64_t row, int k, int RS, int half) {
        cw[RS][half] = *reinterpret_cast<const uint4 *>(p.q + row * rowbytes + h * 32 + k * kSpanBytes + half * 16);
        if (half == 1) sc[RS] = p.scale[row * NK + k];
    };
    Win wsc, wmn;  // the chunk's scales and mins for the final fold (loaded at its third step)
    auto word = [](const Win &w, int s) -> uint32_t {
        if constexpr (NK == 8) return qmm::detail::dword(w, s >> 1);
        else return s < 2 ? w.x : w.y;
    };
    auto bf = [&](const Win &w, int s) {
        const uint32_t d = word(w, s);
        return __uint_as_float((s & 1) ? (d & 0xFFFF0000u) : (d << 16));
    };
    {
        const int64_t r0 = row_of(wave);
        issue(r0, 0, 0, 0), issue(r0, 0, 0, 1), issue(r0, 1, 1, 0), issue(r0, 1, 1, 1);
    }
    // LDS address of the lane's A fragment of MFMA step kk, K step k, half tb: a_base[tb] ^ (kk << 4) plus the
    // stage (the row's slot kk ^ (row & 15), as (h * 8 + kk) ^ (row & 15) = (h * 8 ^ (row & 15)) ^ kk)
    uint32_t a_base[2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        const int row = tb * 32 + j;
        a_base[tb] = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const unsigned char *)(
                         xs + row * 256 + (((h * 8) ^ (row & 15)) * 16));
    }
    auto chunk = [&](int c, int cn) __attribute__((always_inline)) {
        const int64_t rc = row_of(c), rn = row_of(cn);
        f32x16 acc[2] = {f32x16{}, f32x16{}};
        auto kstep = [&](auto k_tag) __attribute__((always_inline)) {
            constexpr int k = decltype(k_tag)::value, RS = k & 1;
            constexpr int kn = (k + 2) % NK;  // the step whose loads this one issues: of this chunk or the next
            const int64_t rl = k + 2 < NK ? rc : rn;
            if constexpr (k == (NK == 8 ? 2 : 1)) {
                wsc = *reinterpret_cast<const Win *>(p.scale + rc * NK);
                wmn = *reinterpret_cast<const Win *>(p.minv + rc * NK);
            }
            // opaque to the compiler: the A addresses below are formed in the step (hoisted, one for every MFMA
            // step and half would hold 16 registers throughout)
            uint32_t ab0 = a_base[0], ab1 = a_base[1];
            asm volatile("" : "+v"(ab0), "+v"(ab1));
            f32x16 D[2];
            bf16x8 aop[2][2];  // [buffer][tb], one MFMA step ahead
            auto load_a = [&](int kk, bf16x8 (&a)[2]) __attribute__((always_inline)) {
#pragma unroll
                for (int tb = 0; tb < 2; ++tb) {
                    if (tb == 1 && !TWO) continue;
                    const uint32_t ad = ((tb == 0 ? ab0 : ab1) ^ (uint32_t)(kk << 4)) + k * kStageBytes;
                    a[tb] = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8 *>((uintptr_t)ad);
                }
            };
            load_a(0, aop[0]);
#pragma unroll
            for (int half = 0; half < 2; ++half) {
#pragma unroll
                for (int kq = 0; kq < 4; ++kq) {
                    const int kk = half * 4 + kq;
                    if (kk < 7) load_a(kk + 1, aop[(kk + 1) & 1]);
                    const bf16x8 bop = codes_nat(qmm::detail::dword(cw[RS][half], kq));
#pragma unroll
                    for (int tb = 0; tb < 2; ++tb) {
                        if (tb == 1 && !TWO) continue;
                        D[tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aop[kk & 1][tb], bop, kk == 0 ? f32x16{} : D[tb],
                                                                        0, 0, 0);
                    }
                }
                if (half == 0) issue(rl, kn, RS, 0);
            }
            const float s_ = __uint_as_float(sc[RS] << 16);
            issue(rl, kn, RS, 1);
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                if (tb == 1 && !TWO) continue;
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[tb][v] = fmaf(s_, D[tb][v], acc[tb][v]);
                pin16(acc[tb]);
            }
        };
        [&]<int... Ks>(std::integer_sequence<int, Ks...>) {
            ((kstep(std::integral_constant<int, Ks>{}), __builtin_amdgcn_sched_barrier(0)), ...);
        }(std::make_integer_sequence<int, NK>{});
        // (m - 128 s)[row] * sum x[slot] over the spans on the MFMA, as gg_kernel's (three BF16 terms a side)
        auto split3 = [](const float (&v)[8], bf16x8 (&t)[3]) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const __bf16 a = (__bf16)v[e];
                const float r1 = v[e] - (float)a;
                const __bf16 b = (__bf16)r1;
                t[0][e] = a, t[1][e] = b, t[2][e] = (__bf16)(r1 - (float)b);
            }
        };
        {
            bf16x8 bt[3];
            float cmv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)  // this lane's 8 spans are h * 8 ..: NK <= 8, so lanes of h = 1 hold none
                cmv[e] = (h == 0 && e < NK) ? fmaf(-128.f, bf(wsc, e & (NK - 1)), bf(wmn, e & (NK - 1))) : 0.f;
            split3(cmv, bt);
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                if (tb == 1 && !TWO) continue;
                float xv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[e] = (h == 0 && e < NK) ? xsum[(tb * 32 + j) * kPdSumStride + e] : 0.f;
                bf16x8 at[3];
                split3(xv, at);
#pragma unroll
                for (int pa = 0; pa < 3; ++pa)
#pragma unroll
                    for (int pb = 0; pb < 3 - pa; ++pb)
                        acc[tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(at[pa], bt[pb], acc[tb], 0, 0, 0);
            }
        }
        // FP32 partials: lane value v = slot tb * 32 + 8 (v / 4) + 4 h + v % 4, row j of the wave's 32. The slots'
        // output rows are read here, from an address the compiler cannot see is the same every chunk (hoisted out
        // of the chunk loop, the 32 row offsets would hold 64 registers throughout)
        const int64_t feat = feat_of(c);
        uint32_t so = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const int64_t *)s_out;
        int Tc = T, hc = h;  // likewise the slot bounds (hoisted: 32 masks in scalar registers)
        asm volatile("" : "+v"(so), "+s"(Tc), "+v"(hc));
        const __attribute__((address_space(3))) int64_t *outs =
            reinterpret_cast<const __attribute__((address_space(3))) int64_t *>((uintptr_t)so);
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = tb * 32 + 8 * (v / 4) + 4 * hc + v % 4;
                if (r < Tc && feat < N) static_cast<float *>(p.y)[outs[r] * N + feat] = acc[tb][v];
            }
    };
    for (int c = wave; c < nsl;) {  // wave-uniform
        int cn = 0;
        if (lane == 0) cn = atomicAdd(slice_ctr, 1);
        cn = __builtin_amdgcn_readfirstlane(cn);
        chunk(c, cn);
        c = cn;
    }
    // vmcnt(0): the clamped register loads issued past the last chunk (never used) land before the waves exit
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

__global__ void __launch_bounds__(kPdThreads, 1) gg_down_kernel(Params p) {
    __shared__ __attribute__((aligned(16))) unsigned char xs[kPdMaxSteps * kStageBytes];
    __shared__ __attribute__((aligned(16))) float xsum[kBM * kPdSumStride];  // [slot][span]
    __shared__ int64_t s_xrow[kBM], s_out[kBM];
    __shared__ int s_T, s_bucket, s_slice;
    const int tid = threadIdx.x, lane = tid & 63;
    const int64_t K = p.K, N = p.N;
    const int E = (int)p.E, nk = (int)(K / kSpan);
    const int u = (int)(blockIdx.x / kPdSplits), part = (int)(blockIdx.x % kPdSplits);

    if (tid < 64) {  // the tile: bucket, slots (gg_kernel's lookup)
        const int32_t *ws = p.ws;
        const int32_t n_wt = ws[3], S = ws[1];
        int T = 0, bucket = -1;
        if (u < n_wt) {
            const int32_t *offsets = ws + 4, *slots = offsets + E + 2;
            const int64_t Tmax = (int64_t)S / 16 + E + 2, WTmax = (int64_t)S / 64 + E + 2;
            const int32_t *wtile_bucket = slots + S + 2 * Tmax, *wtile_start = wtile_bucket + WTmax;
            bucket = wtile_bucket[u];
            const int32_t st = wtile_start[u];
            T = min(kBM, offsets[bucket + 1] - st);
            if (lane < T) {
                const int64_t slot = slots[st + lane];
                s_xrow[lane] = slot * K;
                s_out[lane] = slot;
            }
        }
        if (lane == 0) s_T = T, s_bucket = bucket;
    }
    __syncthreads();
    const int T = __builtin_amdgcn_readfirstlane(s_T), bucket = __builtin_amdgcn_readfirstlane(s_bucket);
    if (T == 0) return;
    const int nchunk = (int)((N + kPdChunkRows - 1) / kPdChunkRows);
    const int c0 = part * nchunk / kPdSplits, c1 = (part + 1) * nchunk / kPdSplits;
    if (c0 >= c1) return;
    if (bucket == E) {  // invalid ids (reported by the grouping): NaN rows, never an out-of-range weight read
        const int64_t f0 = (int64_t)c0 * kPdChunkRows, f1 = min((int64_t)c1 * kPdChunkRows, N);
        for (int64_t i = tid; i < (int64_t)T * (f1 - f0); i += kPdThreads) {
            const int r = (int)(i / (f1 - f0));
            static_cast<float *>(p.y)[s_out[r] * N + f0 + i % (f1 - f0)] = qnan();
        }
        return;
    }
    if (tid >= T && tid < kBM) s_xrow[tid] = s_xrow[T - 1];  // rows past T: row T - 1 again, never stored
    __syncthreads();

    // the tile's activations over the whole K into LDS: chunk c8 (8 BF16) of row r to K step c8 / 16, slot
    // (c8 % 16) ^ (r % 16) of the row (gg_kernel's DMA layout); all loads go out first
    constexpr int kPer = (kPdMaxSteps * kSpan / 8 * kBM + kPdThreads - 1) / kPdThreads;  // 8
    const int chunks8 = (int)(K / 8), n_items = kBM * chunks8;
    uint4 xv[kPer];
#pragma unroll
    for (int b = 0; b < kPer; ++b) {
        const int i = min(b * kPdThreads + tid, n_items - 1);
        xv[b] = *reinterpret_cast<const uint4 *>(p.x + s_xrow[i / chunks8] + (int64_t)(i % chunks8) * 8);
    }
#pragma unroll
    for (int b = 0; b < kPer; ++b) {
        const int i = b * kPdThreads + tid;
        if (i < n_items) {
            const int r = i / chunks8, c8 = i % chunks8;
            *reinterpret_cast<uint4 *>(xs + (c8 >> 4) * kStageBytes + r * 256 + (((c8 & 15) ^ (r & 15)) * 16)) = xv[b];
        }
    }
    __syncthreads();
    // the span sums, as gg_kernel's: 4 threads a (row, span), 4 chunks each in chunk order, then summed across the 4
    for (int it = tid; it < nk * kBM * 4; it += kPdThreads) {
        const int g = it >> 8, r = (it >> 2) & (kBM - 1), qd = it & 3;
        const unsigned char *grp0 = xs + g * kStageBytes + r * 256 + ((qd ^ ((r & 15) >> 2)) * 64);
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // chunk 4 qd + i, in slot (4 qd + i) ^ (r & 15)
            float v[8];
            qmm::detail::unpack8(*reinterpret_cast<const uint4 *>(grp0 + ((i ^ (r & 3)) * 16)), v);
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += v[e];
        }
        sum = qmm::detail::group_sum_c<4>(sum);
        if (qd == 0) xsum[r * kPdSumStride + g] = sum;
    }
    if (tid == 0) s_slice = kPdWaves;  // the first slices are the waves' own
    __syncthreads();
    const bool two = T > 32;
    if (nk == 8) two ? pd_run<8, true>(p, xs, xsum, s_out, T, bucket, c0, c1, &s_slice) : pd_run<8, false>(p, xs, xsum, s_out, T, bucket, c0, c1, &s_slice);
    else two ? pd_run<4, true>(p, xs, xsum, s_out, T, bucket, c0, c1, &s_slice) : pd_run<4, false>(p, xs, xsum, s_out, T, bucket, c0, c1, &s_slice);
}

// ---------------- dense linear below full width: K split over the block's waves ----------------
// gg_kernel gives a block 64 tokens x 256 rows and walks the whole K a step at a time behind a block barrier; with
// few tokens there are few blocks (M = 256, N = 4096: 64 of them, one a CU for a quarter of the chip) and the time is
// the latency of K / 128 steps, whatever M is. Here a block owns 64 tokens x 64 output rows and its four waves take a
// quarter of K each (nk / 4 K steps), so the grid is four times larger and every wave's chain four times shorter.
// A wave loads its step's 64 activation rows into registers with row-contiguous 16-byte loads (kChunks lanes a row),
// two steps ahead, and at the step turns them around through its own LDS stage (gg_kernel's swizzled
// layout) into MFMA operands; the codes of its weight rows come as gg_kernel's. No DMA and no block barrier in the
// K loop: every load is an ordinary one, so the compiler's own wait counts stay exact. A lane sums its half of each
// span from its operand registers (the two halves are added after the loop); the quarter's scales and mins are
// loaded once, up front. At the end the four waves' FP32 sums meet in LDS and wave w adds, in wave order, and stores
// tile (tb, nb) = (w / 2, w % 2).

template <typename TY, int BITS>
__global__ void __launch_bounds__(kThreads, 1) gs_kernel(Params p) {
    using L = Lay<BITS>;
    constexpr int kSpan = L::kSpan, kKk = L::kKk, kMaxQ = L::kMaxGroups / 4;
    constexpr int kChunks = L::kChunks, kRowsPerLoad = 64 / kChunks;
    __shared__ __attribute__((aligned(16))) float red[kWaves][4][16][64];  // [wave][tile][value][lane]
    __shared__ __attribute__((aligned(L::kStageAlign))) unsigned char stage[kWaves][L::kStageBytes];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int j = lane & 31, h = lane >> 5;
    const int64_t K = p.K, N = p.N, M = p.dense_M;
    const int nk = (int)(K / kSpan), nq = nk / 4, q0 = wave * nq;  // this wave's K steps: q0 .. q0 + nq - 1
    const int nrg = (int)((N + 63) / 64);
    const int u = (int)(blockIdx.x / nrg), g = (int)(blockIdx.x % nrg);
    const int64_t t0 = (int64_t)u * kBM, n0 = (int64_t)g * 64;
    const int T = (int)min((int64_t)kBM, M - t0);
    // load i of a step: token row kRowsPerLoad i + lane / kChunks (past M: the last token again, never stored),
    // chunk lane % kChunks; weight rows nb = 0, 1 of the lane (past N: the last row again)
    const int64_t xrow0 = t0 + lane / kChunks;
    const uint16_t *xq = p.x + (int64_t)q0 * kSpan + (lane % kChunks) * 8;
    unsigned char *stg = stage[wave];
    const int64_t rowbytes = BITS == 4 ? K / 2 : K, ngroups = nk;
    const uint8_t *qr[2];
    const uint16_t *sr[2], *mr[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int64_t row = min(n0 + nb * 32 + j, N - 1);
        qr[nb] = p.q + row * rowbytes + (int64_t)q0 * kSpanBytes + h * 32;
        sr[nb] = p.scale + row * ngroups + q0;
        mr[nb] = p.minv + row * ngroups + q0;
    }
    // the quarter's scales and mins (BF16 bits; indices clamped into it)
    uint32_t sq[2][kMaxQ], mq[2][kMaxQ];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int q = 0; q < kMaxQ; ++q) {
            const int qc = min(q, nq - 1);
            sq[nb][q] = sr[nb][qc];
            mq[nb][q] = mr[nb][qc];
        }
    // register slots of activations (kXR) and codes (kCR), each loaded kXR - 1 / kCR - 1 steps ahead (one wave a
    // SIMD: the registers are there). 4096 x 4096 at M = 256 against two of each: q4 three activation and two code
    // slots 23.6 -> 22.1 us (three code slots too: 22.6 us and a 36-byte spill a lane), q8 three of each 31.1 ->
    // 28.2 us (four no better). Separate arrays: one array of the slots ends up in scratch.
    constexpr int kXR = 3, kCR = BITS == 8 ? 3 : 2;
    uint4 xa0[kChunks], xa1[kChunks], xa2[kChunks];  // [load]: activations as loaded, slots 0..2
    uint4 cw[kCR][2][2];  // [slot][nb][half]: codes
    auto issue = [&](int q, int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const uint4 v = *reinterpret_cast<const uint4 *>(xq + min(xrow0 + kRowsPerLoad * i, M - 1) * K +
                                                             (int64_t)q * kSpan);
            if (slot == 0) xa0[i] = v;
            else if (slot == 1) xa1[i] = v;
            else xa2[i] = v;
        }
    };
    auto issue_c = [&](int q, int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
                cw[slot][nb][hf] = *reinterpret_cast<const uint4 *>(qr[nb] + (int64_t)q * kSpanBytes + hf * 16);
    };
    f32x16 acc[2][2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[tb][nb] = f32x16{};
    float hs[2][kMaxQ];  // the lane's half-span sums of its two token rows
#pragma unroll
    for (int s = 0; s < kCR - 1; ++s)
        if (s < nq) issue_c(s, s);
#pragma unroll
    for (int s = 0; s < kXR - 1; ++s)
        if (s < nq) issue(s, s);
    auto step = [&](auto q_tag) __attribute__((always_inline)) {
        constexpr int q = decltype(q_tag)::value, slot = q % kXR;
        if (q >= nq) return;  // uniform
        // the step's rows into the stage (chunk c of row r in slot c ^ swz(r)), then the lane's operands out of it.
        // One stage a wave: its reads of the step before are done (a wave's LDS operations complete in order).
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int r = kRowsPerLoad * i + lane / kChunks;
            *reinterpret_cast<uint4 *>(stg + r * L::kRowBytes + (((lane % kChunks) ^ L::swz(r)) * 16)) =
                slot == 0 ? xa0[i] : slot == 1 ? xa1[i] : xa2[i];
        }
        if (q + kXR - 1 < nq) issue(q + kXR - 1, (q + kXR - 1) % kXR);
        if (q + kCR - 1 < nq) issue_c(q + kCR - 1, (q + kCR - 1) % kCR);
        // lane (j, h)'s operand of MFMA kk, row tb * 32 + j, read one MFMA step ahead
        auto frag = [&](int kk, uint4 (&f)[2]) __attribute__((always_inline)) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                const int row = tb * 32 + j;
                f[tb] = *reinterpret_cast<const uint4 *>(stg + row * L::kRowBytes +
                                                         (((h * (kChunks / 2) + kk) ^ L::swz(row)) * 16));
            }
        };
        uint4 xf[2][2];  // [buffer][tb]
        frag(0, xf[0]);
        float hsum[2] = {0.f, 0.f};
        f32x16 D[2][2];
#pragma unroll
        for (int kk = 0; kk < kKk; ++kk) {
            if (kk + 1 < kKk) frag(kk + 1, xf[(kk + 1) & 1]);
            const int hf = kk / (kKk / 2), kq = kk % (kKk / 2);
            bf16x8 bop[2];
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const uint4 &c = cw[q % kCR][nb][hf];
                if constexpr (BITS == 4) bop[nb] = codes_nat(qmm::detail::dword(c, kq));
                else bop[nb] = codes8(qmm::detail::dword(c, 2 * kq), qmm::detail::dword(c, 2 * kq + 1));
            }
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                const bf16x8 a = __builtin_bit_cast(bf16x8, xf[kk & 1][tb]);
                hsum[tb] = sum_chunk(xf[kk & 1][tb], hsum[tb]);
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
                    D[tb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bop[nb], kk == 0 ? f32x16{} : D[tb][nb], 0, 0,
                                                                        0);
            }
        }
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) hs[tb][q] = hsum[tb];
        float s_[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) s_[nb] = __uint_as_float(sq[nb][q] << 16);
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int v = 0; v < 16; ++v)
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) acc[tb][nb][v] = fmaf(s_[nb], D[tb][nb][v], acc[tb][nb][v]);
    };
    [&]<int... Qs>(std::integer_sequence<int, Qs...>) {
        (step(std::integral_constant<int, Qs>{}), ...);
    }(std::make_integer_sequence<int, kMaxQ>{});

    // (m - kOff s)[row] * sum x[token] over the quarter's spans on the MFMA, as gg_kernel's end (three BF16 terms a
    // side): lane (j, h) holds token j's sums of spans 8 h .. 8 h + 7 (the two halves of a span added, in the same
    // order in both lanes) and row j's terms of the same spans
    static_assert(kMaxQ <= 16, "one 16-span MFMA pass");
    auto split3 = [](const float (&v)[8], bf16x8 (&t)[3]) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const __bf16 a = (__bf16)v[e];
            const float r1 = v[e] - (float)a;
            const __bf16 b = (__bf16)r1;
            t[0][e] = a, t[1][e] = b, t[2][e] = (__bf16)(r1 - (float)b);
        }
    };
    bf16x8 at[2][3], bt[2][3];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        float full[kMaxQ];
#pragma unroll
        for (int q = 0; q < kMaxQ; ++q) {
            const float mine = q < nq ? hs[tb][q] : 0.f;
            full[q] = mine + __shfl_xor(mine, 32);
        }
        float xv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float lo = full[e], hi = 8 + e < kMaxQ ? full[min(8 + e, kMaxQ - 1)] : 0.f;
            xv[e] = h ? hi : lo;
        }
        split3(xv, at[tb]);
    }
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        float cmv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int qlo = e, qhi = min(8 + e, kMaxQ - 1);
            const uint32_t sw = h ? sq[nb][qhi] : sq[nb][qlo], mw = h ? mq[nb][qhi] : mq[nb][qlo];
            const int qq = h * 8 + e;
            cmv[e] = qq < nq ? fmaf(-L::kOff, __uint_as_float(sw << 16), __uint_as_float(mw << 16)) : 0.f;
        }
        split3(cmv, bt[nb]);
    }
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
            for (int pa = 0; pa < 3; ++pa)
#pragma unroll
                for (int pb = 0; pb < 3 - pa; ++pb)
                    acc[tb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(at[tb][pa], bt[nb][pb], acc[tb][nb], 0, 0, 0);

    // ---- the four quarters' sums, added in wave order; wave w stores tile (tb, nb) = (w / 2, w % 2) ----
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) red[wave][t][v][lane] = acc[t / 2][t % 2][v];
    __syncthreads();
    const int tb = wave / 2, nb = wave % 2;
    const int64_t feat = n0 + nb * 32 + j;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const float y = ((red[0][wave][v][lane] + red[1][wave][v][lane]) + red[2][wave][v][lane]) + red[3][wave][v][lane];
        const int r = tb * 32 + 8 * (v / 4) + 4 * h + v % 4;
        if (r < T && feat < N) store_act(static_cast<TY *>(p.y), (t0 + r) * N + feat, y);
    }
}

// ---------------- dense linear at full prefill width: 128 tokens a wave ----------------
// gg_kernel's wave owns 64 tokens x 64 rows: each dequantized weight fragment feeds two MFMAs, and the step's VALU
// work (dequant, the per-span fold, the span sums: ~9 operations an MFMA) is about as long as its MFMAs, which the
// two waves of a SIMD overlap only in part. Here (dense linears above kDenseSplitMaxTokens tokens: every token tile
// but the last is full) a block of 8 waves owns 128 tokens x 256 rows, one block a compute unit (two waves a SIMD),
// and a wave owns 128 tokens x 32 rows as 4 MFMA tiles: each weight fragment feeds four MFMAs, so the dequant an
// MFMA halves (~5.7 VALU operations an MFMA) for twice the activation operand reads from LDS, and one barrier every
// two K steps (the block's eight waves meet at each). Otherwise gg_kernel's arithmetic (span sums, fold, the end's span term on the MFMA) for every
// output: the results are the same bits. Used where its grid fills the chip (128-token tiles x 256-row blocks >= the
// compute units): 4096 x 4096 at M = 2048, q4 81.8 -> 71.5 us, q8 117.9 -> 91.4 us.
constexpr int kGwThreads = 512, kGwWaves = 8, kGwBM = 128, kGwTB = kGwBM / 32, kGwRows = kGwWaves * 32;

template <int BITS>
struct LayW {
    static constexpr int kStageBytes = kGwBM * Lay<BITS>::kRowBytes;  // 32 KB / 16 KB
    static constexpr int kDmaPerWave = kStageBytes / 1024 / kGwWaves;  // 4 / 2
};

template <typename TY, int BITS>
__global__ void __launch_bounds__(kGwThreads, 1) gw_kernel(Params p) {
    using L = Lay<BITS>;
    using W = LayW<BITS>;
    constexpr int kSpan = L::kSpan, kStageBytes = W::kStageBytes, kDmaPerWave = W::kDmaPerWave,
                  kSumStride = L::kSumStride, kChunks = L::kChunks;
    __shared__ __attribute__((aligned(L::kStageAlign))) unsigned char x0[kStageBytes], x1[kStageBytes],
        x2[kStageBytes], x3[kStageBytes];
    __shared__ __attribute__((aligned(16))) float xsum[kGwBM * kSumStride];  // [token][span]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31, h = lane >> 5;
    const int64_t K = p.K, N = p.N, M = p.dense_M;
    const int64_t t0 = (int64_t)tile_of(blockIdx.x, p.nrb) * kGwBM;
    if (t0 >= M) return;  // past the tile count: uniform for the block
    const int T = (int)min((int64_t)kGwBM, M - t0);
    const int64_t r0 = (int64_t)rowblock_of(blockIdx.x, p.nrb) * kGwRows;

    // this lane's weight row, clamped into the weight (stores are masked)
    const int64_t rowbytes = BITS == 4 ? K / 2 : K, ngroups = K / kSpan;
    const int64_t feat = r0 + wave * 32 + j;
    const int64_t wrow = min(feat, N - 1);
    const uint8_t *qrow = p.q + wrow * rowbytes + h * 32;
    const uint16_t *srow = p.scale + wrow * ngroups, *mrow = p.minv + wrow * ngroups;
    // activation DMA: instruction I covers kDmaRows token rows from kDmaRows I (rows past T: token T - 1 again, never
    // stored); lane l writes row kDmaRows I + l / kChunks, slot l % kChunks with chunk (l % kChunks) ^ swz(row)
    constexpr int kDmaRows = 64 / kChunks;
    const uint16_t *xl[kDmaPerWave];
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
        const int r = kDmaRows * (kDmaPerWave * wave + i) + lane / kChunks;
        xl[i] = p.x + (t0 + min(r, T - 1)) * K + (((lane % kChunks) ^ L::swz(r)) * 8);
    }
    auto xs_at = [&](int st) -> unsigned char * { return st == 0 ? x0 : st == 1 ? x1 : st == 2 ? x2 : x3; };
    const int nk = (int)(K / kSpan);
    auto issue_x = [&](int kstep, int st) __attribute__((always_inline)) {
        const int k = min(kstep, nk - 1);
#pragma unroll
        for (int i = 0; i < kDmaPerWave; ++i)
            dma16(xl[i] + (int64_t)k * kSpan, xs_at(st) + (kDmaPerWave * wave + i) * 1024);
    };
    uint4 cw[2][2];      // [ring slot][half of the lane's 32 bytes]
    uint2 wcur, wnxt;    // the scales of 4 steps
    auto issue_codes = [&](int kstep, uint4 (&w)[2], int half) {
        const int k = min(kstep, nk - 1);
        w[half] = *reinterpret_cast<const uint4 *>(qrow + (int64_t)k * kSpanBytes + half * 16);
    };
    auto issue_window = [&](int kstep, uint2 &w) {  // steps kstep .. kstep + 3 (clamped: nk % 4 == 0)
        w = *reinterpret_cast<const uint2 *>(srow + min(kstep, nk - 4));
    };
    // the span sums of stage st's 128 rows (K step grp), gg_kernel's: 4 threads a row, the chunks in chunk order;
    // the reads in asm ending in lgkmcnt(0) (the step's barrier already covers this stage's DMA)
    auto sum_rows = [&](int st, int grp) __attribute__((always_inline)) {
        const int r = tid >> 2, qd = tid & 3;
        float sum = 0.f;
        if constexpr (BITS == 8) {
            const uint32_t at = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const unsigned char *)(
                xs_at(st) + r * 128 + (((2 * qd) ^ L::swz(r)) * 16));
            uint4 raw[2];
            uint32_t tmp;
            asm volatile("ds_read_b128 %0, %3\n\t"
                         "v_xor_b32 %2, 16, %3\n\tds_read_b128 %1, %2\n\ts_waitcnt lgkmcnt(0)"
                         : "=&v"(raw[0]), "=&v"(raw[1]), "=&v"(tmp)
                         : "v"(at));
#pragma unroll
            for (int i = 0; i < 2; ++i) sum = sum_chunk(raw[i], sum);
        } else {
            const uint32_t grp0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const unsigned char *)(
                xs_at(st) + r * 256 + ((qd ^ ((r & 15) >> 2)) * 64));
            const uint32_t at = grp0 + ((uint32_t)(r & 3) << 4);
            uint4 raw[4];
            uint32_t tmp;
            asm volatile("ds_read_b128 %0, %5\n\t"
                         "v_xor_b32 %4, 16, %5\n\tds_read_b128 %1, %4\n\t"
                         "v_xor_b32 %4, 32, %5\n\tds_read_b128 %2, %4\n\t"
                         "v_xor_b32 %4, 48, %5\n\tds_read_b128 %3, %4\n\ts_waitcnt lgkmcnt(0)"
                         : "=&v"(raw[0]), "=&v"(raw[1]), "=&v"(raw[2]), "=&v"(raw[3]), "=&v"(tmp)
                         : "v"(at));
#pragma unroll
            for (int i = 0; i < 4; ++i) sum = sum_chunk(raw[i], sum);
        }
        sum = qmm::detail::group_sum_c<4>(sum);
        if (qd == 0 && grp < nk) xsum[r * kSumStride + grp] = sum;
    };

    f32x16 acc[kGwTB];
#pragma unroll
    for (int tb = 0; tb < kGwTB; ++tb) acc[tb] = f32x16{};
    // one K step on stage st with ring slot RS; the ring slot is re-loaded (step k + 2) as its codes are used
    auto compute = [&](int k, int st, auto rs_tag) __attribute__((always_inline)) {
        constexpr int RS = decltype(rs_tag)::value;
        const unsigned char *xb = xs_at(st);
        f32x16 D[kGwTB];
        bf16x8 aop[2][kGwTB];  // [buffer][tb], one MFMA step ahead
        auto load_a = [&](int kk, bf16x8 (&a)[kGwTB]) __attribute__((always_inline)) {
#pragma unroll
            for (int tb = 0; tb < kGwTB; ++tb) {
                const int row = tb * 32 + j;
                a[tb] = *reinterpret_cast<const bf16x8 *>(xb + row * L::kRowBytes +
                                                          (((h * (kChunks / 2) + kk) ^ L::swz(row)) * 16));
            }
        };
        load_a(0, aop[0]);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
            for (int kq = 0; kq < L::kKk / 2; ++kq) {
                const int kk = half * (L::kKk / 2) + kq;
                if (kk < L::kKk - 1) load_a(kk + 1, aop[(kk + 1) & 1]);
                const uint4 &c = cw[RS][half];
                bf16x8 bop;
                if constexpr (BITS == 4) bop = codes_nat(qmm::detail::dword(c, kq));
                else bop = codes8(qmm::detail::dword(c, 2 * kq), qmm::detail::dword(c, 2 * kq + 1));
#pragma unroll
                for (int tb = 0; tb < kGwTB; ++tb)
                    D[tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aop[kk & 1][tb], bop, kk == 0 ? f32x16{} : D[tb],
                                                                    0, 0, 0);
            }
            issue_codes(k + 2, cw[RS], half);  // this half's codes are in the operands
        }
        const uint32_t wd = (st & 2) ? wcur.y : wcur.x;
        const float s_ = __uint_as_float((st & 1) ? (wd & 0xFFFF0000u) : (wd << 16));
        if (st == 3) {  // the next window becomes current (loaded four steps ago); the one after is issued
            wcur = wnxt;
            issue_window(k + 5, wnxt);
        }
#pragma unroll
        for (int tb = 0; tb < kGwTB; ++tb)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[tb][v] = fmaf(s_, D[tb][v], acc[tb][v]);
    };
    // One barrier every two K steps: at the top of an even step k every wave has finished steps k - 2 and k - 1
    // (their stages are free) and the DMA of steps k and k + 1 (issued at the top of step k - 2) is visible; the DMA of
    // steps k + 2 and k + 3 goes out into the freed stages. Wait count: after a DMA pair a wave issues the code loads
    // of two steps (2 each) and at most one scale window (every fourth step) before the next barrier, so with at most
    // kBetween loads outstanding the pair has landed (vmcnt counts a wave's loads, completed in issue order).
    constexpr int kBetween = 5;
    auto step = [&](int k, auto st_tag, auto rs_tag) __attribute__((always_inline)) {
        constexpr int ST = decltype(st_tag)::value;
        if constexpr (ST % 2 == 0) {
            asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(kBetween) : "memory");
            issue_x(k + 2, (ST + 2) % kStages);
            issue_x(k + 3, (ST + 3) % kStages);
            __builtin_amdgcn_sched_barrier(0);
        }
        sum_rows(ST, k);
        compute(k, ST, rs_tag);
    };
    issue_x(0, 0), issue_x(1, 1);
    issue_codes(0, cw[0], 0), issue_codes(0, cw[0], 1), issue_window(0, wcur);
    issue_codes(1, cw[1], 0), issue_codes(1, cw[1], 1), issue_window(4, wnxt);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    for (int k = 0;; k += kStages) {
        if (k >= nk) break;
        step(k, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
        if (k + 1 >= nk) break;
        step(k + 1, std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
        if (k + 2 >= nk) break;
        step(k + 2, std::integral_constant<int, 2>{}, std::integral_constant<int, 0>{});
        if (k + 3 >= nk) break;
        step(k + 3, std::integral_constant<int, 3>{}, std::integral_constant<int, 1>{});
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // every wave's span sums are in LDS
    // the end's scales and mins (gg_kernel's), then the drain of the clamped loads past the end
    constexpr int kPasses = L::kMaxGroups / 16;
    uint32_t sm[kPasses][2][4];  // [pass][scale, min][pair]
#pragma unroll
    for (int g = 0; g < kPasses; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int at = min(g * 16 + h * 8 + 2 * i, nk - 2);
            sm[g][0][i] = *reinterpret_cast<const uint32_t *>(srow + at);
            sm[g][1][i] = *reinterpret_cast<const uint32_t *>(mrow + at);
        }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // sum over the spans of (m - off s)[row] * sum x[token] on the MFMA, gg_kernel's three BF16 terms a side
    auto split3 = [](const float (&v)[8], bf16x8 (&t)[3]) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const __bf16 a = (__bf16)v[e];
            const float r1 = v[e] - (float)a;
            const __bf16 b = (__bf16)r1;
            t[0][e] = a, t[1][e] = b, t[2][e] = (__bf16)(r1 - (float)b);
        }
    };
#pragma unroll
    for (int g = 0; g < kPasses; ++g) {
        const int g0 = g * 16;
        if (g0 >= nk) break;
        const int gl = g0 + h * 8;
        bf16x8 bt[3];
        {
            float cmv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t sw = sm[g][0][e / 2], mw = sm[g][1][e / 2];
                const float sv = __uint_as_float((e & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
                const float mv = __uint_as_float((e & 1) ? (mw & 0xFFFF0000u) : (mw << 16));
                cmv[e] = gl + e < nk ? fmaf(-L::kOff, sv, mv) : 0.f;
            }
            split3(cmv, bt);
        }
#pragma unroll
        for (int tb = 0; tb < kGwTB; ++tb) {
            float xv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) xv[e] = gl + e < nk ? xsum[(tb * 32 + j) * kSumStride + gl + e] : 0.f;
            bf16x8 at[3];
            split3(xv, at);
#pragma unroll
            for (int pa = 0; pa < 3; ++pa)
#pragma unroll
                for (int pb = 0; pb < 3 - pa; ++pb)
                    acc[tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(at[pa], bt[pb], acc[tb], 0, 0, 0);
        }
    }
    // stores: tile tb, lane value v = token tb * 32 + 8 (v / 4) + 4 h + v % 4, row j of the wave's 32
    if constexpr (sizeof(TY) == 2) {
        if (p.vec_store) {  // BF16 through LDS (every wave is past its K loop and has drained its DMA: the barrier)
            constexpr int kRowB = 32 * 2, kChunksRow = 4, kWaveB = kGwBM * kRowB;  // 8 KB a wave
            static_assert(2 * kWaveB <= kStageBytes, "two waves' staged outputs fit a stage array");
            asm volatile("s_barrier" ::: "memory");
            unsigned char *stg = xs_at(wave >> 1) + (wave & 1) * kWaveB;
#pragma unroll
            for (int tb = 0; tb < kGwTB; ++tb)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = tb * 32 + 8 * (v / 4) + 4 * h + v % 4;
                    *reinterpret_cast<uint16_t *>(stg + r * kRowB + j * 2) = (uint16_t)f32_to_bf16(acc[tb][v]);
                }
            const int64_t fbase = r0 + wave * 32;
            TY *hy = static_cast<TY *>(p.y);
#pragma unroll
            for (int i = 0; i < kGwBM * kChunksRow / 64; ++i) {
                const int c = lane + 64 * i, r = c / kChunksRow, cc = c % kChunksRow;
                const int64_t f = fbase + cc * 8;  // N % 8 == 0: a chunk is wholly in or out
                const uint4 val = *reinterpret_cast<const uint4 *>(stg + r * kRowB + cc * 16);
                if (r < T && f < N) *reinterpret_cast<uint4 *>(hy + (t0 + r) * N + f) = val;
            }
            return;
        }
    }
    if (feat >= N) return;
#pragma unroll
    for (int tb = 0; tb < kGwTB; ++tb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = tb * 32 + 8 * (v / 4) + 4 * h + v % 4;
            if (r < T) store_act(static_cast<TY *>(p.y), (t0 + r) * N + feat, acc[tb][v]);
        }
}

template <int MODE, typename TY, int BITS = 4>
hipError_t go(const Params &p, dim3 grid, hipStream_t stream) {
    hipLaunchKernelGGL((gg_kernel<MODE, TY, BITS>), grid, dim3(kThreads), 0, stream, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_dense(const void *x, const sx_qview *w, void *y, int64_t M, int out_act, hipStream_t stream) {
    Params p{};
    p.x = static_cast<const uint16_t *>(x), p.q = static_cast<const uint8_t *>(w->q);
    p.scale = static_cast<const uint16_t *>(w->scale), p.minv = static_cast<const uint16_t *>(w->minv);
    p.y = y, p.ws = nullptr, p.A = 1, p.N = w->N, p.K = w->K, p.E = 1, p.dense_M = M;
    p.vec_store = out_act == SX_ACT_BF16 && p.N % 8 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0;
    p.nrb = (int)((p.N + kWaves * 64 - 1) / (kWaves * 64));
    const int64_t tiles = (M + kBM - 1) / kBM;
    if (M <= kDenseSplitMaxTokens) {  // K split over each block's waves
        const dim3 gs_grid((unsigned)(tiles * ((p.N + 63) / 64)));
        auto gs = [&](auto tag, auto bits) {
            hipLaunchKernelGGL((gs_kernel<decltype(tag), decltype(bits)::value>), gs_grid, dim3(kThreads), 0, stream, p);
            return hipGetLastError();
        };
        if (w->G == 64)
            return out_act == SX_ACT_F32 ? gs(float{}, std::integral_constant<int, 8>{})
                                         : gs(uint16_t{}, std::integral_constant<int, 8>{});
        return out_act == SX_ACT_F32 ? gs(float{}, std::integral_constant<int, 4>{})
                                     : gs(uint16_t{}, std::integral_constant<int, 4>{});
    }
    const int64_t wt = (M + kGwBM - 1) / kGwBM, nrb_w = (p.N + kGwRows - 1) / kGwRows;
    if (wt * nrb_w >= device_cus()) {  // 128 tokens a wave where that grid fills the chip
        p.nrb = (int)nrb_w;
        const dim3 gw_grid((unsigned)((wt + 7) / 8 * 8 * nrb_w));
        auto gw = [&](auto tag, auto bits) {
            hipLaunchKernelGGL((gw_kernel<decltype(tag), decltype(bits)::value>), gw_grid, dim3(kGwThreads), 0, stream,
                               p);
            return hipGetLastError();
        };
        if (w->G == 64)
            return out_act == SX_ACT_F32 ? gw(float{}, std::integral_constant<int, 8>{})
                                         : gw(uint16_t{}, std::integral_constant<int, 8>{});
        return out_act == SX_ACT_F32 ? gw(float{}, std::integral_constant<int, 4>{})
                                     : gw(uint16_t{}, std::integral_constant<int, 4>{});
    }
    const dim3 grid((unsigned)((tiles + 7) / 8 * 8 * p.nrb));
    if (w->G == 64)  // q8
        return out_act == SX_ACT_F32 ? go<qmm::GATHER, float, 8>(p, grid, stream)
                                     : go<qmm::GATHER, uint16_t, 8>(p, grid, stream);
    return out_act == SX_ACT_F32 ? go<qmm::GATHER, float>(p, grid, stream) : go<qmm::GATHER, uint16_t>(p, grid, stream);
}

bool eligible(int bits, int64_t G, int64_t K, int act) {
    return bits == 4 && G == 128 && K % (4 * kSpan) == 0 && K <= kSpan * kMaxGroups && act == SX_ACT_BF16;
}

bool eligible_dense(int bits, int64_t G, int64_t K, int act) {
    if (bits == 8) return G == 64 && K % (4 * Lay<8>::kSpan) == 0 && K <= 4096 && act == SX_ACT_BF16;
    return eligible(bits, G, K, act);
}

hipError_t launch(int mode, const void *x, const sx_qview *w, void *y, const int32_t *ws, int64_t M, int64_t A,
                  int64_t E, int out_act, hipStream_t stream) {
    Params p{};
    p.x = static_cast<const uint16_t *>(x), p.q = static_cast<const uint8_t *>(w->q);
    p.scale = static_cast<const uint16_t *>(w->scale), p.minv = static_cast<const uint16_t *>(w->minv);
    p.y = y, p.ws = ws, p.A = A, p.N = w->N / E, p.K = w->K, p.E = E;
    const int64_t S = M * A;
    const int64_t wtiles = S / kBM + E + 2;  // WTmax: an upper bound of the 64-slot tiles; the rest exit at once
    const int64_t out_rows = mode == qmm::SWIGLU ? p.N / 2 : p.N;
    p.vec_store = out_act == SX_ACT_BF16 && out_rows % 8 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0;
    const int64_t per_block = mode == qmm::SWIGLU ? kWaves * 32 : kWaves * 64;
    p.nrb = (int)((out_rows + per_block - 1) / per_block);
    const dim3 grid((unsigned)((wtiles + 7) / 8 * 8 * p.nrb));
    hipError_t e;
    switch (mode) {
    case qmm::SWIGLU:
        e = out_act == SX_ACT_F32 ? go<qmm::SWIGLU, float>(p, grid, stream) : go<qmm::SWIGLU, uint16_t>(p, grid, stream);
        break;
    case qmm::GATHER:
        e = out_act == SX_ACT_F32 ? go<qmm::GATHER, float>(p, grid, stream) : go<qmm::GATHER, uint16_t>(p, grid, stream);
        break;
    default:
        if (p.K <= kPdMaxSteps * kSpan && (p.K / kSpan == 8 || p.K / kSpan == 4)) {  // the down projection
            hipLaunchKernelGGL(gg_down_kernel, dim3((unsigned)(wtiles * kPdSplits)), dim3(kPdThreads), 0, stream, p);
            e = hipGetLastError();
        } else {
            e = go<qmm::COMBINE, float>(p, grid, stream);
        }
    }
    return e;
}

}  // namespace sx::gg
