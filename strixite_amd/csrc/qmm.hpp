// Skinny dequantizing GEMM on the matrix cores (gfx950 MFMA), for verify width: up to 16 activation rows per weight
// pass, every weight byte read once per pass.
//
// The weight tile is 16 rows x one 64-byte "span" per row (128 q4 codes or 64 q8 codes); a wave64 loads it with one
// coalesced 16-byte load per lane (lane = row l%16, quarter l/16 of the span). The codes go to the MFMA exactly:
//   q4: a dword's 8 nibbles become 4 BF16 pairs (code | 0x4300 = 128 + code) with 7 bit operations, no conversion;
//   q8: bytes -> FP32 (v_cvt_f32_ubyteN) -> BF16 by dropping the low half (exact for 0..255).
// v_mfma_f32_16x16x32_bf16 then gives D[token][row] = sum_k x[token][k] * (off + code[row][k]) exactly in FP32, and a
// span lies inside one quantization group (q4 G = 128, q8 G = 64 or 128), so
//   sum_k x * (code * s + m) = s * D + (m - off * s) * sum_k x
// (off = 128 for q4, 0 for q8) - the reference's per-chunk s * sum(x*q) + m * sum(x) (kernels/linear_q4.hip:88-94) on
// the matrix cores. The x rows sit in LDS as BF16 (FP32 x: three BF16 planes hi + mid + lo, exact), in the order the
// code unpacking produces, with their per-span sums. MFMA k order is free as long as A and B agree.
// Smaller groups (q4 G = 32 / 64, q8 G = 32: 2 or 4 groups a span) stay on the MFMA: the quarter-spans of different
// groups feed different A rows (a pass then holds 16 / groups-per-span activation rows), so D keeps each group's dot
// apart, and the lanes holding one token's groups add up in the epilogue.
#pragma once

#include "common.hpp"

namespace sx::qmm {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTile = 16;     // weight rows per MFMA tile = activation rows per pass
constexpr int kSpanBytes = 64;

enum Mode {
    DENSE = 0,         // y[m, n] = x[m] . W[n]                          (linear_q4 / linear_q8)
    GATHER = 1,        // grouped: y[slot, n] = x[slot / A] . W[e, n]     (experts_gather_grouped)
    SWIGLU = 2,        // grouped: h[slot, j] = swiglu(gate j, up j)     (gather_grouped + swiglu)
    COMBINE = 3,       // grouped: partial[slot, n] = h[slot] . W[e, n]  (experts_combine_grouped, before the reduce)
    SLOT_GATHER = 4,   // per slot: y[slot, n] = x[slot / A] . W[ids[slot], n]   (experts_gather)
    SLOT_SWIGLU = 5,   // per slot, SwiGLU epilogue                               (experts_gather_swiglu)
    SLOT_COMBINE = 6,  // per token: y[m, n] = sum_a coef * h[m, a] . W[ids[m, a], n]  (experts_combine)
};

struct Params {
    const void *x;        // activations (TX)
    const uint8_t *q;     // codes
    const uint16_t *scale, *minv;
    void *y;              // output (TY), or FP32 partials for COMBINE
    const int32_t *ws;    // grouped modes: the route workspace
    const int32_t *ids;   // per-slot modes
    const float *coef;    // SLOT_COMBINE
    uint32_t *err;        // per-slot modes
    int64_t M;            // DENSE: rows of x; grouped / slot: tokens
    int64_t A;            // slots per token
    int64_t E;            // experts
    int64_t N;            // output rows per expert (DENSE: all rows); SWIGLU: 2I (gate | up)
    int64_t K;
    int G;
    int nchunks;          // row chunks per unit
    int tiles_per_chunk;  // 16-row tiles (SWIGLU: tile pairs) per chunk
    int max_rows;         // LDS rows staged per unit (tokens in a tile; SLOT_COMBINE: A)
};

// Dynamic LDS bytes for a launch: `rows` staged x rows as nsplit BF16 planes; their sums over each run of min(G, span)
// codes, padded to whole spans ([blocks][runs][16] FP32; blocks = A for SLOT_COMBINE, else 1); a 2 KB zero block.
inline size_t lds_bytes(int bits, int nsplit, int64_t K, int64_t G, int rows, int blocks) {
    const int64_t span_codes = bits == 4 ? 128 : 64;
    const int64_t run = G < span_codes ? G : span_codes;
    const int64_t runs = (K + span_codes - 1) / span_codes * (span_codes / run);
    return (size_t)nsplit * rows * (K + 8) * 2 + (size_t)blocks * runs * 16 * 4 + 2048;
}

// Launches one mode; bits 4 / 8, act of x and y, nsplit 1 (BF16 x) or 3 (F32 x). grid.x = units * nchunks,
// grid.y = DENSE m-blocks. Returns hipSuccess or the launch error.
hipError_t launch(int mode, int bits, int act_x, int act_y, const Params &p, dim3 grid, hipStream_t stream);

// Activation rows per weight pass: 16 / (groups per span).
inline int rows_per_pass(int bits, int64_t G) {
    const int64_t span_codes = bits == 4 ? 128 : 64;
    return G >= span_codes ? 16 : (int)(16 * G / span_codes);
}

}  // namespace sx::qmm
