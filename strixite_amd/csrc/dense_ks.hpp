// Dense dequantizing GEMV at decode / verify width with K split over a block's waves (dense_ks.hip).
#pragma once
#include "common.hpp"

namespace sx::dks {

constexpr size_t kLdsMax = 140 * 1024;  // activation planes + span sums; the rest of the 160 KB holds the partials

struct Params {
    const void *x;  // activations [M, K] (BF16 or FP32)
    const uint8_t *q;
    const uint16_t *scale, *minv;
    void *y;        // [M, N] (BF16 or FP32)
    int M;
    int Q;          // K slices a tile (set by launch)
    int64_t N, K;
};

size_t lds_bytes(int act, int64_t M, int64_t K, int bits, int64_t G);
// q4 G = 128 or 64 or q8 G = 64, K of 4 .. 64 spans (a power of two), M <= 16, act / out_act as linear's (BF16 -> BF16 or
// FP32, FP32 -> FP32), the activation planes within kLdsMax, and no more 16-row tiles than blocks (cus): with more,
// qmm's dense mode already fills the chip and measured as fast or faster (configs 2 and 5: 11.7 vs 12.6 us, 81 vs
// 84 us; config 1, 256 tiles: 14.4 vs 12.1 us)
bool eligible(int bits, int64_t G, int64_t N, int64_t K, int64_t M, int act, int out_act, int cus);
hipError_t launch(int bits, int64_t G, int act, int out_act, const Params &p, int cus, hipStream_t stream);

}  // namespace sx::dks
