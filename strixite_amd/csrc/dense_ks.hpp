// Dense dequantizing GEMV at decode / verify width with K split over a block's waves (dense_ks.hip).
#pragma once
#include "common.hpp"
#include "pick.hpp"

namespace sx::dks {

constexpr size_t kLdsMax = 140 * 1024;  // activation planes + span sums; the rest of the 160 KB holds the partials

struct Params {
    const void *x;  // activations [M, K] (BF16 or FP32)
    const uint8_t *q;
    const uint16_t *scale, *minv;
    void *y;        // [M, N] (BF16 or FP32)
    int M;
    int Q;          // K slices a tile (set by launch)
    int strided;    // a block's tiles: every G-th one (set by launch for 16 or more a block), else an adjacent run
    int64_t N, K;
    pick::Args pick;  // pick.ws set: the MTP pick of row 0 of y (FP32 y, M = 1) fused after the GEMV, gridDim <= 256
};

size_t lds_bytes(int act, int64_t M, int64_t K, int bits, int64_t G);
// q4 G = 128 or 64 or q8 G = 64, K of 4 .. 64 spans (a power of two), M <= 16, act / out_act as linear's (BF16 -> BF16 or
// FP32, FP32 -> FP32) and the activation planes within kLdsMax; any number of 16-row tiles
bool eligible(int bits, int64_t G, int64_t N, int64_t K, int64_t M, int act, int out_act, int cus);
hipError_t launch(int bits, int64_t G, int act, int out_act, const Params &p, int cus, hipStream_t stream);

}  // namespace sx::dks
