// Weight-format work on the device: the MTP draft head's Q4 copy of the Q8 LM head (formats/q4_from_q8.hpp).
//
// The reference makes the copy on the host at load (runtime/qwen4exp.cpp:192-238: read the Q8 rows back, requantize
// with threads, upload); here the resident Q8 rows are requantized where they lie. A thread owns one Q4 group of one
// row: it dequantizes the group's Q8 codes exactly as formats/q8.cpp:117-127 does (code * s, then + m, each rounded),
// finds the group's range and requantizes as formats/q4.cpp:44-86 does (s = bf16((hi - lo) / 15), m = bf16(lo),
// code = clamp(round-half-even((w - m) / s), 0, 15)), every operation the IEEE-rounded one the host computes, so
// the bytes equal the reference's. HBM-bound: K bytes read and K / 2 + 4 K / G4 written a row.
#include "common.hpp"

namespace sx {
namespace {

__device__ __forceinline__ uint32_t word_of(const uint4 &v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

template <int G4>
__global__ void __launch_bounds__(256) q4_from_q8_kernel(const uint8_t *q8, const uint16_t *s8, const uint16_t *m8,
                                                         int64_t N, int64_t K, int64_t G8, uint8_t *q4, uint16_t *s4,
                                                         uint16_t *m4, uint32_t *err) {
    const int64_t groups = K / G4, idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= N * groups) return;
    const int64_t n = idx / groups, g = idx - n * groups, k0 = g * G4;
    constexpr int kChunks = G4 / 16;
    uint4 raw[kChunks];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) raw[c] = *reinterpret_cast<const uint4 *>(q8 + n * K + k0 + 16 * c);
    // the Q8 groups this Q4 group spans: one when G8 >= G4, else G4 / G8 (<= 4) of G8 codes each
    constexpr int kSub = G4 / 32;  // the most Q8 groups a Q4 group spans (G8 >= 32)
    const int lg8 = __builtin_ctz((unsigned)G8);
    const int64_t g0 = n * (K >> lg8) + (k0 >> lg8);
    float s_[kSub], m_[kSub];
#pragma unroll
    for (int j = 0; j < kSub; ++j) {
        const int64_t gi = g0 + min(j, (int)((G4 - 1) >> lg8));
        s_[j] = bf16_to_f32(s8[gi]), m_[j] = bf16_to_f32(m8[gi]);
    }
    float w[G4];
#pragma unroll
    for (int i = 0; i < G4; ++i) {
        const uint32_t word = word_of(raw[i / 16], (i % 16) / 4);
        const uint32_t code = (word >> (8 * (i % 4))) & 0xFFu;
        const int j = min(i >> lg8, kSub - 1);  // G8 >= G4: always 0
        float s = s_[0], m = m_[0];
#pragma unroll
        for (int t = 1; t < kSub; ++t) s = j == t ? s_[t] : s, m = j == t ? m_[t] : m;
        w[i] = __fadd_rn(__fmul_rn((float)code, s), m);
    }
    float lo = w[0], hi = w[0];
    bool finite = true;
#pragma unroll
    for (int i = 0; i < G4; ++i) {
        finite &= isfinite(w[i]);
        lo = fminf(lo, w[i]);
        hi = fmaxf(hi, w[i]);
    }
    if (!finite) flag_error(err, (uint32_t)n, (uint32_t)k0);  // the reference throws; the row's group gets zeros
    const uint32_t sb = finite ? f32_to_bf16(__fdiv_rn(__fsub_rn(hi, lo), 15.0f)) : 0u;
    const uint32_t mb = finite ? f32_to_bf16(lo) : 0u;
    const float s = bf16_to_f32(sb), m = bf16_to_f32(mb);
    uint32_t packed[G4 / 8];
#pragma unroll
    for (int j = 0; j < G4 / 8; ++j) packed[j] = 0u;
#pragma unroll
    for (int i = 0; i < G4; ++i) {
        uint32_t code = 0u;
        if (s > 0.0f) code = (uint32_t)fminf(fmaxf(rintf(__fdiv_rn(__fsub_rn(w[i], m), s)), 0.0f), 15.0f);
        packed[i / 8] |= code << (4 * (i % 8));  // low nibble = even k (formats/q4.hpp:4)
    }
    uint8_t *dst = q4 + n * (K / 2) + k0 / 2;
#pragma unroll
    for (int c = 0; c < G4 / 32; ++c)
        *reinterpret_cast<uint4 *>(dst + 16 * c) =
            uint4{packed[4 * c], packed[4 * c + 1], packed[4 * c + 2], packed[4 * c + 3]};
    s4[n * groups + g] = (uint16_t)sb;
    m4[n * groups + g] = (uint16_t)mb;
}

}  // namespace
}  // namespace sx

using namespace sx;

extern "C" {

int sx_quantize_q4_from_q8(const sx_qview *src, int64_t G, uint8_t *q, uint16_t *scale, uint16_t *minv,
                           uint32_t *err, sx_stream stream) {
    SX_CHECK(src != nullptr && src->q && src->scale && src->minv && q && scale && minv && err, "null pointer");
    SX_CHECK(src->G == 32 || src->G == 64 || src->G == 128, "Q8 group size ", src->G, ", expected 32, 64 or 128");
    SX_CHECK(G == 32 || G == 64 || G == 128, "Q4 group size ", G, ", expected 32, 64 or 128");
    SX_CHECK(src->N >= 1 && src->K >= G && src->K % G == 0 && src->K % src->G == 0, "[", src->N, ", ", src->K,
             "]: K must be a multiple of the Q8 group ", src->G, " and of the Q4 group ", G);
    SX_CHECK(aligned(src->q, 16) && aligned(q, 16) && src->K % 32 == 0, "code arrays must be 16-byte aligned");
    const int64_t threads = src->N * (src->K / G), blocks = (threads + 255) / 256;
    SX_CHECK(blocks <= 0x7fffffff, "too many rows: ", src->N);
    auto go = [&](auto g4) {
        q4_from_q8_kernel<decltype(g4)::value><<<(unsigned)blocks, 256, 0, stream_of(stream)>>>(
            src->q, src->scale, src->minv, src->N, src->K, src->G, q, scale, minv, err);
    };
    if (G == 32) go(std::integral_constant<int, 32>{});
    else if (G == 64) go(std::integral_constant<int, 64>{});
    else go(std::integral_constant<int, 128>{});
    SX_LAUNCHED("quantize_q4_from_q8 N=", src->N, " K=", src->K, " G=", G);
    return SX_OK;
}

}  // extern "C"
