// Hardware ceilings the path is judged against, measured on the part itself: a streaming read of a large buffer (what
// HBM delivers to plain 16-byte vector loads with no cache reuse) and a loop of independent BF16 MFMAs (what the
// matrix cores deliver with no memory traffic). Measurement helpers only; nothing on the verify path calls them.
#include "common.hpp"

namespace sx {
namespace {

typedef __bf16 pr_bf16x8 __attribute__((ext_vector_type(8)));
typedef float pr_f32x16 __attribute__((ext_vector_type(16)));

constexpr int kStreamThreads = 512, kStreamUnroll = 8;

// Each thread reads kStreamUnroll 16-byte vectors a trip, all issued before any is used, striding over the buffer by
// the whole grid; the XOR of everything read goes to sink only if it equals a value it practically never takes, so
// the loads are live but the kernel stores nothing.
__global__ void __launch_bounds__(kStreamThreads) stream_read_kernel(const uint4 *p, int64_t n16, uint32_t *sink) {
    const int64_t stride = (int64_t)gridDim.x * kStreamThreads;
    int64_t i = (int64_t)blockIdx.x * kStreamThreads + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (kStreamUnroll - 1) * stride < n16; i += kStreamUnroll * stride) {
        uint4 v[kStreamUnroll];
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) v[u] = p[i + u * stride];
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

constexpr int kMfmaChains = 4;  // independent accumulators a wave: the matrix pipe never waits for a result

// iters x kMfmaChains v_mfma_f32_32x32x16_bf16 a wave (32 x 32 x 16 x 2 = 32,768 flops each); the operands are fixed
// registers, the sums go to sink only under a condition the data never meets.
__global__ void __launch_bounds__(256) mfma_loop_kernel(int iters, float *sink) {
    pr_bf16x8 a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        a[j] = (__bf16)(float)((threadIdx.x + j) & 7);
        b[j] = (__bf16)(float)((threadIdx.x * 3 + j) & 7);
    }
    pr_f32x16 acc[kMfmaChains];
#pragma unroll
    for (int c = 0; c < kMfmaChains; ++c)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[c][j] = 0.f;
    for (int it = 0; it < iters; ++it)
#pragma unroll
        for (int c = 0; c < kMfmaChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < kMfmaChains; ++c)
#pragma unroll
        for (int j = 0; j < 16; ++j) s += acc[c][j];
    if (s == -1.f) sink[0] = s;
}

}  // namespace
}  // namespace sx

using namespace sx;

extern "C" {

int sx_probe_stream_read(const void *buf, uint64_t bytes, int blocks, uint32_t *sink, sx_stream stream) {
    SX_CHECK(buf != nullptr && sink != nullptr, "null pointer");
    SX_CHECK(aligned(buf, 16) && bytes % 16 == 0 && bytes > 0, "buffer must be 16-byte aligned and a multiple of 16 bytes");
    SX_CHECK(blocks >= 1 && blocks <= 65536, "blocks = ", blocks);
    stream_read_kernel<<<blocks, kStreamThreads, 0, stream_of(stream)>>>(static_cast<const uint4 *>(buf),
                                                                         (int64_t)(bytes / 16), sink);
    SX_LAUNCHED("stream_read bytes=", bytes);
    return SX_OK;
}

int sx_probe_mfma(int blocks, int iters, float *sink, double *flops, sx_stream stream) {
    SX_CHECK(sink != nullptr, "null pointer");
    SX_CHECK(blocks >= 1 && blocks <= 65536 && iters >= 1, "blocks = ", blocks, ", iters = ", iters);
    if (flops) *flops = (double)blocks * 4 * iters * kMfmaChains * 32.0 * 32 * 16 * 2;
    mfma_loop_kernel<<<blocks, 256, 0, stream_of(stream)>>>(iters, sink);
    SX_LAUNCHED("mfma_loop blocks=", blocks);
    return SX_OK;
}

}  // extern "C"
