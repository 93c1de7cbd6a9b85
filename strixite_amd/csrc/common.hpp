// Shared host/device helpers for the gfx950 verify-path library: BF16 bit conversions, the C-ABI error channel
// (status code + thread-local message), precondition checks and launch checks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <sstream>
#include <string>

#include "strixite_amd.h"

namespace sx {

// ---------------- device helpers ----------------

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// FP32 -> BF16 bits, round to nearest even, NaN kept quiet: the rounding every store of the reference's kernels
// uses (kernels/linear_q4.hip:22-27).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u) return (u >> 16) | ((u & 0x007fffffu) ? 0x0040u : 0u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float as_bf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ void store_act(float *p, int64_t i, float v) { p[i] = v; }
__device__ __forceinline__ void store_act(uint16_t *p, int64_t i, float v) { p[i] = (uint16_t)f32_to_bf16(v); }
__device__ __forceinline__ float load_act(const float *p, int64_t i) { return p[i]; }
__device__ __forceinline__ float load_act(const uint16_t *p, int64_t i) { return bf16_to_f32(p[i]); }
// The value a store in T then a reload gives back (BF16: rounded once; F32: itself).
__device__ __forceinline__ float as_stored(float v, const float *) { return v; }
__device__ __forceinline__ float as_stored(float v, const uint16_t *) { return as_bf16(v); }

// A block barrier ordering LDS accesses only: __syncthreads() would also wait for every global load in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float qnan() { return __uint_as_float(0x7fc00000u); }

// SiLU in the reference's form v / (1 + exp(-v)) (kernels/swiglu.hip:19).
__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

// Records the first data error into a 3-word device error slot (first writer wins): err[0] = 1, err[1..2] = what.
__device__ __forceinline__ void flag_error(uint32_t *err, uint32_t a, uint32_t b) {
    if (atomicCAS(err, 0u, 1u) == 0u) {
        err[1] = a;
        err[2] = b;
    }
}

// ---------------- host error channel ----------------

void set_error(const std::string &msg);

template <typename... Args>
std::string cat(Args &&...args) {
    std::ostringstream os;
    (os << ... << args);
    return os.str();
}

struct Failure {
    int code;
};

}  // namespace sx

// Precondition check in a C-ABI entry point: on failure, records "fn: message" and returns SX_EINVAL.
#define SX_CHECK(cond, ...)                                                                          \
    do {                                                                                             \
        if (!(cond)) {                                                                               \
            ::sx::set_error(::sx::cat(__func__, ": check `", #cond, "` failed: ", __VA_ARGS__));     \
            return SX_EINVAL;                                                                        \
        }                                                                                            \
    } while (0)

// A HIP runtime call in a C-ABI entry point: on failure records the HIP error and returns SX_EHIP.
#define SX_HIP(expr, ...)                                                                            \
    do {                                                                                             \
        hipError_t sx_e_ = (expr);                                                                   \
        if (sx_e_ != hipSuccess) {                                                                   \
            ::sx::set_error(::sx::cat(__func__, ": ", #expr, " -> ", hipGetErrorName(sx_e_), " (",   \
                                      hipGetErrorString(sx_e_), ") ", __VA_ARGS__));                 \
            return SX_EHIP;                                                                          \
        }                                                                                            \
    } while (0)

// After a launch: a bad launch configuration is reported here, not at the next synchronisation.
#define SX_LAUNCHED(...) SX_HIP(hipGetLastError(), "kernel launch: ", __VA_ARGS__)

namespace sx {

inline hipStream_t stream_of(sx_stream s) { return reinterpret_cast<hipStream_t>(s); }

inline bool apart(const void *a, int64_t an, const void *b, int64_t bn) {
    const auto ab = reinterpret_cast<uintptr_t>(a), bb = reinterpret_cast<uintptr_t>(b);
    return ab + (uintptr_t)an <= bb || bb + (uintptr_t)bn <= ab;
}

inline bool aligned(const void *p, uintptr_t n) { return reinterpret_cast<uintptr_t>(p) % n == 0; }

inline int act_bytes(int act) { return act == SX_ACT_F32 ? 4 : 2; }

// Number of compute units of the current device (cached per device).
int device_cus();

// The route workspace (kernels/moe_grouped.hip:63-81) for S = M * A slots over E experts, in int32 words.
struct Layout {
    int64_t S, E, Tmax, WTmax;
    int64_t ints() const { return 4 + (E + 2) + S + 2 * Tmax + 2 * WTmax; }
};
Layout layout_of(int64_t M, int64_t A, int64_t E);

// y[m, n] = sum_a coef[m, a] * partial[m * A + a, n], a in order, rounded once; NaN rows for tokens with a bad id
// (the grouped combine's second step, route.hip).
int combine_reduce(const float *partial, const int32_t *ids, const float *coef, int64_t M, int64_t A, int64_t E,
                   int64_t N, void *y, int act, hipStream_t stream);

}  // namespace sx
