// Shared device helpers and host-side argument/error plumbing of libqwen_state (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qwen_state.h"

namespace qs {

// ------------------------------------------------------------------------------------------- device helpers

// bf16 bit pattern -> fp32 (exact)
__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }
// low / high bf16 of a packed pair -> fp32
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 with round-to-nearest-even (torch's .bfloat16()); NaN stays a quiet NaN
__device__ __forceinline__ uint32_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) { return f2bf(lo) | (f2bf(hi) << 16); }

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// sum / max over the 64 lanes of a wavefront (butterfly: every lane ends with the result)
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// Workgroup i is dispatched to XCD i % 8. Map hardware ids so that consecutive logical ids land on one XCD
// (and share its L2): logical = (hw % 8) * (n / 8) + hw / 8. Identity when n is not a multiple of 8.
__device__ __forceinline__ int xcd_logical(int hw, int n) {
    if (n & 7) return hw;
    return (hw & 7) * (n >> 3) + (hw >> 3);
}

}  // namespace qs

// ------------------------------------------------------------------------------------------- host plumbing

namespace qs {
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
int launch_status(const char *what);
}  // namespace qs

#define QS_REQUIRE(cond, ...)          \
    do {                               \
        if (!(cond)) {                 \
            qs::set_error(__VA_ARGS__); \
            return QS_EINVAL;          \
        }                              \
    } while (0)

#define QS_STREAM(s) reinterpret_cast<hipStream_t>(s)
