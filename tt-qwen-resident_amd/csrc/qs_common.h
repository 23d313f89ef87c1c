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

// SiLU as torch states it, x / (1 + e^-x): the library exponential (within 1 ulp), then the quotient from the
// hardware reciprocal with one Newton correction (q + (x - q d) / d), which lands within about half an ulp
// of the correctly rounded quotient for a fraction of an IEEE divide's instructions. The fp32 result is
// within about an ulp of torch's CPU value, so its bf16 rounding agrees except where the fp32 value sits
// within an ulp or two of a bf16 rounding boundary. When e^-x overflows (x < -88.7) the quotient is x / inf,
// a signed zero, as in torch.
__device__ __forceinline__ float silu(float x) {
    const float d = 1.0f + expf(-x);
    const float r = __builtin_amdgcn_rcpf(d);
    const float q = x * r;
    return __builtin_isinf(d) ? x * 0.0f : fmaf(fmaf(-q, d, x), r, q);
}

// v op (v of lane ^ 16) and v op (v of lane ^ 32) on the VALU (gfx950 v_permlane16_swap / v_permlane32_swap,
// no LDS round trip). With both operands v, the swap returns, in every lane, the values of the lower and
// the upper lane of its pair (row pair 2r, 2r + 1 of 16 lanes, or the two 32-lane halves), so both lanes
// of a pair compute the same lower op upper.
__device__ __forceinline__ float xor16_sum(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// sum / max over the 64 lanes of a wavefront (butterfly: every lane ends with the result)
__device__ __forceinline__ float wave_sum(float v) {
    v = xor32_sum(v);
    v = xor16_sum(v);
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    v = xor32_max(v);
    v = xor16_max(v);
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// Cross-lane moves inside 16-lane rows with DPP (no LDS round trip). CTRL: 0xB1 quad_perm [1,0,3,2]
// (xor 1), 0x4E quad_perm [2,3,0,1] (xor 2), 0x104 row_shl:4 (lane i reads lane i + 4; lanes 12..15 of
// a row read 0), 0x124 / 0x128 row_ror:4 / row_ror:8 (0x128 is xor 8). bound_ctrl set and no old value,
// so the compiler folds the move into the consuming add / max as its DPP source.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ float lane_val(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Wave-wide max / sum with DPP inside each 16-lane row and readlane across the 4 rows. Every lane of a row
// holds bit-identical partials (the pairwise combines are commutative), so the result is wave-uniform and
// deterministic.
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x124>(v));
    v = fmaxf(v, dpp<0x128>(v));
    return fmaxf(fmaxf(lane_val(v, 0), lane_val(v, 16)), fmaxf(lane_val(v, 32), lane_val(v, 48)));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x124>(v);
    v += dpp<0x128>(v);
    return (lane_val(v, 0) + lane_val(v, 16)) + (lane_val(v, 32) + lane_val(v, 48));
}

// Wave-wide max, wave-uniform result: DPP inside each 16-lane row, then row_bcast:15 (into rows 1, 3) and
// row_bcast:31 (into rows 2, 3) fold the rows so lane 63 holds the maximum; one readlane broadcasts it.
__device__ __forceinline__ float wave_max_bcast(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x124>(v));
    v = fmaxf(v, dpp<0x128>(v));
    const int vi = __builtin_bit_cast(int, v);
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(vi, vi, 0x142, 0xA, 0xF, false)));
    const int vj = __builtin_bit_cast(int, v);
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(vj, vj, 0x143, 0xC, 0xF, false)));
    return lane_val(v, 63);
}

// Two fp32 to packed bf16 (lo = a, hi = b), round-to-nearest-even (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
    typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
    bf16x2_v v;
    v[0] = (__bf16)a;
    v[1] = (__bf16)b;
    return __builtin_bit_cast(uint32_t, v);
}

// Waits until every vector memory operation of the wave has completed. Through the builtin rather than
// inline assembly: the compiler's own wait placement then knows nothing is in flight afterwards (after an
// inline "s_waitcnt" it still counts earlier stores as pending, and at the next use of a loaded value waits
// for everything). The empty asm statements keep memory accesses from moving across it.
__device__ __forceinline__ void wait_vmem() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt and lgkmcnt at their maxima (gfx9 encoding)
    asm volatile("" ::: "memory");
}

// A pointer made wave-uniform (its value in the first active lane), for buffer descriptors built from a
// per-wave base.
template <class T>
__device__ __forceinline__ T *uniform_ptr(T *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<T *>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Cache-policy bits of the buffer load / store builtins on gfx950: nt = streaming (the line is not kept),
// sc1 = coherent at agent scope (stores write through the XCD's L2, loads miss in it). Data that another
// workgroup of the same launch reads back is stored and loaded with sc1, so it needs no L2 writeback.
constexpr int CP_NT = 2, CP_SC1 = 16;

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
