// Weight-streaming projections and the MLP half of a decoder layer on gfx950 (the streamer kernels' role:
// kernels/streamer_compute.cpp:371-473, the MLP half of tests/bench_resident_mlp.py:98-105).
//
// Weights are OCP microscaling blocks: 32 consecutive values along K share one E8M0 scale 2^(e - 127);
// MXFP4 stores E2M1 values (gate and up projections; the reference streams these in 4-bit block floating
// point); MXINT8 stores two's-complement int8 values times 2^-6, a sign and 7 magnitude bits under the shared
// scale, the precision of the reference's 8-bit block floating point (down projection and the 8-bit
// projections: bfloat8_b, sign + 7-bit mantissa per value, model.py:53-58); MXFP8 stores E4M3 values (3
// mantissa bits, kept as an option). A weight
// W [K, N] (y = h W) is laid out once, by qs_mx_quantize, in MFMA fragment order: for each 16-column tile t
// and K group q (128 values of K for MXFP4, 64 for the 8-bit formats) one block of 1024 value bytes and the
// group's scales, lane l = 16 g + r (r the column in the tile) owning 16 bytes: the values of K steps
// KG q + 32 s + 8 g .. + 7 for each 32-value step s of the group (4 steps of 4 bytes for MXFP4, low nibble
// first; 2 steps of 8 bytes for MXFP8 / MXINT8), then column r's scales (one per step) at 1024 + SCALES r. A
// wave loads its part of a block as one contiguous kilobyte plus a 4- or 2-byte scale word and converts it to
// bf16 exactly: with the hardware's scaled conversions (v_cvt_scalef32_pk_bf16_fp4 / _fp8, the scale folded
// in) or, for MXINT8, on the VALU (each int8 as an integer, one signed-byte conversion, exact in bf16; the
// scale, a power of two, multiplies the 32-value step's product instead, which is exact). It multiplies on
// v_mfma_f32_16x16x32_bf16 with the activations (bf16, up to 16 rows) as the A operand.
// The kernels stream weights at the HBM rate; the conversions and MFMAs hide under the loads.
//
// MLP half (qs_mlp_decode; down in MXINT8 or MXFP8): h = bf16(x rsqrt(mean(x^2) + eps) gamma); z = bf16(silu(h G) (h U)) in one
// launch (gate and up tiles in the same workgroup; for one row the workgroups also form h themselves); the
// down projection split over K (four ways for one row), its last split per tile adding the partials and the
// residual: x_out = x + z D. Two launches per layer for one row; the gate | up grid keeps every CU equally
// loaded (tail_whole).
#include <algorithm>

#include "qs_common.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int FMT_FP4 = 4, FMT_FP8 = 8, FMT_INT8 = 9;
constexpr int TILE_N = 16;
constexpr int MAX_ROWS = 16;  // activation rows per call: the MFMA's M
constexpr int DOWN_SPLIT = 4;

template <int FMT>
struct Mx;
template <>
struct Mx<FMT_FP4> {
    static constexpr int KG = 128;      // K values per block
    static constexpr int STEPS = 4;     // 32-value steps (one scale each) per block
    static constexpr int BYTES = 1088;  // 1024 value bytes + 16 columns x 4 scales
};
template <>
struct Mx<FMT_FP8> {
    static constexpr int KG = 64;
    static constexpr int STEPS = 2;
    static constexpr int BYTES = 1056;
};
template <>
struct Mx<FMT_INT8> : Mx<FMT_FP8> {};  // the same 8-bit layout

__host__ __device__ inline bool fmt_ok(int fmt) { return fmt == FMT_FP4 || fmt == FMT_FP8 || fmt == FMT_INT8; }
__host__ __device__ inline int kg_of(int fmt) { return fmt == FMT_FP4 ? Mx<FMT_FP4>::KG : Mx<FMT_FP8>::KG; }
__host__ __device__ inline size_t mx_bytes(int K, int N, int fmt) {
    return (size_t)(N / TILE_N) * (K / kg_of(fmt)) * (fmt == FMT_FP4 ? Mx<FMT_FP4>::BYTES : Mx<FMT_FP8>::BYTES);
}

// E8M0 scale byte -> fp32 2^(e - 127) (e = 0 is the subnormal 2^-127)
__device__ __forceinline__ float e8m0(uint32_t e) {
    return e ? __uint_as_float(e << 23) : __uint_as_float(0x00400000u);
}

__device__ __forceinline__ uint32_t bits(decltype(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(0u, 1.f, 0)) v) {
    return __builtin_bit_cast(uint32_t, v);
}

// MXINT8 step s of a block: its scale 2^(e - 127) 2^-6 for the lane's column
__device__ __forceinline__ float int8_scale(uint32_t sc, int s) { return e8m0((sc >> (8 * s)) & 0xffu) * 0.015625f; }

// the lane's B fragments of one block: step s holds K values KG q + 32 s + 8 g .. + 7 of the lane's column,
// already multiplied by their scale (MXINT8: the integer codes; the scale is applied to the step's product)
template <int FMT>
__device__ __forceinline__ void dequant(const u32x4 v, uint32_t sc, bf16x8 (&b)[Mx<FMT>::STEPS]) {
    if constexpr (FMT == FMT_FP4) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float f = e8m0((sc >> (8 * s)) & 0xffu);
            b[s] = __builtin_bit_cast(bf16x8, u32x4{bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v[s], f, 0)),
                                                    bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v[s], f, 1)),
                                                    bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v[s], f, 2)),
                                                    bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v[s], f, 3))});
        }
    } else if constexpr (FMT == FMT_INT8) {
        // the integers q themselves (-128 .. 127, exact in bf16; one signed-byte conversion each): the block's
        // scale 2^(e - 133) multiplies the step's product instead (int8_scale, in the stream loop)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            uint32_t wd[4];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t u = v[2 * s + h];
                wd[2 * h] = qs::cvt_pk_bf16((float)(int8_t)(u & 0xffu), (float)(int8_t)((u >> 8) & 0xffu));
                wd[2 * h + 1] = qs::cvt_pk_bf16((float)(int8_t)((u >> 16) & 0xffu), (float)(int8_t)(u >> 24));
            }
            b[s] = __builtin_bit_cast(bf16x8, u32x4{wd[0], wd[1], wd[2], wd[3]});
        }
    } else {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const float f = e8m0((sc >> (8 * s)) & 0xffu);
            b[s] = __builtin_bit_cast(
                bf16x8, u32x4{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[2 * s], f, false)),
                              __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[2 * s], f, true)),
                              __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[2 * s + 1], f, false)),
                              __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[2 * s + 1], f, true))});
        }
    }
}

// ------------------------------------------------------------------------------------------- quantize

// E2M1 code of |y| (round to nearest, ties to the even code; saturates at 6)
__device__ __forceinline__ uint32_t e2m1_code(float a) {
    return a <= 0.25f ? 0u : a < 0.75f ? 1u : a <= 1.25f ? 2u : a < 1.75f ? 3u : a <= 2.5f ? 4u
                                         : a < 3.5f  ? 5u : a <= 5.f ? 6u : 7u;
}
// E4M3 (OCP, no infinities) code of |y|: round to nearest even, saturating at 448 (code 0x7e)
__device__ __forceinline__ uint32_t e4m3_code(float a) {
    if (!(a < 448.f)) return 0x7eu;
    if (a < 0.015625f) return (uint32_t)rintf(a * 512.f);  // subnormals m 2^-9 (m = 8 is 2^-6, code 0x08)
    uint32_t u = __float_as_uint(a);
    u += 0x7ffffu + ((u >> 20) & 1u);  // round the mantissa to 3 bits, ties to even
    const int E = (int)(u >> 23) - 127;
    const uint32_t m = (u >> 20) & 7u;
    if (E > 8 || (E == 8 && m == 7u)) return 0x7eu;
    return ((uint32_t)(E + 7) << 3) | m;
}

// INT8 code (two's complement) of y in units of 2^-6: round to nearest even, saturating at +-127
__device__ __forceinline__ uint32_t int8_code(float y) {
    const float q = fminf(fmaxf(rintf(y), -127.f), 127.f);
    return (uint32_t)(int)q & 0xffu;
}

// one thread per (column n, 32-value K step): the block's scale 2^(floor(log2 amax) - emax), emax 2 (E2M1),
// 8 (E4M3) or 0 (INT8), e clamped to [1, 254] (an all-zero block keeps e = 127), then every value's code,
// written into the fragment-order layout
template <int FMT>
__global__ __launch_bounds__(256) void mx_quantize_kernel(const float *w, uint8_t *out, int K, int N) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    const int steps = K / 32;
    if (i >= (long)steps * N) return;
    const int n = (int)(i % N), ks = (int)(i / N);
    float v[32];
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        v[j] = w[(size_t)(32 * ks + j) * N + n];
        amax = fmaxf(amax, fabsf(v[j]));
    }
    constexpr int emax = FMT == FMT_FP4 ? 2 : FMT == FMT_FP8 ? 8 : 0;
    int e = 127;
    if (amax > 0.f) {
        int ex;
        frexpf(amax, &ex);  // amax = f 2^ex, f in [0.5, 1): floor(log2 amax) = ex - 1
        e = min(254, max(1, ex - 1 - emax + 127));
    }
    const float inv = __uint_as_float((uint32_t)(254 - e) << 23);  // 2^(127 - e), exact
    using M = Mx<FMT>;
    const int t = n / TILE_N, r = n % TILE_N, q = ks / M::STEPS, s = ks % M::STEPS;
    uint8_t *blk = out + ((size_t)t * (K / M::KG) + q) * M::BYTES;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        uint32_t c[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if constexpr (FMT == FMT_INT8) {
                c[j] = int8_code(ldexpf(v[8 * g + j], 133 - e));  // units of 2^(e - 133), scaled exactly
            } else {
                const float y = v[8 * g + j] * inv;
                const uint32_t code = FMT == FMT_FP4 ? e2m1_code(fabsf(y)) : e4m3_code(fabsf(y));
                c[j] = code | (y < 0.f && code ? (FMT == FMT_FP4 ? 8u : 0x80u) : 0u);
            }
        }
        uint8_t *lane = blk + 16 * (16 * g + r);
        if constexpr (FMT == FMT_FP4) {
            *reinterpret_cast<uint32_t *>(lane + 4 * s) = c[0] | (c[1] << 4) | (c[2] << 8) | (c[3] << 12) | (c[4] << 16) |
                                                          (c[5] << 20) | (c[6] << 24) | (c[7] << 28);
        } else {
            *reinterpret_cast<u32x2 *>(lane + 8 * s) =
                u32x2{c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24), c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24)};
        }
    }
    blk[1024 + M::STEPS * r + s] = (uint8_t)e;
}

// --------------------------------------------------------------------------------------- projections

constexpr int WAVES = 4;             // waves per projection workgroup
constexpr int RING2 = 2, RING1 = 4;  // weight groups in flight per wave, with two weights / one
constexpr int H_LDS = 24576;         // most bytes of activation rows a workgroup stages in LDS
constexpr size_t CNT_BYTES = 65536;  // arrival counters at the head of a workspace, one per column tile
constexpr int EPI_SUM = 0, EPI_SILU = 1, EPI_RESID = 2;
constexpr int NX = 5;  // NORM: 16-byte pieces of x and of gamma per thread, rows up to 5120 values

// a buffer descriptor over n bytes from p: reads past the range return zeros without touching memory
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, uint32_t n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)n, 0x00020000);
}

struct Proj {
    const uint8_t *W0, *W1;  // packed weights (W1: the up projection of EPI_SILU)
    const uint16_t *h;       // activation rows [B, K] bf16
    const float *x;          // EPI_RESID: residual rows [B, N]; NORM: the row to normalise [K]
    const float *gamma;      // NORM: [K], or null when the norm weight is folded into the weights (unit gamma)
    float eps;               // NORM
    float *y;                // EPI_SUM, EPI_RESID: output rows [B, N] fp32 (may alias x)
    uint16_t *z;             // EPI_SILU: output rows [B, N] bf16
    float *part;             // nsplit > 1: partial sums [nsplit, NM, B, N] fp32
    int *cnt;                // nsplit > 1: [N / 16] arrival counters, zero between launches
    int B, K, N, nsplit;
    int nwhole;              // > 0: tiles [0, nwhole) in one split each, the others in nsplit (a balanced grid)
};

// K groups [q0, q1) of split `split` out of nq
__host__ __device__ inline int split_begin(int nq, int split, int nsplit) { return (int)((long)nq * split / nsplit); }
// h row pitch in LDS (bf16 values): a split's K range plus a 16-byte skew between rows
__host__ __device__ inline int h_pitch(int ngmax, int kg) { return ngmax * kg + 8; }

// One workgroup per (16-column tile t, K split): the split's activation rows are staged in LDS once, then
// each wave streams every 4th K group of the NM weights through a ring of RING groups held in registers
// (requested RING groups ahead, streaming loads that do not keep the lines in the caches). The ring is
// requested in the same order every step and requests past the split's range read zeros without a memory
// access, so every wave issues an identical, unconditional sequence and the compiler's memory-counter waits
// stay exact. A operand: h rows from LDS (lane (r, g) holds h[r][32 s + 8 g .. + 7] of each 32-value step;
// rows past B repeat row B - 1 and land in output rows that are never stored). The 4 waves' sums meet in
// LDS. With one split the workgroup applies the epilogue; otherwise it stores its partial (written through
// to memory), counts itself in (the count wraps to zero at the last arrival), and the workgroup that
// completes the tile's count sums the partials in split order and applies the epilogue: EPI_SUM y = sum,
// EPI_RESID y = x + sum, EPI_SILU z = bf16(silu(h W0) (h W1)). NORM (one row, one split, K <= 5120): the workgroup forms the
// rmsnorm'd row h from x and gamma itself instead of reading it. HREG: no staging; each ring slot also
// holds the group's A fragments, requested from L2 with its weights (lanes of rows past B read zeros).
template <int FMT, int NM, int EPI, bool NORM, bool HREG>
__global__ __launch_bounds__(256, HREG ? 4 : 5) void proj_kernel(Proj a) {
    using M = Mx<FMT>;
    extern __shared__ __align__(16) uint16_t s_h[];
    __shared__ float s_red[WAVES - 1][NM][4][64];
    __shared__ float s_part[WAVES];
    __shared__ int s_last;
    const int ntile = a.N / TILE_N;
    // tile t, split `split` of nsp: every tile in a.nsplit splits (split-major), or with a.nwhole > 0 the first
    // a.nwhole tiles whole and the rest in a.nsplit consecutive workgroups each
    int t = (int)blockIdx.x % ntile, split = (int)blockIdx.x / ntile, nsp = a.nsplit;
    if (a.nwhole > 0) {
        const int i = (int)blockIdx.x - a.nwhole;
        if (i < 0)
            t = (int)blockIdx.x, split = 0, nsp = 1;
        else
            t = a.nwhole + i / a.nsplit, split = i % a.nsplit;
    }
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, r = lane & 15, g = lane >> 4;
    const int nq = a.K / M::KG;
    const int q0 = split_begin(nq, split, nsp), ng = split_begin(nq, split + 1, nsp) - q0;
    const int P = h_pitch((nq + nsp - 1) / nsp, M::KG);

    // 1. activation rows of the split: B x ng KG values, 16 bytes per request, the first HV per thread
    // requested before the weight ring, any others after it; or, with NORM (one row, one split), the row of
    // x and gamma, NX x 16 bytes of each per thread
    constexpr int HV = NORM ? 1 : 6;
    const int per_row = ng * M::KG / 8, total = a.B * per_row;
    const auto hr = rsrc(a.h, NORM ? 0u : (uint32_t)a.B * a.K * 2);
    u32x4 hv[HV];
    f32x4 xv[NORM ? NX : 1], gv[NORM ? NX : 1];
    if constexpr (NORM) {
        const auto xr = rsrc(a.x, (uint32_t)a.K * 4), gr = rsrc(a.gamma, a.gamma ? (uint32_t)a.K * 4 : 0u);
#pragma unroll
        for (int c = 0; c < NX; ++c) {
            const int i = tid + 256 * c;
            const uint32_t off = i < a.K / 4 ? (uint32_t)i * 16 : 0xffffff00u;
            xv[c] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
            gv[c] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(gr, a.gamma ? off : 0xffffff00u, 0, 0));
        }
        // x and gamma leave before the weight ring: the loads in flight when the stream starts are then the
        // ring's alone, as on every later pass, and the compiler's wait for each ring slot stays exact (with
        // gamma scheduled after the ring it waited for every load at the top of each pass)
        __builtin_amdgcn_sched_barrier(0);
    }
    auto fetch_h = [&](int i0) {
#pragma unroll
        for (int c = 0; c < HV; ++c) {
            const int i = i0 + tid + 256 * c, b = i / per_row, j = i - b * per_row;
            const uint32_t off = i < total ? (uint32_t)((b * a.K + q0 * M::KG + 8 * j) * 2) : 0xffffff00u;
            hv[c] = __builtin_amdgcn_raw_buffer_load_b128(hr, off, 0, 0);
        }
    };
    auto put_h = [&](int i0) {
#pragma unroll
        for (int c = 0; c < HV; ++c) {
            const int i = i0 + tid + 256 * c, b = i / per_row, j = i - b * per_row;
            if (i < total) *reinterpret_cast<u32x4 *>(s_h + b * P + 8 * j) = hv[c];
        }
    };
    if constexpr (!NORM && !HREG) fetch_h(0);

    // 2. the weight ring
    struct Buf {
        u32x4 v[NM];
        uint32_t sc[NM];
        u32x4 a[HREG ? M::STEPS : 1];  // HREG: the group's activation fragments
    };
    const auto har = rsrc(a.h, HREG ? (uint32_t)a.B * a.K * 2 : 0u);
    __amdgpu_buffer_rsrc_t wr[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m)
        wr[m] = rsrc((m == 0 ? a.W0 : a.W1) + ((size_t)t * nq + q0) * M::BYTES, (uint32_t)ng * M::BYTES);
    auto load = [&](int lg, Buf &bf) {
        const uint32_t base = (uint32_t)lg * M::BYTES;
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            bf.v[m] = __builtin_amdgcn_raw_buffer_load_b128(wr[m], base + 16 * lane, 0, qs::CP_NT);
            if constexpr (FMT == FMT_FP4)
                bf.sc[m] = __builtin_amdgcn_raw_buffer_load_b32(wr[m], base + 1024 + 4 * r, 0, qs::CP_NT);
            else
                bf.sc[m] = __builtin_amdgcn_raw_buffer_load_b16(wr[m], base + 1024 + 2 * r, 0, qs::CP_NT);
        }
        if constexpr (HREG)
#pragma unroll
            for (int s = 0; s < M::STEPS; ++s) {
                const uint32_t off = r < a.B && lg < ng
                                         ? (uint32_t)((r * a.K + (q0 + lg) * M::KG + 32 * s + 8 * g) * 2) : 0xffffff00u;
                bf.a[s] = __builtin_amdgcn_raw_buffer_load_b128(har, off, 0, 0);
            }
    };
    constexpr int RING = NM == 2 || (HREG && FMT == FMT_FP4) ? RING2 : RING1;
    Buf ring[RING];
#pragma unroll
    for (int j = 0; j < RING; ++j) load(w + WAVES * j, ring[j]);

    // 3. rows into LDS (row b at b P); NORM: h = bf16(x rsqrt(mean(x^2) + eps) gamma) first, the same
    // arithmetic as rmsnorm_kernel
    if constexpr (HREG) {
    } else if constexpr (NORM) {
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < NX; ++c) ss += xv[c][0] * xv[c][0] + xv[c][1] * xv[c][1] + xv[c][2] * xv[c][2] + xv[c][3] * xv[c][3];
        ss = qs::wave_sum(ss);
        if (lane == 0) s_part[w] = ss;
        __syncthreads();
        const float inv = rsqrtf((s_part[0] + s_part[1] + s_part[2] + s_part[3]) / (float)a.K + a.eps);
        if (!a.gamma)
#pragma unroll
            for (int c = 0; c < NX; ++c) gv[c] = f32x4{1.f, 1.f, 1.f, 1.f};
        const int i0 = q0 * M::KG / 4, i1 = (q0 + ng) * M::KG / 4;  // the split's K range, in float4 pieces
#pragma unroll
        for (int c = 0; c < NX; ++c) {
            const int i = tid + 256 * c;
            if (i >= i0 && i < i1)
                *reinterpret_cast<u32x2 *>(s_h + 4 * (i - i0)) =
                    u32x2{qs::pack_bf2(xv[c][0] * inv * gv[c][0], xv[c][1] * inv * gv[c][1]),
                          qs::pack_bf2(xv[c][2] * inv * gv[c][2], xv[c][3] * inv * gv[c][3])};
        }
    } else {
        put_h(0);
        for (int i0 = 256 * HV; i0 < total; i0 += 256 * HV) {
            fetch_h(i0);
            put_h(i0);
        }
    }
    __syncthreads();

    // 4. stream
    f32x4 acc[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint16_t *hrow = s_h + min(r, a.B - 1) * P + 8 * g;
    const int iters = ((ng + WAVES - 1) / WAVES + RING - 1) / RING;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < RING; ++j) {
            const int lg = w + WAVES * (it * RING + j);
            bf16x8 bw[NM][M::STEPS];
            uint32_t scs[NM];
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                dequant<FMT>(ring[j].v[m], ring[j].sc[m], bw[m]);
                scs[m] = ring[j].sc[m];
            }
            u32x4 ha[HREG ? M::STEPS : 1];
            if constexpr (HREG)
#pragma unroll
                for (int s = 0; s < M::STEPS; ++s) ha[s] = ring[j].a[s];
            load(lg + WAVES * RING, ring[j]);
            __builtin_amdgcn_sched_barrier(0);  // the requests leave before the multiplies
            const uint16_t *hq = hrow + min(lg, ng - 1) * M::KG;
#pragma unroll
            for (int s = 0; s < M::STEPS; ++s) {
                const bf16x8 av = HREG ? __builtin_bit_cast(bf16x8, ha[s]) : *reinterpret_cast<const bf16x8 *>(hq + 32 * s);
#pragma unroll
                for (int m = 0; m < NM; ++m) {
                    if constexpr (FMT == FMT_INT8) {
                        // h q exactly (products of bf16 and 8-bit integers, fp32 sums), then times the scale
                        const f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bw[m][s], f32x4{0.f, 0.f, 0.f, 0.f},
                                                                                0, 0, 0);
                        const float f = int8_scale(scs[m], s);
                        acc[m] = f32x4{fmaf(f, p[0], acc[m][0]), fmaf(f, p[1], acc[m][1]), fmaf(f, p[2], acc[m][2]),
                                       fmaf(f, p[3], acc[m][3])};
                    } else {
                        acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bw[m][s], acc[m], 0, 0, 0);
                    }
                }
            }
        }
    }

    // 5. the 4 waves' sums into wave 0 (lane (r, g) holds rows 4 g + i of column r)
    if (w > 0)
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i) s_red[w - 1][m][i][lane] = acc[m][i];
    __syncthreads();
    const int col = TILE_N * t + r;
    if (w == 0)
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[m][i] += s_red[0][m][i][lane] + s_red[1][m][i][lane] + s_red[2][m][i][lane];

    // 6. partials and the arrival count
    if (nsp > 1) {
        if (w == 0) {
            const auto pr = rsrc(a.part, (uint32_t)nsp * NM * a.B * a.N * 4);
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int b = 4 * g + i;
                    if (b < a.B)
                        __builtin_amdgcn_raw_buffer_store_b32(
                            __float_as_uint(acc[m][i]), pr,
                            (uint32_t)((((split * NM + m) * a.B + b) * a.N + col) * 4), 0, qs::CP_SC1);
                }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) {
            // an increment modulo the splits: the last arrival leaves the count at zero for the next launch
            unsigned *c = reinterpret_cast<unsigned *>(a.cnt) + t;
            s_last = __builtin_amdgcn_atomic_inc32(c, nsp - 1, __ATOMIC_RELAXED, "agent") == (unsigned)nsp - 1;
        }
        __syncthreads();
        if (!s_last || w != 0) return;
        asm volatile("" ::: "memory");
        const auto pr = rsrc(a.part, (uint32_t)nsp * NM * a.B * a.N * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = 4 * g + i;
            if (b >= a.B) continue;
            float v[NM] = {};
            constexpr int PB = 8 / NM;  // splits' partials per round trip, summed in split order
            for (int c0 = 0; c0 < nsp; c0 += PB) {
                float pv[NM][PB];
#pragma unroll
                for (int k = 0; k < PB; ++k)
#pragma unroll
                    for (int m = 0; m < NM; ++m) {
                        const int sp = c0 + k;
                        const uint32_t off =
                            sp < nsp ? (uint32_t)((((sp * NM + m) * a.B + b) * a.N + col) * 4) : 0xffffff00u;
                        pv[m][k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pr, off, 0, qs::CP_SC1));
                    }
#pragma unroll
                for (int k = 0; k < PB; ++k)
#pragma unroll
                    for (int m = 0; m < NM; ++m) v[m] += pv[m][k];
            }
#pragma unroll
            for (int m = 0; m < NM; ++m) acc[m][i] = v[m];
        }
    } else if (w != 0) {
        return;
    }

    // 7. epilogue (wave 0)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int b = 4 * g + i;
        if (b >= a.B) continue;
        const size_t o = (size_t)b * a.N + col;
        if constexpr (EPI == EPI_SILU)
            a.z[o] = (uint16_t)qs::f2bf(qs::silu(acc[0][i]) * acc[NM - 1][i]);
        else if constexpr (EPI == EPI_RESID)
            a.y[o] = a.x[o] + acc[0][i];
        else
            a.y[o] = acc[0][i];
    }
}

// h[b] = bf16(x[b] rsqrt(mean(x[b]^2) + eps) gamma) (gamma null: 1); one workgroup per row. Each chunk of 8192
// values is requested at once (8 x 16 bytes of x and gamma per thread); rows of one chunk are normalised from
// registers.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *x, const float *gamma, uint16_t *h, int H, float eps) {
    __shared__ float s_part[4];
    constexpr int V = 8, CHUNK = 256 * V;  // float4 per thread, float4 per chunk
    const int b = blockIdx.x, tid = threadIdx.x, n4 = H / 4;
    const auto xr = rsrc(x + (size_t)b * H, (uint32_t)H * 4), gr = rsrc(gamma, gamma ? (uint32_t)H * 4 : 0u);
    f32x4 xv[V], gv[V];
    auto fetch = [&](int c0) {
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const int i = c0 + tid + 256 * j;
            const uint32_t off = i < n4 ? (uint32_t)i * 16 : 0xffffff00u;
            xv[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
            gv[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(gr, off, 0, 0));
        }
    };
    float ss = 0.f;
    for (int c0 = 0; c0 < n4; c0 += CHUNK) {
        fetch(c0);
#pragma unroll
        for (int j = 0; j < V; ++j) ss += xv[j][0] * xv[j][0] + xv[j][1] * xv[j][1] + xv[j][2] * xv[j][2] + xv[j][3] * xv[j][3];
    }
    ss = qs::wave_sum(ss);
    if ((tid & 63) == 0) s_part[tid >> 6] = ss;
    __syncthreads();
    const float inv = rsqrtf((s_part[0] + s_part[1] + s_part[2] + s_part[3]) / (float)H + eps);
    for (int c0 = 0; c0 < n4; c0 += CHUNK) {
        if (n4 > CHUNK) fetch(c0);
        if (!gamma)
#pragma unroll
            for (int j = 0; j < V; ++j) gv[j] = f32x4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const int i = c0 + tid + 256 * j;
            if (i < n4)
                *reinterpret_cast<u32x2 *>(h + (size_t)b * H + 4 * i) =
                    u32x2{qs::pack_bf2(xv[j][0] * inv * gv[j][0], xv[j][1] * inv * gv[j][1]),
                          qs::pack_bf2(xv[j][2] * inv * gv[j][2], xv[j][3] * inv * gv[j][3])};
        }
    }
}

// Splits of K for one projection: enough that a split's activation rows fit in LDS, then doubled while the
// grid has fewer than 1024 workgroups and each split keeps at least 16 groups (4 per wave).
// Activation rows: staged in LDS per workgroup (read by every wave; 24 KB of rows bound the K split), or,
// from 8 rows (MXFP4) / 16 rows (MXFP8) on, requested from L2 with each weight group, where the LDS bound
// would cut K into too many short splits (measured per layer at H 5120 / I 17408: gate | up 26.9 against
// 30.7 us at 8 rows, down 34.8 against 38.8 us at 16 rows; slower below those counts).
bool use_hreg(int B, int fmt) { return B >= (fmt == FMT_FP4 ? 8 : 16); }  // 8-bit formats alike

int proj_splits(int B, int K, int N, int fmt) {
    const int kg = kg_of(fmt);
    const int nq = K / kg;
    int s = 1;
    while (!use_hreg(B, fmt) && s < nq && (size_t)B * h_pitch((nq + s - 1) / s, kg) * 2 > (size_t)H_LDS) ++s;
    while ((N / TILE_N) * s < 1024 && nq / (2 * s) >= 16) s *= 2;
    return s;
}
size_t h_lds_bytes(int B, int K, int fmt, int nsplit) {
    const int kg = kg_of(fmt);
    return (size_t)B * h_pitch((K / kg + nsplit - 1) / nsplit, kg) * 2;
}

bool mx_shape_ok(int K, int N, int fmt) {
    return fmt_ok(fmt) && K > 0 && N > 0 && N % TILE_N == 0 && K % kg_of(fmt) == 0 && (size_t)N / TILE_N * 4 <= CNT_BYTES &&
           (long)K * MAX_ROWS * 2 < (1L << 31) && mx_bytes(K, N, fmt) < (1UL << 32);
}

template <int FMT, int NM, int EPI, bool NORM = false, bool HREG = false>
int launch_proj(const Proj &a, hipStream_t st, const char *what) {
    const int ntile = a.N / TILE_N;
    const size_t lds = HREG ? 0 : h_lds_bytes(a.B, a.K, FMT, a.nwhole > 0 ? 1 : a.nsplit);
    const unsigned grid = a.nwhole > 0 ? (unsigned)(a.nwhole + (ntile - a.nwhole) * a.nsplit) : (unsigned)(ntile * a.nsplit);
    proj_kernel<FMT, NM, EPI, NORM, HREG><<<grid, 256, lds, st>>>(a);
    return qs::launch_status(what);
}

// A balanced grid for a one-split projection whose tile count is not a multiple of the 256 CUs: a launch's
// time follows the most workgroups any CU holds (gate | up at I 17408: 1088 tiles, 4.25 per CU, took as long as
// 1280 tiles), so the tiles past the last multiple of 256 are split in nst = 256 / (their count) parts, and
// every CU holds the same work. 0 when the count does not divide 256 or the splits would be shorter than 4
// K groups.
int tail_whole(int ntile, int nq, int *nst) {
    const int whole = ntile / 256 * 256, rest = ntile - whole;
    *nst = 1;
    if (whole == 0 || rest == 0 || 256 % rest || 256 / rest > 8 || nq / (256 / rest) < 4) return 0;
    *nst = 256 / rest;
    return whole;
}

// workspace: counters | partials
size_t proj_ws_bytes(int B, int N, int nm, int nsplit) {
    return nsplit > 1 ? CNT_BYTES + (size_t)nsplit * nm * B * N * 4 : 0;
}

struct MlpWs {
    size_t h, z, part, total;
    int sg, sd;  // K splits of gate | up and of down
    int gw, gst; // one row, one split: gate | up tiles kept whole and the split count of the rest (tail_whole)
};
MlpWs mlp_ws(int B, int H, int I) {
    auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
    MlpWs l;
    l.sg = proj_splits(B, H, I, FMT_FP4);
    l.sd = proj_splits(B, I, H, FMT_FP8);  // the same for MXINT8 (one layout)
    l.gst = 1;
    l.gw = B == 1 && l.sg == 1 && H <= 4 * 256 * NX ? tail_whole(I / TILE_N, H / kg_of(FMT_FP4), &l.gst) : 0;
    l.h = CNT_BYTES;
    l.z = l.h + up((size_t)B * H * 2);
    l.part = l.z + up((size_t)B * I * 2);
    l.total = l.part + up(std::max({(size_t)l.sg * 2 * B * I, (size_t)l.gst * 2 * B * I, (size_t)l.sd * B * H}) * 4);
    return l;
}

}  // namespace

extern "C" size_t qs_mx_packed_bytes(int K, int N, int fmt) {
    if (!mx_shape_ok(K, N, fmt)) return 0;
    return mx_bytes(K, N, fmt);
}

extern "C" int qs_mx_quantize(const float *w, uint8_t *packed, int K, int N, int fmt, void *stream) {
    QS_REQUIRE(w && packed, "qs_mx_quantize: null pointer");
    QS_REQUIRE(mx_shape_ok(K, N, fmt),
               "qs_mx_quantize: fmt %d (4, 8 or 9) needs N %% 16 == 0 and K %% %d == 0 (got K %d, N %d)", fmt,
               kg_of(fmt), K, N);
    const long n = (long)(K / 32) * N;
    const unsigned grid = (unsigned)((n + 255) / 256);
    if (fmt == FMT_FP4)
        mx_quantize_kernel<FMT_FP4><<<grid, 256, 0, QS_STREAM(stream)>>>(w, packed, K, N);
    else if (fmt == FMT_FP8)
        mx_quantize_kernel<FMT_FP8><<<grid, 256, 0, QS_STREAM(stream)>>>(w, packed, K, N);
    else
        mx_quantize_kernel<FMT_INT8><<<grid, 256, 0, QS_STREAM(stream)>>>(w, packed, K, N);
    return qs::launch_status("qs_mx_quantize");
}

extern "C" size_t qs_mx_gemv_workspace_bytes(int B, int K, int N, int fmt) {
    if (!mx_shape_ok(K, N, fmt) || B <= 0 || B > MAX_ROWS) return 0;
    const size_t n = proj_ws_bytes(B, N, 1, proj_splits(B, K, N, fmt));
    return n < (1UL << 32) ? n : 0;
}

extern "C" int qs_mx_gemv(const uint16_t *h, const uint8_t *w, float *y, void *workspace, int B, int K, int N, int fmt,
                          void *stream) {
    QS_REQUIRE(h && w && y, "qs_mx_gemv: null pointer");
    QS_REQUIRE(B > 0 && B <= MAX_ROWS, "qs_mx_gemv: 1 to %d activation rows (got %d)", MAX_ROWS, B);
    QS_REQUIRE(mx_shape_ok(K, N, fmt),
               "qs_mx_gemv: fmt %d (4, 8 or 9) needs N %% 16 == 0 and K %% %d == 0 (got K %d, N %d)", fmt, kg_of(fmt),
               K, N);
    const int s = proj_splits(B, K, N, fmt);
    QS_REQUIRE(proj_ws_bytes(B, N, 1, s) < (1UL << 32), "qs_mx_gemv: K %d, N %d need too many K splits", K, N);
    QS_REQUIRE(s == 1 || workspace, "qs_mx_gemv: this shape needs a workspace of qs_mx_gemv_workspace_bytes");
    Proj a{};
    a.W0 = a.W1 = w;
    a.h = h;
    a.y = y;
    a.cnt = static_cast<int *>(workspace);
    a.part = s > 1 ? reinterpret_cast<float *>(static_cast<char *>(workspace) + CNT_BYTES) : nullptr;
    a.B = B, a.K = K, a.N = N, a.nsplit = s;
    hipStream_t st = QS_STREAM(stream);
    const bool hreg = use_hreg(B, fmt);
    if (fmt == FMT_FP4)
        return hreg ? launch_proj<FMT_FP4, 1, EPI_SUM, false, true>(a, st, "qs_mx_gemv")
                    : launch_proj<FMT_FP4, 1, EPI_SUM>(a, st, "qs_mx_gemv");
    if (fmt == FMT_FP8)
        return hreg ? launch_proj<FMT_FP8, 1, EPI_SUM, false, true>(a, st, "qs_mx_gemv")
                    : launch_proj<FMT_FP8, 1, EPI_SUM>(a, st, "qs_mx_gemv");
    return hreg ? launch_proj<FMT_INT8, 1, EPI_SUM, false, true>(a, st, "qs_mx_gemv")
                : launch_proj<FMT_INT8, 1, EPI_SUM>(a, st, "qs_mx_gemv");
}

extern "C" size_t qs_mlp_decode_workspace_bytes(int B, int H, int I) {
    if (B <= 0 || B > MAX_ROWS || !mx_shape_ok(H, I, FMT_FP4) || !mx_shape_ok(I, H, FMT_FP8)) return 0;
    return mlp_ws(B, H, I).total;
}

extern "C" int qs_mlp_decode(const float *x, const float *gamma, const uint8_t *gate, const uint8_t *up,
                             const uint8_t *down, int down_fmt, float *x_out, void *workspace, int B, int H, int I,
                             float eps, void *stream) {
    QS_REQUIRE(x && gate && up && down && x_out && workspace, "qs_mlp_decode: null pointer");
    QS_REQUIRE(B > 0 && B <= MAX_ROWS, "qs_mlp_decode: 1 to %d rows (got %d)", MAX_ROWS, B);
    QS_REQUIRE(down_fmt == FMT_INT8 || down_fmt == FMT_FP8, "qs_mlp_decode: down_fmt must be %d (MXINT8) or %d (MXFP8), got %d",
               FMT_INT8, FMT_FP8, down_fmt);
    QS_REQUIRE(mx_shape_ok(H, I, FMT_FP4) && mx_shape_ok(I, H, FMT_FP8),
               "qs_mlp_decode: H must be a multiple of 128 and I of 64 (got H %d, I %d)", H, I);
    const MlpWs L = mlp_ws(B, H, I);
    char *ws = static_cast<char *>(workspace);
    uint16_t *h = reinterpret_cast<uint16_t *>(ws + L.h);
    uint16_t *z = reinterpret_cast<uint16_t *>(ws + L.z);
    hipStream_t st = QS_STREAM(stream);
    Proj a{};
    a.cnt = static_cast<int *>(workspace);
    a.part = reinterpret_cast<float *>(ws + L.part);
    a.W0 = gate, a.W1 = up, a.h = h, a.z = z;
    a.B = B, a.K = H, a.N = I, a.nsplit = L.sg;
    if (B == 1 && L.sg == 1 && H <= 4 * 256 * NX) {  // one row: the gate | up workgroups normalise it themselves
        a.x = x, a.gamma = gamma, a.eps = eps;
        if (L.gw > 0) a.nwhole = L.gw, a.nsplit = L.gst;  // a grid that loads every CU alike
        if (int e = launch_proj<FMT_FP4, 2, EPI_SILU, true, false>(a, st, "qs_mlp_decode (rmsnorm, gate, up)")) return e;
    } else {
        rmsnorm_kernel<<<B, 256, 0, st>>>(x, gamma, h, H, eps);
        if (int e = qs::launch_status("qs_mlp_decode (rmsnorm)")) return e;
        const int e = use_hreg(B, FMT_FP4) ? launch_proj<FMT_FP4, 2, EPI_SILU, false, true>(a, st, "qs_mlp_decode (gate, up)")
                                  : launch_proj<FMT_FP4, 2, EPI_SILU>(a, st, "qs_mlp_decode (gate, up)");
        if (e) return e;
    }
    a.W0 = a.W1 = down, a.h = z, a.x = x, a.y = x_out, a.z = nullptr;
    a.K = I, a.N = H, a.nsplit = L.sd, a.nwhole = 0;
    const char *what = "qs_mlp_decode (down, residual)";
    if (down_fmt == FMT_INT8)
        return use_hreg(B, FMT_INT8) ? launch_proj<FMT_INT8, 1, EPI_RESID, false, true>(a, st, what)
                                     : launch_proj<FMT_INT8, 1, EPI_RESID>(a, st, what);
    return use_hreg(B, FMT_FP8) ? launch_proj<FMT_FP8, 1, EPI_RESID, false, true>(a, st, what)
                                : launch_proj<FMT_FP8, 1, EPI_RESID>(a, st, what);
}
