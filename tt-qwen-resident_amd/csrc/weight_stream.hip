// Weight-streaming projections and the MLP half of a decoder layer on gfx950 (the streamer kernels' role:
// kernels/streamer_compute.cpp:371-473, the MLP half of tests/bench_resident_mlp.py:98-105).
//
// Weights are OCP microscaling blocks: 32 consecutive values along K share one E8M0 scale 2^(e - 127);
// MXFP4 stores E2M1 values (gate and up projections; the reference streams these in 4-bit block floating
// point), MXFP8 stores E4M3 values (down projection; 8-bit block floating point in the reference). A weight
// W [K, N] (y = h W) is laid out once, by qs_mx_quantize, in MFMA fragment order: for each 16-column tile t
// and K group q (128 values of K for MXFP4, 64 for MXFP8) one block of 1024 value bytes and the group's
// scales, lane l = 16 g + r (r the column in the tile) owning 16 bytes: the values of K steps
// KG q + 32 s + 8 g .. + 7 for each 32-value step s of the group (4 steps of 4 bytes for MXFP4, low nibble
// first; 2 steps of 8 bytes for MXFP8), then column r's scales (one per step) at 1024 + SCALES r. A wave
// loads its part of a block as one contiguous kilobyte plus a 4- or 2-byte scale word, converts it to bf16
// with the hardware's scaled conversions (v_cvt_scalef32_pk_bf16_fp4 / _fp8: exact, the scale folded in)
// and multiplies on v_mfma_f32_16x16x32_bf16 with the activations (bf16, up to 16 rows) as the A operand.
// The kernels stream weights at the HBM rate; the conversions and MFMAs hide under the loads.
//
// MLP half (qs_mlp_decode): h = bf16(x rsqrt(mean(x^2) + eps) gamma); z = bf16(silu(h G) (h U)) in one
// launch (gate and up tiles in the same workgroup); the down projection split four ways over K into fp32
// partials; x_out = x + the partials' sum.
#include "qs_common.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int FMT_FP4 = 4, FMT_FP8 = 8;
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

__host__ __device__ inline size_t mx_bytes(int K, int N, int fmt) {
    return fmt == FMT_FP4 ? (size_t)(N / TILE_N) * (K / Mx<FMT_FP4>::KG) * Mx<FMT_FP4>::BYTES
                          : (size_t)(N / TILE_N) * (K / Mx<FMT_FP8>::KG) * Mx<FMT_FP8>::BYTES;
}

// E8M0 scale byte -> fp32 2^(e - 127) (e = 0 is the subnormal 2^-127)
__device__ __forceinline__ float e8m0(uint32_t e) {
    return e ? __uint_as_float(e << 23) : __uint_as_float(0x00400000u);
}

__device__ __forceinline__ uint32_t bits(decltype(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(0u, 1.f, 0)) v) {
    return __builtin_bit_cast(uint32_t, v);
}

// the lane's B fragments of one block: step s holds K values KG q + 32 s + 8 g .. + 7 of the lane's column,
// already multiplied by their scale
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

// one thread per (column n, 32-value K step): the block's scale 2^(floor(log2 amax) - emax), emax 2 (E2M1) or
// 8 (E4M3), e clamped to [1, 254] (an all-zero block keeps e = 127), then every value's code, written into the
// fragment-order layout
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
    constexpr int emax = FMT == FMT_FP4 ? 2 : 8;
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
            const float y = v[8 * g + j] * inv;
            const uint32_t code = FMT == FMT_FP4 ? e2m1_code(fabsf(y)) : e4m3_code(fabsf(y));
            c[j] = code | (y < 0.f && code ? (FMT == FMT_FP4 ? 8u : 0x80u) : 0u);
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

// Each workgroup (4 waves) takes NM matrices' 16-column tile t over K groups [q0, q1); wave w takes groups
// q0 + w, q0 + w + 4, ... and the partial sums meet in LDS. Two register sets alternate: the next group's
// blocks and activation rows are requested before the current group is converted and multiplied. A operand:
// rows of h (bf16 [B, K]), lane (r, g) holding h[r][32 s + 8 g .. + 7] of each step; lanes of rows past B
// request nothing and hold zeros.
template <int FMT, int NM>
struct Tile {
    f32x4 acc[NM];
    struct Buf {
        u32x4 v[NM];
        uint32_t sc[NM];
        u32x4 a[Mx<FMT>::STEPS];
    };
    __device__ __forceinline__ void run(const uint8_t *const (&W)[NM], const uint16_t *h, int B, int K, int t, int q0,
                                        int q1, int w, int lane) {
        using M = Mx<FMT>;
        const int r = lane & 15, g = lane >> 4;
        const size_t tile_off = (size_t)t * (K / M::KG) * M::BYTES;
        const uint16_t *hrow = h + (size_t)r * K + 8 * g;
#pragma unroll
        for (int m = 0; m < NM; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto load = [&](int q, Buf &b) {
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const uint8_t *p = W[m] + tile_off + (size_t)q * M::BYTES;
                b.v[m] = *reinterpret_cast<const u32x4 *>(p + 16 * lane);
                b.sc[m] = FMT == FMT_FP4 ? *reinterpret_cast<const uint32_t *>(p + 1024 + 4 * r)
                                         : (uint32_t)*reinterpret_cast<const uint16_t *>(p + 1024 + 2 * r);
            }
#pragma unroll
            for (int s = 0; s < M::STEPS; ++s) {
                b.a[s] = u32x4{0u, 0u, 0u, 0u};
                if (r < B) b.a[s] = *reinterpret_cast<const u32x4 *>(hrow + q * M::KG + 32 * s);
            }
        };
        auto compute = [&](const Buf &b) {
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                bf16x8 bw[M::STEPS];
                dequant<FMT>(b.v[m], b.sc[m], bw);
#pragma unroll
                for (int s = 0; s < M::STEPS; ++s)
                    acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, b.a[s]), bw[s], acc[m], 0, 0, 0);
            }
        };
        Buf b0, b1;
        int q = q0 + w;
        if (q < q1) load(q, b0);
        while (q < q1) {
            if (q + 4 < q1) load(q + 4, b1);
            compute(b0);
            q += 4;
            if (q >= q1) break;
            if (q + 4 < q1) load(q + 4, b0);
            compute(b1);
            q += 4;
        }
    }
    // sum of the 4 waves' partials, left in wave 0 (acc holds rows 4 g + i, column r of the tile)
    __device__ __forceinline__ void reduce(float (*s_red)[NM][4][64], int w, int lane) {
        if (w > 0)
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i) s_red[w - 1][m][i][lane] = acc[m][i];
        __syncthreads();
        if (w == 0)
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[m][i] += s_red[0][m][i][lane] + s_red[1][m][i][lane] + s_red[2][m][i][lane];
    }
};

// y[split][b][n] = sum over the split's K groups of h[b][k] W[k][n] (fp32); grid (N / 16) x nsplit
template <int FMT>
__global__ __launch_bounds__(256) void mx_gemv_kernel(const uint8_t *W, const uint16_t *h, float *y, int B, int K,
                                                      int N, int nsplit) {
    __shared__ float s_red[3][1][4][64];
    const int t = blockIdx.x % (N / TILE_N), split = blockIdx.x / (N / TILE_N);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nq = K / Mx<FMT>::KG;
    const int q0 = (int)((long)nq * split / nsplit), q1 = (int)((long)nq * (split + 1) / nsplit);
    Tile<FMT, 1> tile;
    const uint8_t *Ws[1] = {W};
    tile.run(Ws, h, B, K, t, q0, q1, w, lane);
    tile.reduce(s_red, w, lane);
    if (w == 0) {
        const int col = TILE_N * t + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = 4 * (lane >> 4) + i;
            if (b < B) y[((size_t)split * B + b) * N + col] = tile.acc[0][i];
        }
    }
}

// z[b][n] = bf16(silu(h G)[b][n] (h U)[b][n]); grid N / 16
__global__ __launch_bounds__(256) void gate_up_kernel(const uint8_t *G, const uint8_t *U, const uint16_t *h, uint16_t *z,
                                                      int B, int K, int N) {
    __shared__ float s_red[3][2][4][64];
    const int t = blockIdx.x;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    Tile<FMT_FP4, 2> tile;
    const uint8_t *Ws[2] = {G, U};
    tile.run(Ws, h, B, K, t, 0, K / Mx<FMT_FP4>::KG, w, lane);
    tile.reduce(s_red, w, lane);
    if (w == 0) {
        const int col = TILE_N * t + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = 4 * (lane >> 4) + i;
            if (b < B) z[(size_t)b * N + col] = (uint16_t)qs::f2bf(qs::silu(tile.acc[0][i]) * tile.acc[1][i]);
        }
    }
}

// h[b] = bf16(x[b] rsqrt(mean(x[b]^2) + eps) gamma); one workgroup per row
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *x, const float *gamma, uint16_t *h, int H, float eps) {
    __shared__ float s_part[4];
    const int b = blockIdx.x, tid = threadIdx.x;
    const float *xr = x + (size_t)b * H;
    float ss = 0.f;
    for (int k = tid; k < H; k += 256) ss = fmaf(xr[k], xr[k], ss);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((tid & 63) == 0) s_part[tid >> 6] = ss;
    __syncthreads();
    const float inv = rsqrtf((s_part[0] + s_part[1] + s_part[2] + s_part[3]) / (float)H + eps);
    for (int k = tid; k < H; k += 256) h[(size_t)b * H + k] = (uint16_t)qs::f2bf(xr[k] * inv * gamma[k]);
}

// out[i] = (x ? x[i] : 0) + sum over splits of part[s][i]
__global__ __launch_bounds__(256) void sum_splits_kernel(const float *x, const float *part, float *out, long n,
                                                         int nsplit) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float v = x ? x[i] : 0.f;
    for (int s = 0; s < nsplit; ++s) v += part[(size_t)s * n + i];
    out[i] = v;
}

int gemv_splits(int K, int N, int fmt) {
    const int nq = K / (fmt == FMT_FP4 ? Mx<FMT_FP4>::KG : Mx<FMT_FP8>::KG);
    int s = 1;
    while ((N / TILE_N) * s < 1024 && nq / (2 * s) >= 4) s *= 2;  // enough workgroups, >= 4 groups per split
    return s;
}

bool mx_shape_ok(int K, int N, int fmt) {
    return (fmt == FMT_FP4 || fmt == FMT_FP8) && K > 0 && N > 0 && N % TILE_N == 0 &&
           K % (fmt == FMT_FP4 ? Mx<FMT_FP4>::KG : Mx<FMT_FP8>::KG) == 0 && (long)K * MAX_ROWS * 2 < (1L << 31);
}

struct MlpWs {
    size_t h, z, part, total;
};
MlpWs mlp_ws(int B, int H, int I) {
    auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
    MlpWs l;
    l.h = 0;
    l.z = up((size_t)B * H * 2);
    l.part = l.z + up((size_t)B * I * 2);
    l.total = l.part + up((size_t)DOWN_SPLIT * B * H * 4);
    return l;
}

}  // namespace

extern "C" size_t qs_mx_packed_bytes(int K, int N, int fmt) {
    if (!mx_shape_ok(K, N, fmt)) return 0;
    return mx_bytes(K, N, fmt);
}

extern "C" int qs_mx_quantize(const float *w, uint8_t *packed, int K, int N, int fmt, void *stream) {
    QS_REQUIRE(w && packed, "qs_mx_quantize: null pointer");
    QS_REQUIRE(mx_shape_ok(K, N, fmt), "qs_mx_quantize: fmt %d (4 or 8) needs N %% 16 == 0 and K %% %d == 0 (got K %d, N %d)",
               fmt, fmt == FMT_FP4 ? 128 : 64, K, N);
    const long n = (long)(K / 32) * N;
    const unsigned grid = (unsigned)((n + 255) / 256);
    if (fmt == FMT_FP4)
        mx_quantize_kernel<FMT_FP4><<<grid, 256, 0, QS_STREAM(stream)>>>(w, packed, K, N);
    else
        mx_quantize_kernel<FMT_FP8><<<grid, 256, 0, QS_STREAM(stream)>>>(w, packed, K, N);
    return qs::launch_status("qs_mx_quantize");
}

extern "C" size_t qs_mx_gemv_workspace_bytes(int B, int K, int N, int fmt) {
    if (!mx_shape_ok(K, N, fmt) || B <= 0 || B > MAX_ROWS) return 0;
    const int s = gemv_splits(K, N, fmt);
    return s > 1 ? (size_t)s * B * N * 4 : 0;
}

extern "C" int qs_mx_gemv(const uint16_t *h, const uint8_t *w, float *y, void *workspace, int B, int K, int N, int fmt,
                          void *stream) {
    QS_REQUIRE(h && w && y, "qs_mx_gemv: null pointer");
    QS_REQUIRE(B > 0 && B <= MAX_ROWS, "qs_mx_gemv: 1 to %d activation rows (got %d)", MAX_ROWS, B);
    QS_REQUIRE(mx_shape_ok(K, N, fmt), "qs_mx_gemv: fmt %d (4 or 8) needs N %% 16 == 0 and K %% %d == 0 (got K %d, N %d)",
               fmt, fmt == FMT_FP4 ? 128 : 64, K, N);
    const int s = gemv_splits(K, N, fmt);
    QS_REQUIRE(s == 1 || workspace, "qs_mx_gemv: this shape needs a workspace of qs_mx_gemv_workspace_bytes");
    float *dst = s > 1 ? static_cast<float *>(workspace) : y;
    hipStream_t st = QS_STREAM(stream);
    const unsigned grid = (unsigned)((N / TILE_N) * s);
    if (fmt == FMT_FP4)
        mx_gemv_kernel<FMT_FP4><<<grid, 256, 0, st>>>(w, h, dst, B, K, N, s);
    else
        mx_gemv_kernel<FMT_FP8><<<grid, 256, 0, st>>>(w, h, dst, B, K, N, s);
    if (int e = qs::launch_status("qs_mx_gemv")) return e;
    if (s > 1) {
        const long n = (long)B * N;
        sum_splits_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(nullptr, dst, y, n, s);
        return qs::launch_status("qs_mx_gemv (sum)");
    }
    return QS_OK;
}

extern "C" size_t qs_mlp_decode_workspace_bytes(int B, int H, int I) {
    if (B <= 0 || B > MAX_ROWS || !mx_shape_ok(H, I, FMT_FP4) || !mx_shape_ok(I, H, FMT_FP8) ||
        I % (DOWN_SPLIT * Mx<FMT_FP8>::KG) != 0)
        return 0;
    return mlp_ws(B, H, I).total;
}

extern "C" int qs_mlp_decode(const float *x, const float *gamma, const uint8_t *gate, const uint8_t *up,
                             const uint8_t *down, float *x_out, void *workspace, int B, int H, int I, float eps,
                             void *stream) {
    QS_REQUIRE(x && gamma && gate && up && down && x_out && workspace, "qs_mlp_decode: null pointer");
    QS_REQUIRE(B > 0 && B <= MAX_ROWS, "qs_mlp_decode: 1 to %d rows (got %d)", MAX_ROWS, B);
    QS_REQUIRE(mx_shape_ok(H, I, FMT_FP4) && mx_shape_ok(I, H, FMT_FP8) && I % (DOWN_SPLIT * Mx<FMT_FP8>::KG) == 0,
               "qs_mlp_decode: H must be a multiple of 128 and I of 256 (got H %d, I %d)", H, I);
    const MlpWs L = mlp_ws(B, H, I);
    char *ws = static_cast<char *>(workspace);
    uint16_t *h = reinterpret_cast<uint16_t *>(ws + L.h);
    uint16_t *z = reinterpret_cast<uint16_t *>(ws + L.z);
    float *part = reinterpret_cast<float *>(ws + L.part);
    hipStream_t st = QS_STREAM(stream);
    rmsnorm_kernel<<<B, 256, 0, st>>>(x, gamma, h, H, eps);
    if (int e = qs::launch_status("qs_mlp_decode (rmsnorm)")) return e;
    gate_up_kernel<<<I / TILE_N, 256, 0, st>>>(gate, up, h, z, B, H, I);
    if (int e = qs::launch_status("qs_mlp_decode (gate, up)")) return e;
    mx_gemv_kernel<FMT_FP8><<<(H / TILE_N) * DOWN_SPLIT, 256, 0, st>>>(down, z, part, B, I, H, DOWN_SPLIT);
    if (int e = qs::launch_status("qs_mlp_decode (down)")) return e;
    const long n = (long)B * H;
    sum_splits_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(x, part, x_out, n, DOWN_SPLIT);
    return qs::launch_status("qs_mlp_decode (residual)");
}
