// Chunked-prefill gated delta rule (WY / UT-transform form) on gfx950, chunk 64, MFMA bf16 with fp32 state.
//
// Per chunk of C = 64 tokens, value head h (key head h / (NV / NK)), start state S0 [DK, DV], raw bf16
// rows q, k (L2 norms r_q (times scale), r_k applied as fp32 row scalings), cumulative log decay G and
// gamma = e^G:
//   A_ij = beta_i r_k,i r_k,j (k_i . k_j) e^(G_i - G_j)   (i > j),   Tm = (I + A)^-1
//   P_ij = r_q,i r_k,j (q_i . k_j) e^(G_i - G_j)           (i >= j)
//   X  = beta V - diag(beta gamma r_k) (K S0)
//   d  = Tm X
//   O  = diag(gamma r_q) (Q S0) + P d
//   S  = gamma_C S0 + K^T diag(r_k gamma_C / gamma) d
// (the chunked gated delta rule of Yang et al., "Gated Delta Networks", as FLA's chunk_gated_delta_rule
// computes it). Two kernels:
//   chunk_prep  one workgroup per (chunk, value head), fully parallel: K K^T and Q K^T on MFMA from the raw
//               bf16 rows (exact products, fp32 sums), A and P from the accumulators, the triangular inverse
//               Tm (16 x 16 diagonal blocks by forward substitution, then the 32 x 32 and 64 x 64 levels of
//               the block recursion [T1 0; -T2 A21 T1  T2] on fp32 MFMA) and the per-token scalars into the
//               workspace (Tm and P as bf16 hi + lo planes);
//   chunk_walk  one 8-wave workgroup per (value head, 32-column slab of S): the 128 x 32 fp32 state slab stays
//               on chip while the workgroup walks the chunks in order. Every product that touches S or d
//               splits the fp32 operand into bf16 hi + lo halves (two MFMAs, three for Tm x X), so the
//               state keeps fp32-level accuracy.
//
// Row order of the prep's MFMA tiles: row r of a 16-row tile t stands for token sig(t, r) = 32 (t / 2) +
// 8 (r / 4) + 4 (t % 2) + r % 4; with the chunk swizzle sw16 of the K / Q images the 16 rows of any tile read
// 16 different 16-byte bank groups.
// MFMA: v_mfma_f32_16x16x32_bf16; lane l holds A[l % 16][8 (l / 16) + j], B[8 (l / 16) + j][l % 16] (j < 8)
// and C[4 (l / 16) + i][l % 16] (i < 4).
#include "qs_common.h"

namespace {

constexpr int CH = 64;  // chunk
constexpr int DK = 128;
constexpr int DV = 128;
constexpr int FP = CH + 1;  // fp32 row stride of the 64 x 64 matrices of the inverse in LDS
constexpr int SLAB = 32;    // state columns per walk workgroup
constexpr int NSLAB = DV / SLAB;
constexpr int KP = DK + 8;  // bf16 row stride of the walk's K / Q chunk tiles in LDS (272 bytes)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 frag(const void *p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
}
__device__ __forceinline__ bf16x8 as_frag(uint4 u) { return __builtin_bit_cast(bf16x8, u32x4{u.x, u.y, u.z, u.w}); }

// physical row of MFMA row r of tile t
__device__ __forceinline__ int sig(int t, int r) { return 32 * (t >> 1) + 8 * (r >> 2) + 4 * (t & 1) + (r & 3); }
// 16-byte chunk swizzle of the prep's K / Q images: chunk c of token row p sits at position c ^ sw16(p).
// Over the 16 rows sig(t, 0 .. 15) of any tile, sw16 takes 16 distinct values, so the 16 lanes of a fragment
// read hit 16 different 16-byte bank groups.
__device__ __forceinline__ int sw16(int p) { return ((p & 3) << 2) | ((p >> 3) & 3); }

// a buffer descriptor over n bytes from p: reads past the range return zeros, writes past it are dropped
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, int n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, n, 0x00020000);
}
// 16 bytes per lane from byte offset off of r into LDS at lds + 16 lane (lds is wave-uniform)
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void *lds, int off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 16, off, 0, 0, 0);
}

struct PrefillArgs {
    const uint16_t *q, *k, *v;  // [T, NK, DK], [T, NK, DK], [T, NV, DV]
    const float *g, *beta;      // [T, NV]
    const float *S0;            // [NV, DK, DV]
    float *ST;                  // [NV, DK, DV]
    uint16_t *o;                // [T, NV, DV]
    uint16_t *Tm;               // workspace [nch, NV, 2, 64, 64] bf16: hi and lo planes of Tm
    uint16_t *P;                // workspace [nch, NV, 2, 64, 64] bf16: hi and lo planes of P
    float *sc;                  // workspace [nch, NV, 5, 64]: beta | beta gamma r_k | gamma r_q | r_k gamma_C/gamma | gamma_C
    int T, NK, NV, nch;
    float scale, eps;
};

// ------------------------------------------------------------------------------------------------ prep

// C += X Y for 16 x 16 fp32 blocks in LDS (row strides xs, ys) on v_mfma_f32_16x16x4_f32: lane l supplies
// X[l % 16][4 kc + l / 16] and Y[4 kc + l / 16][l % 16]; C is in the accumulator layout C[4 (l / 16) + i][l % 16].
__device__ __forceinline__ void mm16(f32x4 &c, const float *X, int xs, const float *Y, int ys, int lane) {
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(X[(lane & 15) * xs + 4 * kc + (lane >> 4)],
                                                 Y[(4 * kc + (lane >> 4)) * ys + (lane & 15)], c, 0, 0, 0);
}
// an accumulator-layout 16 x 16 block into LDS
__device__ __forceinline__ void put16(float *D, int ds, f32x4 c, int lane) {
#pragma unroll
    for (int i = 0; i < 4; ++i) D[(4 * (lane >> 4) + i) * ds + (lane & 15)] = c[i];
}

__global__ __launch_bounds__(256) void chunk_prep_kernel(PrefillArgs a) {
    const int lid = qs::xcd_logical(blockIdx.x, a.nch * a.NV);
    const int c = lid / a.NV, h = lid % a.NV;  // the value heads of one key head on consecutive ids
    const int rep = a.NV / a.NK, kh = h / rep;
    const int t0 = c * CH, nval = min(CH, a.T - t0);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int fr = lane & 15, g = lane >> 4;

    // the K / Q images are dead once K K^T, Q K^T and the norms exist: A and Tm reuse their space,
    // which keeps the workgroup at 38 KB of LDS (four per CU)
    __shared__ __align__(16) char s_u[2 * CH * FP * 4];
    __shared__ float s_rk[CH], s_rq[CH], s_G[CH], s_b[CH];
    __shared__ float sM[4][16][16];
    const uint16_t *sK = reinterpret_cast<const uint16_t *>(s_u);
    const uint16_t *sQ = sK + CH * DK;
    float(*sA)[FP] = reinterpret_cast<float(*)[FP]>(s_u);
    float(*sT)[FP] = reinterpret_cast<float(*)[FP]>(s_u + CH * FP * 4);
    static_assert(2 * CH * DK * 2 <= 2 * CH * FP * 4, "the K / Q images must fit in the A / Tm space");

    // 1. the chunk's raw k, q rows of key head kh into swizzled LDS images (zeros past the sequence); the
    //    gates of value head h (wave 0: lane = token, g = 0 and beta = 0 past the sequence)
    {
        const size_t krow = (size_t)a.NK * DK * 2;  // bytes per token
        const auto rk = rsrc(a.k + (size_t)t0 * a.NK * DK, (int)(nval * krow));
        const auto rq = rsrc(a.q + (size_t)t0 * a.NK * DK, (int)(nval * krow));
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int e = 256 * m + tid, p = e >> 4;
            const int off = (int)(p * krow) + (kh * DK + ((e & 15) ^ sw16(p)) * 8) * 2;
            dma16(rk, s_u + 4096 * m + 1024 * w, off);
            dma16(rq, s_u + CH * DK * 2 + 4096 * m + 1024 * w, off);
        }
    }
    float gi = 0.f, bi = 0.f;
    if (w == 0 && lane < nval) {
        gi = a.g[(size_t)(t0 + lane) * a.NV + h];
        bi = a.beta[(size_t)(t0 + lane) * a.NV + h];
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    // 2. row norms (4 lanes per row; the sum runs over the row's chunks in stored order); cumulative log
    //    decay (wave 0, inclusive scan over the 64 tokens)
    {
        const int r = tid >> 2, part = tid & 3;
        float kk = 0.f, qq = 0.f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint4 kv = *reinterpret_cast<const uint4 *>(sK + r * DK + (part * 4 + u) * 8);
            const uint4 qv = *reinterpret_cast<const uint4 *>(sQ + r * DK + (part * 4 + u) * 8);
            const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w}, qw[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kk = fmaf(qs::bf_lo(kw[e]), qs::bf_lo(kw[e]), kk);
                kk = fmaf(qs::bf_hi(kw[e]), qs::bf_hi(kw[e]), kk);
                qq = fmaf(qs::bf_lo(qw[e]), qs::bf_lo(qw[e]), qq);
                qq = fmaf(qs::bf_hi(qw[e]), qs::bf_hi(qw[e]), qq);
            }
        }
        kk += qs::dpp<0xB1>(kk);
        kk += qs::dpp<0x4E>(kk);
        qq += qs::dpp<0xB1>(qq);
        qq += qs::dpp<0x4E>(qq);
        if (part == 0) {
            s_rk[r] = rsqrtf(kk + a.eps);
            s_rq[r] = rsqrtf(qq + a.eps) * a.scale;
        }
    }
    if (w == 0) {
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const float up = __shfl_up(gi, d, 64);
            if (lane >= d) gi += up;
        }
        s_G[lane] = gi;
        s_b[lane] = bi;
    }

    // 3. K K^T and Q K^T in row order sig (exact bf16 products, fp32 sums): wave w owns row tile w; element
    //    (4 g + i, fr) of column tile tc pairs tokens sig(w, 4 g + i) and sig(tc, fr)
    f32x4 ckk[4], cqk[4];
    {
        const int pa = sig(w, fr);
        bf16x8 ak[4], aq[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int off = pa * DK + (((4 * ks + g) ^ sw16(pa)) << 3);
            ak[ks] = frag(sK + off);
            aq[ks] = frag(sQ + off);
        }
#pragma unroll
        for (int tc = 0; tc < 4; ++tc) {
            const int pb = sig(tc, fr);
            ckk[tc] = f32x4{0.f, 0.f, 0.f, 0.f};
            cqk[tc] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const bf16x8 bk = frag(sK + pb * DK + (((4 * ks + g) ^ sw16(pb)) << 3));
                ckk[tc] = mfma(ak[ks], bk, ckk[tc]);
                cqk[tc] = mfma(aq[ks], bk, cqk[tc]);
            }
        }
    }
    __syncthreads();  // every read of the K / Q images is done before A overwrites them

    // 4. A (strictly lower) and P (lower with the diagonal, bf16 hi and lo planes) from the accumulators into
    //    LDS; P is staged in the space Tm takes later and leaves in 16-byte rows
    uint16_t(*sPh)[CH] = reinterpret_cast<uint16_t(*)[CH]>(s_u + CH * FP * 4);
    uint16_t(*sPl)[CH] = reinterpret_cast<uint16_t(*)[CH]>(s_u + CH * FP * 4 + CH * CH * 2);
    static_assert(2 * CH * CH * 2 <= CH * FP * 4, "P's planes must fit in the Tm space");
    {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ti = sig(w, 4 * g + i);
            const float Gi = s_G[ti], rqi = s_rq[ti], bki = s_b[ti] * s_rk[ti];
#pragma unroll
            for (int tc = 0; tc < 4; ++tc) {
                const int tj = sig(tc, fr);
                float av = 0.f, p = 0.f;
                if (ti >= tj) {
                    // e^(G_i - G_j) as 2^((G_i - G_j) log2 e) on the hardware exponential (the rounding of
                    // G_i - G_j dominates the error either way)
                    const float rkj = s_rk[tj] * __builtin_amdgcn_exp2f((Gi - s_G[tj]) * 1.4426950408889634f);
                    if (ti > tj) av = bki * rkj * ckk[tc][i];
                    p = rqi * rkj * cqk[tc][i];
                }
                sA[ti][tj] = av;
                const uint32_t ph = qs::cvt_pk_bf16(p, 0.f) & 0xffffu;
                sPh[ti][tj] = (uint16_t)ph;
                sPl[ti][tj] = (uint16_t)qs::cvt_pk_bf16(p - qs::bf2f(ph), 0.f);
            }
        }
    }
    __syncthreads();
    {
        uint16_t *Pd = a.P + ((size_t)c * a.NV + h) * 2 * CH * CH;
        const int i = tid >> 2, j0 = (tid & 3) * 16;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            *reinterpret_cast<uint4 *>(Pd + i * CH + j0 + 8 * u) = *reinterpret_cast<const uint4 *>(&sPh[i][j0 + 8 * u]);
            *reinterpret_cast<uint4 *>(Pd + CH * CH + i * CH + j0 + 8 * u) = *reinterpret_cast<const uint4 *>(&sPl[i][j0 + 8 * u]);
        }
    }
    __syncthreads();  // P's staging space becomes Tm's

    // 5. Tm = (I + A)^-1 by 16 x 16 blocks.
    //  (a) diagonal blocks by forward substitution, wave 0, one column per lane (16 lanes per block):
    //      t_i = [i == col] - sum_{k < i} A_ik t_k, the column held in registers;
    if (w == 0) {
        const int b0 = 16 * (lane >> 4), col = lane & 15;
        float t[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float s = i == col ? 1.f : 0.f;
#pragma unroll
            for (int k = 0; k < i; ++k) s = fmaf(-sA[b0 + i][b0 + k], t[k], s);
            t[i] = s;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) sT[b0 + i][b0 + col] = t[i];
    }
    __syncthreads();
    //  (b) 32 x 32 diagonal blocks: T_10 = -T_11 (A_10 T_00) and T_32 = -T_33 (A_32 T_22), waves 0 and 1;
    if (w < 2) {
        const int b = 32 * w;
        f32x4 m = {0.f, 0.f, 0.f, 0.f};
        mm16(m, &sA[b + 16][b], FP, &sT[b][b], FP, lane);
        put16(&sM[w][0][0], 16, m, lane);
    }
    __syncthreads();
    if (w < 2) {
        const int b = 32 * w;
        f32x4 r = {0.f, 0.f, 0.f, 0.f};
        mm16(r, &sT[b + 16][b + 16], FP, &sM[w][0][0], 16, lane);
        put16(&sT[b + 16][b], FP, -r, lane);
    }
    __syncthreads();
    //  (c) the lower-left 32 x 32 quarter: X_IJ = sum_{K=J}^{1} A_IK T_KJ, then T_IJ = -sum_{K=2}^{I} T_IK X_KJ,
    //      wave w owns block (I, J) = (2 + w / 2, w % 2). MFMA 16x16x4 fp32: exact fp32 products.
    const int I = 2 + (w >> 1), J = w & 1;
    {
        f32x4 x = {0.f, 0.f, 0.f, 0.f};
        for (int K = J; K < 2; ++K) mm16(x, &sA[16 * I][16 * K], FP, &sT[16 * K][16 * J], FP, lane);
        put16(&sM[w][0][0], 16, x, lane);
    }
    __syncthreads();
    {
        f32x4 r = {0.f, 0.f, 0.f, 0.f};
        for (int K = 2; K <= I; ++K) mm16(r, &sT[16 * I][16 * K], FP, &sM[2 * (K - 2) + J][0][0], 16, lane);
        put16(&sT[16 * I][16 * J], FP, -r, lane);
    }
    __syncthreads();

    // 6. Tm (bf16 hi and lo planes, zero above the diagonal) and the per-token scalars to the workspace
    const size_t mat = ((size_t)c * a.NV + h) * CH * CH;
    {
        const int i = tid >> 2, j0 = (tid & 3) * 16;
        uint32_t th[8], tl[8];
#pragma unroll
        for (int u = 0; u < 16; u += 2) {
            const float v0 = i >= j0 + u ? sT[i][j0 + u] : 0.f, v1 = i >= j0 + u + 1 ? sT[i][j0 + u + 1] : 0.f;
            th[u / 2] = qs::cvt_pk_bf16(v0, v1);
            tl[u / 2] = qs::cvt_pk_bf16(v0 - qs::bf_lo(th[u / 2]), v1 - qs::bf_hi(th[u / 2]));
        }
        uint4 *dh = reinterpret_cast<uint4 *>(a.Tm + 2 * mat + i * CH + j0);
        uint4 *dl = reinterpret_cast<uint4 *>(a.Tm + 2 * mat + CH * CH + i * CH + j0);
        dh[0] = make_uint4(th[0], th[1], th[2], th[3]);
        dh[1] = make_uint4(th[4], th[5], th[6], th[7]);
        dl[0] = make_uint4(tl[0], tl[1], tl[2], tl[3]);
        dl[1] = make_uint4(tl[4], tl[5], tl[6], tl[7]);
    }
    if (tid < CH) {
        const int i = tid;
        const float gam = expf(s_G[i]);
        float *scp = a.sc + ((size_t)c * a.NV + h) * 5 * CH;
        scp[0 * CH + i] = s_b[i];
        scp[1 * CH + i] = s_b[i] * gam * s_rk[i];
        scp[2 * CH + i] = s_rq[i] * gam;
        scp[3 * CH + i] = s_rk[i] * expf(s_G[CH - 1] - s_G[i]);
        scp[4 * CH + i] = expf(s_G[CH - 1]);
    }
}

// ------------------------------------------------------------------------------------------------ walk

typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));

// four fp32 -> bf16 hi = rne(x), lo = rne(x - hi), each as four packed bf16 (8 bytes)
__device__ __forceinline__ void split4(float x0, float x1, float x2, float x3, uint2 &hi, uint2 &lo) {
    const uint32_t h0 = qs::cvt_pk_bf16(x0, x1), h1 = qs::cvt_pk_bf16(x2, x3);
    hi = make_uint2(h0, h1);
    lo = make_uint2(qs::cvt_pk_bf16(x0 - __uint_as_float(h0 << 16), x1 - __uint_as_float(h0 & 0xffff0000u)),
                    qs::cvt_pk_bf16(x2 - __uint_as_float(h1 << 16), x3 - __uint_as_float(h1 & 0xffff0000u)));
}

__device__ __forceinline__ bf16x8 frag(const uint16_t *p) { return as_frag(*reinterpret_cast<const uint4 *>(p)); }

// K^T [d][token] rows are 64 tokens (128 bytes) with the 16-byte token groups XOR-swizzled by
// (d ^ d / 8) % 8: the paired-token writes of the transpose and the MFMA fragment reads are both free of
// bank conflicts without padding.
__device__ __forceinline__ int kt_index(int d, int t) {
    return d * CH + ((((t >> 3) ^ (d ^ (d >> 3))) & 7) << 3) + (t & 7);
}

// One workgroup (8 waves) per (value head, 32-column slab of S). Wave (w, nh) = (wave / 2, wave % 2) owns the
// 16-token tile w of every chunk product and the 16-column half nh of the slab; for the state update it owns
// state rows 32 w .. 32 w + 31 of that column half. Two waves per SIMD interleave their dependent MFMA and
// LDS chains, and each wave's chain per chunk is half the one a 4-wave workgroup walks. The slab's fp32
// state lives in registers and is mirrored in LDS as bf16 hi + lo planes, the operand of K S0 and Q S0.
// Every other operand sits in LDS in the orientation its MFMA fragments read (S^T, X^T, d^T [v][token],
// K^T [d][token], K, Q, Tm, P [token][.]) and is split into bf16 hi + lo once, by the wave that produces it.
// The next chunk's K, Q, V, Tm, P and scalars are loaded into registers while the current chunk computes;
// reads past the sequence end return zeros through the buffer descriptors' range checks and writes past it
// are dropped the same way.
constexpr int WALK_THREADS = 512;
__global__ __launch_bounds__(WALK_THREADS) void chunk_walk_kernel(PrefillArgs a) {
    constexpr int SKP = DK + 16;  // bf16 row stride of the S^T planes
    constexpr int TP = CH + 16;   // bf16 row stride of the [.][token] planes
    const int nwg = a.NV * NSLAB;
    const int lid = qs::xcd_logical(blockIdx.x, nwg);
    const int slab = lid % NSLAB, h = lid / NSLAB;
    const int kh = h / (a.NV / a.NK);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int w = wv >> 1, nh = wv & 1;
    const int fr = lane & 15, fk = (lane >> 4) * 8, fq = (lane >> 4) * 4;

    __shared__ __align__(16) uint16_t sS[2][SLAB][SKP];
    __shared__ __align__(16) uint16_t sK[CH][KP];
    __shared__ __align__(16) uint16_t sQ[CH][KP];
    __shared__ __align__(16) uint16_t sKt[DK * CH];
    __shared__ __align__(16) uint16_t sVt[SLAB][CH + 4];
    __shared__ __align__(16) uint16_t sTm[2][CH][TP];
    __shared__ __align__(16) uint16_t sP[2][CH][TP];
    __shared__ __align__(16) uint16_t sX[2][SLAB][TP];
    __shared__ __align__(16) uint16_t sD[2][SLAB][TP];
    __shared__ __align__(16) uint16_t sE[2][SLAB][TP];
    __shared__ __align__(16) float s_c[5 * CH];

    // state rows 32 w + 16 mt + fq + i, column 32 slab + 16 nh + fr
    float S[2][4];
    auto mirror = [&](int mt) {
        uint2 hi, lo;
        split4(S[mt][0], S[mt][1], S[mt][2], S[mt][3], hi, lo);
        const int v = 16 * nh + fr, d = 32 * w + 16 * mt + fq;
        *reinterpret_cast<uint2 *>(&sS[0][v][d]) = hi;
        *reinterpret_cast<uint2 *>(&sS[1][v][d]) = lo;
    };
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            S[mt][i] = a.S0[((size_t)h * DK + 32 * w + 16 * mt + fq + i) * DV + SLAB * slab + 16 * nh + fr];
        mirror(mt);
    }

    // per-thread share of a chunk: 16-byte group kc = tid % 16 of K and Q rows 2 p and 2 p + 1, p = tid / 16
    // (16 consecutive threads read one 256-byte row); V rows 2 (tid / 16) and + 1, columns 2 (tid % 16) .. + 1;
    // Tm and P 16-byte pieces tid + 512 m of their hi | lo planes; scalars tid < 320. K, Q, V of the next
    // chunk are requested after the barrier that follows K S0, Tm, P and the scalars after the next one: no
    // prefetch register is live while K S0 and Q S0 read their operands (issued earlier, measured slower).
    const int kc = tid & 15, pp = tid >> 4;
    const size_t krow = (size_t)a.NK * DK * 2, vrow = (size_t)a.NV * DV * 2;  // bytes per token
    // (vectors, not arrays: they stay in registers whatever the unroll order)
    u32x8 pk, pq, ptm, ppm;
    uint32_t pv0, pv1;
    float psc;
    auto fetch_kqv = [&](int c) {
        const int t0 = c * CH, nv = min(CH, a.T - t0);
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a.k) + (size_t)t0 * a.NK * DK,
                                                          (short)0, (int)(nv * krow), 0x00020000);
        const auto rq = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a.q) + (size_t)t0 * a.NK * DK,
                                                          (short)0, (int)(nv * krow), 0x00020000);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a.v) + (size_t)t0 * a.NV * DV,
                                                          (short)0, (int)(nv * vrow), 0x00020000);
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int off = (int)((2 * pp + m) * krow) + (kh * DK + kc * 8) * 2;
            const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0);
            const u32x4 y = __builtin_amdgcn_raw_buffer_load_b128(rq, off, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) pk[4 * m + j] = x[j], pq[4 * m + j] = y[j];
        }
        const int vo = (int)(2 * pp * vrow) + (h * DV + SLAB * slab + kc * 2) * 2;
        pv0 = __builtin_amdgcn_raw_buffer_load_b32(rv, vo, 0, 0);
        pv1 = __builtin_amdgcn_raw_buffer_load_b32(rv, vo + (int)vrow, 0, 0);
    };
    auto fetch_tp = [&](int c) {
        const size_t mat = ((size_t)c * a.NV + h) * CH * CH;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const uint4 x = *reinterpret_cast<const uint4 *>(a.Tm + 2 * mat + (tid + WALK_THREADS * m) * 8);
            const uint4 y = *reinterpret_cast<const uint4 *>(a.P + 2 * mat + (tid + WALK_THREADS * m) * 8);
            ptm[4 * m] = x.x, ptm[4 * m + 1] = x.y, ptm[4 * m + 2] = x.z, ptm[4 * m + 3] = x.w;
            ppm[4 * m] = y.x, ppm[4 * m + 1] = y.y, ppm[4 * m + 2] = y.z, ppm[4 * m + 3] = y.w;
        }
        psc = tid < 5 * CH ? a.sc[((size_t)c * a.NV + h) * 5 * CH + tid] : 0.f;
    };
    fetch_kqv(0);
    fetch_tp(0);

    // a chunk's output rows are stored at the start of the next chunk, after that chunk's operands have
    // been waited for, so the stores never sit in front of a prefetch in the memory counter
    f32x4 opend;
    auto store_o = [&](int c) {
        const int t0 = c * CH, nv = min(CH, a.T - t0), r0 = 16 * w + fq;
        const auto ro = __builtin_amdgcn_make_buffer_rsrc(a.o + (size_t)t0 * a.NV * DV, (short)0, (int)(nv * vrow),
                                                          0x00020000);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_buffer_store_b16((unsigned short)qs::cvt_pk_bf16(opend[i], 0.f), ro,
                                                  (int)((r0 + i) * vrow) + (h * DV + SLAB * slab + nh * 16 + fr) * 2, 0,
                                                  0);
    };

    for (int c = 0; c < a.nch; ++c) {
        // ---- this chunk's operands from registers into LDS
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int r = 2 * pp + m;
            *reinterpret_cast<uint4 *>(&sK[r][kc * 8]) = make_uint4(pk[4 * m], pk[4 * m + 1], pk[4 * m + 2], pk[4 * m + 3]);
            *reinterpret_cast<uint4 *>(&sQ[r][kc * 8]) = make_uint4(pq[4 * m], pq[4 * m + 1], pq[4 * m + 2], pq[4 * m + 3]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {  // K^T: token pair (2 pp, 2 pp + 1) as one 32-bit word per d
            const int d = kc * 8 + 2 * e;
            const uint32_t ev = pk[e], od = pk[4 + e];
            *reinterpret_cast<uint32_t *>(&sKt[kt_index(d, 2 * pp)]) = (ev & 0xffffu) | (od << 16);
            *reinterpret_cast<uint32_t *>(&sKt[kt_index(d + 1, 2 * pp)]) = (ev >> 16) | (od & 0xffff0000u);
        }
        {  // V^T: the token pair as one 32-bit word per column
            const int col = kc * 2, t = 2 * pp;
            *reinterpret_cast<uint32_t *>(&sVt[col][t]) = (pv0 & 0xffffu) | (pv1 << 16);
            *reinterpret_cast<uint32_t *>(&sVt[col + 1][t]) = (pv0 >> 16) | (pv1 & 0xffff0000u);
        }
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int idx = tid + WALK_THREADS * m;
            *reinterpret_cast<uint4 *>(&sTm[idx >> 9][(idx >> 3) & 63][(idx & 7) * 8]) =
                make_uint4(ptm[4 * m], ptm[4 * m + 1], ptm[4 * m + 2], ptm[4 * m + 3]);
            *reinterpret_cast<uint4 *>(&sP[idx >> 9][(idx >> 3) & 63][(idx & 7) * 8]) =
                make_uint4(ppm[4 * m], ppm[4 * m + 1], ppm[4 * m + 2], ppm[4 * m + 3]);
        }
        if (tid < 5 * CH) s_c[tid] = psc;
        if (c > 0) store_o(c - 1);
        __syncthreads();

        // ---- K S0 and Q S0 for token tile w, column half nh (S0 as hi + lo); every fragment is requested
        // before the first MFMA (the scheduler barrier keeps the reads together)
        f32x4 kacc = {0.f, 0.f, 0.f, 0.f}, qacc = {0.f, 0.f, 0.f, 0.f};
        {
            bf16x8 ak[4], aq[4], bh[4], bl[4];
#pragma unroll
            for (int ks = 0; ks < DK / 32; ++ks) {
                ak[ks] = frag(&sK[16 * w + fr][ks * 32 + fk]);
                aq[ks] = frag(&sQ[16 * w + fr][ks * 32 + fk]);
                bh[ks] = frag(&sS[0][nh * 16 + fr][ks * 32 + fk]);
                bl[ks] = frag(&sS[1][nh * 16 + fr][ks * 32 + fk]);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int ks = 0; ks < DK / 32; ++ks) {
                kacc = mfma(ak[ks], bh[ks], kacc);
                kacc = mfma(ak[ks], bl[ks], kacc);
                qacc = mfma(aq[ks], bh[ks], qacc);
                qacc = mfma(aq[ks], bl[ks], qacc);
            }
        }

        // ---- X = beta V - (beta gamma r_k) (K S0), as X^T hi + lo
        {
            const int r0 = 16 * w + fq;
            const float4 c0 = *reinterpret_cast<const float4 *>(&s_c[0 * CH + r0]);
            const float4 c1 = *reinterpret_cast<const float4 *>(&s_c[1 * CH + r0]);
            const int col = nh * 16 + fr;
            const uint2 v4 = *reinterpret_cast<const uint2 *>(&sVt[col][r0]);
            uint2 hi, lo;
            split4(c0.x * qs::bf_lo(v4.x) - c1.x * kacc[0], c0.y * qs::bf_hi(v4.x) - c1.y * kacc[1],
                   c0.z * qs::bf_lo(v4.y) - c1.z * kacc[2], c0.w * qs::bf_hi(v4.y) - c1.w * kacc[3], hi, lo);
            *reinterpret_cast<uint2 *>(&sX[0][col][r0]) = hi;
            *reinterpret_cast<uint2 *>(&sX[1][col][r0]) = lo;
        }
        __syncthreads();
        if (c + 1 < a.nch) fetch_kqv(c + 1);  // lands during d, O, S and the next fill

        // ---- d = Tm X (hi*hi + hi*lo + lo*hi), as d^T hi + lo and e^T = (d (r_k gamma_C / gamma))^T hi + lo
        {
            f32x4 dacc = {0.f, 0.f, 0.f, 0.f};
            bf16x8 th[2], tl[2], xh[2], xl[2];
#pragma unroll
            for (int ks = 0; ks < CH / 32; ++ks) {
                th[ks] = frag(&sTm[0][16 * w + fr][ks * 32 + fk]);
                tl[ks] = frag(&sTm[1][16 * w + fr][ks * 32 + fk]);
                xh[ks] = frag(&sX[0][nh * 16 + fr][ks * 32 + fk]);
                xl[ks] = frag(&sX[1][nh * 16 + fr][ks * 32 + fk]);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int ks = 0; ks < CH / 32; ++ks) {
                dacc = mfma(th[ks], xh[ks], dacc);
                dacc = mfma(th[ks], xl[ks], dacc);
                dacc = mfma(tl[ks], xh[ks], dacc);
            }
            const int r0 = 16 * w + fq;
            const float4 c3 = *reinterpret_cast<const float4 *>(&s_c[3 * CH + r0]);
            const int col = nh * 16 + fr;
            uint2 hi, lo;
            split4(dacc[0], dacc[1], dacc[2], dacc[3], hi, lo);
            *reinterpret_cast<uint2 *>(&sD[0][col][r0]) = hi;
            *reinterpret_cast<uint2 *>(&sD[1][col][r0]) = lo;
            split4(dacc[0] * c3.x, dacc[1] * c3.y, dacc[2] * c3.z, dacc[3] * c3.w, hi, lo);
            *reinterpret_cast<uint2 *>(&sE[0][col][r0]) = hi;
            *reinterpret_cast<uint2 *>(&sE[1][col][r0]) = lo;
        }
        __syncthreads();
        if (c + 1 < a.nch) fetch_tp(c + 1);

        // ---- O = (gamma r_q) (Q S0) + P d  (hi*hi + hi*lo + lo*hi) for token tile w, column half nh, and
        // S = gamma_C S0 + K^T e for state rows 32 w .. 32 w + 31, column half nh; the fragments of both are
        // requested before the first MFMA
        {
            bf16x8 ap[2], apl[2], dh[2], dl[2], ka[2][2], eh[2], el[2];
#pragma unroll
            for (int ks = 0; ks < CH / 32; ++ks) {
                ap[ks] = frag(&sP[0][16 * w + fr][ks * 32 + fk]);
                apl[ks] = frag(&sP[1][16 * w + fr][ks * 32 + fk]);
                dh[ks] = frag(&sD[0][nh * 16 + fr][ks * 32 + fk]);
                dl[ks] = frag(&sD[1][nh * 16 + fr][ks * 32 + fk]);
                eh[ks] = frag(&sE[0][nh * 16 + fr][ks * 32 + fk]);
                el[ks] = frag(&sE[1][nh * 16 + fr][ks * 32 + fk]);
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) ka[ks][mt] = frag(&sKt[kt_index(32 * w + 16 * mt + fr, ks * 32 + fk)]);
            }
            const int r0 = 16 * w + fq;
            const float4 c2 = *reinterpret_cast<const float4 *>(&s_c[2 * CH + r0]);
            const float gC = s_c[4 * CH];
            __builtin_amdgcn_sched_barrier(0);
            f32x4 oacc;
            oacc[0] = c2.x * qacc[0];
            oacc[1] = c2.y * qacc[1];
            oacc[2] = c2.z * qacc[2];
            oacc[3] = c2.w * qacc[3];
#pragma unroll
            for (int ks = 0; ks < CH / 32; ++ks) {
                oacc = mfma(ap[ks], dh[ks], oacc);
                oacc = mfma(ap[ks], dl[ks], oacc);
                oacc = mfma(apl[ks], dh[ks], oacc);
            }
            opend = oacc;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < CH / 32; ++ks) {
                    sacc = mfma(ka[ks][mt], eh[ks], sacc);
                    sacc = mfma(ka[ks][mt], el[ks], sacc);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) S[mt][i] = fmaf(gC, S[mt][i], sacc[i]);
                mirror(mt);
            }
        }
        __syncthreads();
    }
    store_o(a.nch - 1);

#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            a.ST[((size_t)h * DK + 32 * w + 16 * mt + fq + i) * DV + SLAB * slab + 16 * nh + fr] = S[mt][i];
}

struct PrefillWs {
    size_t tm, p, sc, total;
};
PrefillWs prefill_ws(int T, int NV) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t nch = (size_t)(T + CH - 1) / CH;
    PrefillWs l;
    l.tm = 0;
    l.p = up(nch * NV * 2 * CH * CH * 2);
    l.sc = l.p + up(nch * NV * 2 * CH * CH * 2);
    l.total = l.sc + up(nch * NV * 5 * CH * 4);
    return l;
}

}  // namespace

extern "C" size_t qs_gdn_chunk_prefill_workspace_bytes(int T, int NK, int NV, int DKa, int DVa, int chunk) {
    if (T <= 0 || NK <= 0 || NV <= 0 || NV % NK || DKa != DK || DVa != DV || chunk != CH) return 0;
    return prefill_ws(T, NV).total;
}

extern "C" int qs_gdn_chunk_prefill(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *g,
                                    const float *beta, const float *initial_state, uint16_t *o, float *final_state,
                                    void *workspace, int T, int NK, int NV, int DKa, int DVa, int chunk, float scale,
                                    float eps, void *stream) {
    QS_REQUIRE(q && k && v && g && beta && initial_state && o && final_state && workspace,
               "qs_gdn_chunk_prefill: null pointer");
    QS_REQUIRE(T > 0, "qs_gdn_chunk_prefill: T must be positive (got %d)", T);
    QS_REQUIRE(DKa == DK && DVa == DV, "qs_gdn_chunk_prefill: DK and DV must be 128 (got %d, %d)", DKa, DVa);
    QS_REQUIRE(NK > 0 && NV > 0 && NV % NK == 0, "qs_gdn_chunk_prefill: NV (%d) must be a multiple of NK (%d)", NV, NK);
    QS_REQUIRE(chunk == CH, "qs_gdn_chunk_prefill: only chunk %d is built (got %d)", CH, chunk);
    QS_REQUIRE((long)(T + CH) * NV * DV * 2 < (1L << 31) && (long)(T + CH) * NK * DK * 2 < (1L << 31),
               "qs_gdn_chunk_prefill: T = %d tokens exceed the 2 GB buffer range", T);
    const PrefillWs L = prefill_ws(T, NV);
    char *ws = static_cast<char *>(workspace);
    PrefillArgs a{};
    a.q = q, a.k = k, a.v = v, a.g = g, a.beta = beta, a.S0 = initial_state, a.ST = final_state, a.o = o;
    a.Tm = reinterpret_cast<uint16_t *>(ws + L.tm);
    a.P = reinterpret_cast<uint16_t *>(ws + L.p);
    a.sc = reinterpret_cast<float *>(ws + L.sc);
    a.T = T, a.NK = NK, a.NV = NV, a.nch = (T + CH - 1) / CH, a.scale = scale, a.eps = eps;
    hipStream_t st = QS_STREAM(stream);
    chunk_prep_kernel<<<a.nch * NV, 256, 0, st>>>(a);
    if (int e = qs::launch_status("qs_gdn_chunk_prefill (prep)")) return e;
    chunk_walk_kernel<<<NV * NSLAB, WALK_THREADS, 0, st>>>(a);
    return qs::launch_status("qs_gdn_chunk_prefill (walk)");
}
