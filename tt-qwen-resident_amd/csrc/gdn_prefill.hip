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
//   chunk_prep  one workgroup per (chunk, key head), fully parallel: the row norms, K K^T and Q K^T on MFMA
//               from the raw bf16 rows (exact products, fp32 sums) once for the key head, then for each of its
//               value heads in turn A and P from the accumulators, the triangular inverse Tm (16 x 16
//               diagonal blocks by forward substitution, then the 32 x 32 and 64 x 64 levels of the block
//               recursion [T1 0; -T2 A21 T1  T2] on fp32 MFMA) and the per-token scalars into the workspace;
//               Tm and P (bf16 hi + lo planes) and a copy of the chunk's k and q rows go there in MFMA
//               fragment order, so the walk loads each fragment as one contiguous kilobyte;
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
constexpr int MAXREP = 4;  // value heads per key head the prep handles (one gate scan per wave)

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

// Fragment order of a matrix the walk multiplies by (its rows are the A operand of 16x16x32 MFMAs): the 16 x 32
// block (row tile rt, column step ks) is one kilobyte, lane l = 16 g + r holding row 16 rt + r, columns
// 32 ks + 8 g .. + 7 in its 16 bytes, blocks ordered by (rt, ks). A wave loads a block as one contiguous
// kilobyte (whole 128-byte lines). Element offset of the 8-column group starting at (row, col):
__device__ __forceinline__ int frag_off(int row, int col, int nks) {
    return (((row >> 4) * nks + (col >> 5)) * 64 + ((col >> 3) & 3) * 16 + (row & 15)) * 8;
}

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
    uint16_t *Tm;               // workspace [nch, NV, 2, 64 x 64] bf16: hi and lo planes of Tm, fragment order
    uint16_t *P;                // workspace [nch, NV, 2, 64 x 64] bf16: hi and lo planes of P, fragment order
    uint16_t *KQ;               // workspace [nch, NK, 2, 64 x 128] bf16: the chunk's k and q rows, fragment order
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

__global__ __launch_bounds__(256, 4) void chunk_prep_kernel(PrefillArgs a) {
    // one workgroup per (chunk, key head): the k, q rows, their norms, K K^T and Q K^T are shared by the rep
    // value heads of the key head, which then take turns for A, P and Tm
    const int lid = qs::xcd_logical(blockIdx.x, a.nch * a.NK);
    const int c = lid / a.NK, kh = lid % a.NK;
    const int rep = a.NV / a.NK;
    const int t0 = c * CH, nval = min(CH, a.T - t0);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int fr = lane & 15, g = lane >> 4;

    // the K / Q images are dead once K K^T, Q K^T and the norms exist: A and Tm reuse their space,
    // which keeps the workgroup at 38 KB of LDS (four per CU)
    __shared__ __align__(16) char s_u[2 * CH * FP * 4];
    __shared__ float s_rk[CH], s_rq[CH], s_G[MAXREP][CH], s_b[MAXREP][CH];
    __shared__ float sM[4][16][16];
    const uint16_t *sK = reinterpret_cast<const uint16_t *>(s_u);
    const uint16_t *sQ = sK + CH * DK;
    float(*sA)[FP] = reinterpret_cast<float(*)[FP]>(s_u);
    float(*sT)[FP] = reinterpret_cast<float(*)[FP]>(s_u + CH * FP * 4);
    static_assert(2 * CH * DK * 2 <= 2 * CH * FP * 4, "the K / Q images must fit in the A / Tm space");

    // 1. the chunk's raw k, q rows of key head kh into swizzled LDS images (zeros past the sequence); the
    //    gates of value head kh rep + w (waves w < rep: lane = token, g = 0 and beta = 0 past the sequence)
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
    if (w < rep && lane < nval) {
        gi = a.g[(size_t)(t0 + lane) * a.NV + kh * rep + w];
        bi = a.beta[(size_t)(t0 + lane) * a.NV + kh * rep + w];
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    // 2. row norms (4 lanes per row; the sum runs over the row's chunks in stored order); cumulative log
    //    decay of each value head (waves w < rep, inclusive scan over the 64 tokens)
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
    if (w < rep) {
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const float up = __shfl_up(gi, d, 64);
            if (lane >= d) gi += up;
        }
        s_G[w][lane] = gi;
        s_b[w][lane] = bi;
    }

    // 2b. the chunk's k and q rows in fragment order for the walk
    {
        uint16_t *dst = a.KQ + ((size_t)c * a.NK + kh) * 2 * CH * DK;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int idx = tid + 256 * m, mat = idx >> 10, piece = idx & 1023;
            const int f = piece >> 6, l = piece & 63;
            const int row = 16 * (f >> 2) + (l & 15), q = 4 * (f & 3) + (l >> 4);
            const uint16_t *img = mat ? sQ : sK;
            *reinterpret_cast<uint4 *>(dst + mat * CH * DK + piece * 8) =
                *reinterpret_cast<const uint4 *>(img + row * DK + ((q ^ sw16(row)) << 3));
        }
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

#pragma unroll 1
    for (int hv = 0; hv < rep; ++hv) {
        const int h = kh * rep + hv;
        const float *sG = s_G[hv], *sB = s_b[hv];
        // 4. A (strictly lower) and P (lower with the diagonal, bf16 hi and lo planes) from the accumulators into
        //    LDS; P is staged in the space Tm takes later and leaves in 16-byte rows
        uint16_t(*sPh)[CH] = reinterpret_cast<uint16_t(*)[CH]>(s_u + CH * FP * 4);
        uint16_t(*sPl)[CH] = reinterpret_cast<uint16_t(*)[CH]>(s_u + CH * FP * 4 + CH * CH * 2);
        static_assert(2 * CH * CH * 2 <= CH * FP * 4, "P's planes must fit in the Tm space");
        {
    #pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ti = sig(w, 4 * g + i);
                const float Gi = sG[ti], rqi = s_rq[ti], bki = sB[ti] * s_rk[ti];
    #pragma unroll
                for (int tc = 0; tc < 4; ++tc) {
                    const int tj = sig(tc, fr);
                    float av = 0.f, p = 0.f;
                    if (ti >= tj) {
                        // e^(G_i - G_j) as 2^((G_i - G_j) log2 e) on the hardware exponential (the rounding of
                        // G_i - G_j dominates the error either way)
                        const float rkj = s_rk[tj] * __builtin_amdgcn_exp2f((Gi - sG[tj]) * 1.4426950408889634f);
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
        // the 16 x 16 blocks above the diagonal (16-column segment past the 16-row tile) are zero in P and Tm:
        // they are not stored, and the walk reads them as an empty range
        if ((tid & 3) <= ((tid >> 2) >> 4)) {
            uint16_t *Pd = a.P + ((size_t)c * a.NV + h) * 2 * CH * CH;
            const int i = tid >> 2, j0 = (tid & 3) * 16;
    #pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int off = frag_off(i, j0 + 8 * u, CH / 32);
                *reinterpret_cast<uint4 *>(Pd + off) = *reinterpret_cast<const uint4 *>(&sPh[i][j0 + 8 * u]);
                *reinterpret_cast<uint4 *>(Pd + CH * CH + off) = *reinterpret_cast<const uint4 *>(&sPl[i][j0 + 8 * u]);
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
            uint16_t *Td = a.Tm + 2 * mat;
            const int o0 = frag_off(i, j0, CH / 32), o1 = frag_off(i, j0 + 8, CH / 32);
            if ((j0 >> 4) <= (i >> 4)) {  // no block above the diagonal (all zero; the walk reads none)
                *reinterpret_cast<uint4 *>(Td + o0) = make_uint4(th[0], th[1], th[2], th[3]);
                *reinterpret_cast<uint4 *>(Td + o1) = make_uint4(th[4], th[5], th[6], th[7]);
                *reinterpret_cast<uint4 *>(Td + CH * CH + o0) = make_uint4(tl[0], tl[1], tl[2], tl[3]);
                *reinterpret_cast<uint4 *>(Td + CH * CH + o1) = make_uint4(tl[4], tl[5], tl[6], tl[7]);
            }
        }
        if (tid < CH) {
            const int i = tid;
            const float gam = expf(sG[i]);
            float *scp = a.sc + ((size_t)c * a.NV + h) * 5 * CH;
            scp[0 * CH + i] = sB[i];
            scp[1 * CH + i] = sB[i] * gam * s_rk[i];
            scp[2 * CH + i] = s_rq[i] * gam;
            scp[3 * CH + i] = s_rk[i] * expf(sG[CH - 1] - sG[i]);
            scp[4 * CH + i] = expf(sG[CH - 1]);
        }
        __syncthreads();  // the next head's A and P overwrite what this head's Tm store reads
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

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// The walk's K image: token rows of 128 d (256 bytes), the 16-byte d groups XOR-swizzled by
// kswz(row) = 2 (row % 4) | (row / 4) % 2. The 16-byte fragment writes (8 consecutive rows per 8 lanes) and
// the transposing reads (4 consecutive rows x 32 bytes per 16 lanes) are both free of bank conflicts.
__device__ __forceinline__ int kimg(int row, int d) {
    return row * DK + ((((d >> 3) ^ (((row & 3) << 1) | ((row >> 2) & 1)))) << 3) + (d & 7);
}

// One workgroup (8 waves) per (value head, 32-column slab of S). Wave (w, role) = (wave % 4, wave / 4) works on
// the 16-token tile w of every chunk product; the two waves of a tile share a SIMD. The k wave (role 0)
// forms K S0 for both column halves of the slab, X = beta V - (beta gamma r_k) K S0 and d = Tm X; the q wave
// (role 1) forms Q S0 and O = (gamma r_q) Q S0 + P d. For the state update S = gamma_C S0 + K^T e each
// wave owns state rows 32 w .. 32 w + 31 of column half `role`; the slab's fp32 state lives in registers
// and is mirrored in LDS as bf16 hi + lo planes (S^T [v][d]), the operand of K S0 and Q S0. Each wave loads only the fragments it multiplies
// by, from the prep's fragment-order copies (one contiguous kilobyte per load, every byte loaded once per
// workgroup): k wave K rows and Tm, q wave Q rows and P, one chunk ahead. What crosses waves goes through
// LDS: the state mirror, X^T, d^T and e^T (split into bf16 hi + lo by the wave that produces them), the
// chunk's K rows (read transposed, K^T [d][token], with ds_read_b64_tr_b16) and the per-token scalars.
// Three barriers per chunk: after X, after d, after the state update. Reads past the sequence end return
// zeros through the buffer descriptors' range checks and writes past it are dropped the same way.
// The walk's X image: token rows of 32 slab columns (64 bytes, no padding), the 8-byte column groups u = v / 4
// XOR-swizzled by xswz(t / 2) = 4 ((t / 2) % 2) + (t / 2) / 2 % 4. The 8-byte writes of 16 consecutive rows and
// the transposing reads (4 consecutive rows x 32 bytes per 16 lanes) are both free of bank conflicts.
__device__ __forceinline__ int ximg(int t, int v) {
    const int m = t >> 1;
    return t * SLAB + ((((v >> 2) ^ (((m & 1) << 2) | ((m >> 1) & 3))) << 2)) + (v & 3);
}

// A B (or A) fragment of 8 rows x 16 columns read across: lane fr of each 16-lane group receives column
// c0 + fr of rows r0 .. r0 + 3 from p0 and of rows r0 + 4 .. r0 + 7 from p4, where each lane points p0 at
// row r0 + fr / 4, columns c0 + 4 (fr % 4) .. + 3 (ds_read_b64_tr_b16) and p4 four rows further
__device__ __forceinline__ bf16x8 tr_frag(const uint16_t *p0, const uint16_t *p4) {
    const i16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4 *)p0);
    const i16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4 *)p4);
    return __builtin_bit_cast(bf16x8, u32x4{__builtin_bit_cast(u32x2, lo4)[0], __builtin_bit_cast(u32x2, lo4)[1],
                                            __builtin_bit_cast(u32x2, hi4)[0], __builtin_bit_cast(u32x2, hi4)[1]});
}

// keeps a group of memory requests where it is written: neither the optimizer nor the scheduler moves code
// across it
__device__ __forceinline__ void fence_issue() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

constexpr int WALK_THREADS = 512;
__global__ __launch_bounds__(WALK_THREADS) void chunk_walk_kernel(PrefillArgs a) {
    // row strides (bf16) of the S^T planes and of the [.][token] planes: 272 and 144 bytes, 16 bytes past a
    // multiple of 128, so the 8 lanes that share a cycle of a 16-byte fragment read (8 consecutive rows) hit
    // 8 different 16-byte bank groups
    constexpr int SKP = DK + 8;
    constexpr int TP = CH + 8;
    const int nwg = a.NV * NSLAB;
    const int lid = qs::xcd_logical(blockIdx.x, nwg);
    const int slab = lid % NSLAB, h = lid / NSLAB;
    const int kh = h / (a.NV / a.NK);
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int w = wv & 3, role = wv >> 2;
    // the k waves issue ahead of the q waves on a shared SIMD: their X, d and Tm requests lead every chunk's
    // chain (the reverse order measured 25% slower, this one 0.5% faster than equal priority)
    if (role == 0) __builtin_amdgcn_s_setprio(1);
    const int fr = lane & 15, g = lane >> 4, fk = g * 8, fq = g * 4;

    __shared__ __align__(16) uint16_t sS[2][SLAB][SKP];
    __shared__ __align__(16) uint16_t sK[CH * DK];
    __shared__ __align__(16) uint16_t sX[2][CH * SLAB];
    __shared__ __align__(16) uint16_t sD[2][SLAB][TP];
    __shared__ __align__(16) uint16_t sE[2][SLAB][TP];
    __shared__ __align__(16) float s_c[2][5][CH];

    // state rows 32 w + 16 mt + fq + i, column 32 slab + 16 role + fr
    float S[2][4];
    auto mirror = [&](int mt) {
        uint2 hi, lo;
        split4(S[mt][0], S[mt][1], S[mt][2], S[mt][3], hi, lo);
        const int v = 16 * role + fr, d = 32 * w + 16 * mt + fq;
        *reinterpret_cast<uint2 *>(&sS[0][v][d]) = hi;
        *reinterpret_cast<uint2 *>(&sS[1][v][d]) = lo;
    };
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            S[mt][i] = a.S0[((size_t)h * DK + 32 * w + 16 * mt + fq + i) * DV + SLAB * slab + 16 * role + fr];
        mirror(mt);
    }

    // Registers of the chunk in flight: fA = the wave's K (role 0) or Q (role 1) fragments, column steps 0..3;
    // fB = its Tm (role 0) or P (role 1) fragments, [plane][column step]; fV = V at row 16 w + fr, columns
    // 16 nh + fq .. + 3 (the accumulator layout of X^T; role 1 reads an empty range); psc = row `wave` of the five
    // per-token scalar rows (waves 0..4; the others an empty range). Every wave issues the same requests in the
    // same order, without a branch, so the compiler's memory-counter waits are exact: a wait for one set skips
    // every set requested after it. The fetches of chunk nch (one past the last) read empty ranges or repeat
    // the last chunk.
    const size_t vrow = (size_t)a.NV * DV * 2;  // bytes per token
    u32x4 fA[4], fB[4];
    u32x2 fV[2];
    uint32_t psc;
    auto fetch_a = [&](int c) {
        const int cc = min(c, a.nch - 1);
        const auto rs = rsrc(a.sc + ((size_t)cc * a.NV + h) * 5 * CH, wv < 5 ? 5 * CH * 4 : 0);
        psc = __builtin_amdgcn_raw_buffer_load_b32(rs, (wv * CH + lane) * 4, 0, 0);
        const uint16_t *src = a.KQ + (((size_t)cc * a.NK + kh) * 2 + role) * CH * DK + frag_off(16 * w + fr, fk, 4);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) fA[ks] = *reinterpret_cast<const u32x4 *>(src + ks * 512);
        const int t0 = c * CH, nv = __builtin_amdgcn_readfirstlane(role == 0 ? max(0, min(CH, a.T - t0)) : 0);
        const auto rv = rsrc(a.v + (size_t)t0 * a.NV * DV, (int)(nv * vrow));
        const int vo = (int)((16 * w + fr) * vrow) + (h * DV + SLAB * slab + fq) * 2;
#pragma unroll
        for (int nh = 0; nh < 2; ++nh) fV[nh] = __builtin_amdgcn_raw_buffer_load_b64(rv, vo + 32 * nh, 0, 0);
    };
    // (the 16 x 16 blocks above the diagonal are zero and never stored: lane group g of wave w reads column
    // step ks as an empty range when its 16-column segment 2 ks + g / 2 lies past row tile w)
    auto fetch_b = [&](int c) {
        const int cc = min(c, a.nch - 1);
        const auto rb = rsrc((role ? a.P : a.Tm) + ((size_t)cc * a.NV + h) * 2 * CH * CH, 2 * CH * CH * 2);
        const int fo = frag_off(16 * w + fr, fk, 2) * 2;
#pragma unroll
        for (int pl = 0; pl < 2; ++pl)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
                fB[2 * pl + ks] = __builtin_amdgcn_raw_buffer_load_b128(
                    rb, 2 * ks + (g >> 1) > w ? 0x7fffff00 : fo + (pl * CH * CH + ks * 512) * 2, 0, 0);
    };
    // output row 16 w + fr, columns 16 nh + fq .. + 3 of chunk c (q waves: O^T accumulators), or nothing (k
    // waves: an empty range), so that every wave issues the same stores
    auto store_o = [&](int c, const f32x4 (&o)[2]) {
        const int t0 = c * CH, nv = __builtin_amdgcn_readfirstlane(role == 1 ? max(0, min(CH, a.T - t0)) : 0);
        const auto ro = rsrc(a.o + (size_t)t0 * a.NV * DV, (int)(nv * vrow));
        const int oo = (int)((16 * w + fr) * vrow) + (h * DV + SLAB * slab + fq) * 2;
#pragma unroll
        for (int nh = 0; nh < 2; ++nh)
            __builtin_amdgcn_raw_buffer_store_b64(
                u32x2{qs::cvt_pk_bf16(o[nh][0], o[nh][1]), qs::cvt_pk_bf16(o[nh][2], o[nh][3])}, ro, oo + 32 * nh, 0, 0);
    };

    // the requests in flight at the top of every chunk, oldest first: the scalars (already consumed), fA and fV
    // of the chunk; its fB; the previous chunk's eight output stores (before the first chunk, eight with an
    // empty range)
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    fence_issue();
    fetch_a(0);
    fence_issue();
    fetch_b(0);
    fence_issue();
    store_o(a.nch, acc);
    fence_issue();
    if (wv < 5) s_c[0][wv][lane] = __uint_as_float(psc);
    __syncthreads();

    for (int c = 0; c < a.nch; ++c) {
        const int cb = c & 1;
        // ---- k wave: the chunk's K rows into the K image; (K S0)^T = S0^T K^T (S0 as hi + lo) and X^T for both
        // column halves, into the X image as hi + lo. q wave: (Q S0)^T for both halves, kept for O^T. The
        // transposed products leave four consecutive columns of one token in each lane.
        if (role == 0) {
#pragma unroll
            for (int ks = 0; ks < DK / 32; ++ks) *reinterpret_cast<u32x4 *>(&sK[kimg(16 * w + fr, 32 * ks + fk)]) = fA[ks];
            bf16x8 bh[2][4], bl[2][4];
#pragma unroll
            for (int nh = 0; nh < 2; ++nh)
#pragma unroll
                for (int ks = 0; ks < DK / 32; ++ks) {
                    bh[nh][ks] = frag(&sS[0][nh * 16 + fr][ks * 32 + fk]);
                    bl[nh][ks] = frag(&sS[1][nh * 16 + fr][ks * 32 + fk]);
                }
#pragma unroll
            for (int nh = 0; nh < 2; ++nh) {
                acc[nh] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < DK / 32; ++ks) {
                    const bf16x8 bk = __builtin_bit_cast(bf16x8, fA[ks]);
                    acc[nh] = mfma(bh[nh][ks], bk, acc[nh]);
                    acc[nh] = mfma(bl[nh][ks], bk, acc[nh]);
                }
            }
            const int t = 16 * w + fr;
            const float c0 = s_c[cb][0][t], c1 = s_c[cb][1][t];
#pragma unroll
            for (int nh = 0; nh < 2; ++nh) {
                uint2 hi, lo;
                split4(c0 * qs::bf_lo(fV[nh][0]) - c1 * acc[nh][0], c0 * qs::bf_hi(fV[nh][0]) - c1 * acc[nh][1],
                       c0 * qs::bf_lo(fV[nh][1]) - c1 * acc[nh][2], c0 * qs::bf_hi(fV[nh][1]) - c1 * acc[nh][3], hi, lo);
                *reinterpret_cast<uint2 *>(&sX[0][ximg(t, 16 * nh + fq)]) = hi;
                *reinterpret_cast<uint2 *>(&sX[1][ximg(t, 16 * nh + fq)]) = lo;
            }
        } else {
            bf16x8 bh[2][4], bl[2][4];
#pragma unroll
            for (int nh = 0; nh < 2; ++nh)
#pragma unroll
                for (int ks = 0; ks < DK / 32; ++ks) {
                    bh[nh][ks] = frag(&sS[0][nh * 16 + fr][ks * 32 + fk]);
                    bl[nh][ks] = frag(&sS[1][nh * 16 + fr][ks * 32 + fk]);
                }
#pragma unroll
            for (int nh = 0; nh < 2; ++nh) {
                acc[nh] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < DK / 32; ++ks) {
                    const bf16x8 bq = __builtin_bit_cast(bf16x8, fA[ks]);
                    acc[nh] = mfma(bh[nh][ks], bq, acc[nh]);
                    acc[nh] = mfma(bl[nh][ks], bq, acc[nh]);
                }
            }
        }
        __syncthreads();
        fence_issue();
        fetch_a(c + 1);  // the scalars land during d; fA and fV during d, O, S and the next barrier
        fence_issue();

        // ---- k wave: d = Tm X (hi*hi + hi*lo + lo*hi) for both halves, as d^T hi + lo and
        // e^T = (d (r_k gamma_C / gamma))^T hi + lo
        if (role == 0) {
            // X fragments (B: tokens 32 ks + fk .. + 7 of column 16 nh + fr) by transposing reads of the X image
            bf16x8 xh[2][2], xl[2][2];
#pragma unroll
            for (int nh = 0; nh < 2; ++nh)
#pragma unroll
                for (int ks = 0; ks < CH / 32; ++ks) {
                    const int row = 32 * ks + fk + (fr >> 2), col = 16 * nh + 4 * (fr & 3);
                    xh[nh][ks] = tr_frag(&sX[0][ximg(row, col)], &sX[0][ximg(row + 4, col)]);
                    xl[nh][ks] = tr_frag(&sX[1][ximg(row, col)], &sX[1][ximg(row + 4, col)]);
                }
            const int r0 = 16 * w + fq;
            const float4 c3 = *reinterpret_cast<const float4 *>(&s_c[cb][3][r0]);
#pragma unroll
            for (int nh = 0; nh < 2; ++nh) {
                f32x4 dacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < CH / 32; ++ks) {
                    const bf16x8 th = __builtin_bit_cast(bf16x8, fB[ks]), tl = __builtin_bit_cast(bf16x8, fB[2 + ks]);
                    dacc = mfma(th, xh[nh][ks], dacc);
                    dacc = mfma(th, xl[nh][ks], dacc);
                    dacc = mfma(tl, xh[nh][ks], dacc);
                }
                const int col = nh * 16 + fr;
                uint2 hi, lo;
                split4(dacc[0], dacc[1], dacc[2], dacc[3], hi, lo);
                *reinterpret_cast<uint2 *>(&sD[0][col][r0]) = hi;
                *reinterpret_cast<uint2 *>(&sD[1][col][r0]) = lo;
                split4(dacc[0] * c3.x, dacc[1] * c3.y, dacc[2] * c3.z, dacc[3] * c3.w, hi, lo);
                *reinterpret_cast<uint2 *>(&sE[0][col][r0]) = hi;
                *reinterpret_cast<uint2 *>(&sE[1][col][r0]) = lo;
            }
        }
        __syncthreads();

        // ---- every wave: S = gamma_C S0 + K^T e for state rows 32 w .. 32 w + 31 of column half `role`. K^T
        // fragments: lane fr of a 16-lane group receives column d0 + fr of token rows R0 .. R0 + 3 from the
        // transposing read. q wave: O^T = (gamma r_q) (Q S0)^T + d^T P^T (hi*hi + lo*hi + hi*lo) for both halves.
        {
            bf16x8 eh[2], el[2], ka[2][2];
#pragma unroll
            for (int ks = 0; ks < CH / 32; ++ks) {
                eh[ks] = frag(&sE[0][role * 16 + fr][ks * 32 + fk]);
                el[ks] = frag(&sE[1][role * 16 + fr][ks * 32 + fk]);
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    const int row = 32 * ks + fk + (fr >> 2), col = 32 * w + 16 * mt + 4 * (fr & 3);
                    ka[ks][mt] = tr_frag(&sK[kimg(row, col)], &sK[kimg(row + 4, col)]);
                }
            }
            if (role == 1) {
                bf16x8 dh[2][2], dl[2][2];
#pragma unroll
                for (int nh = 0; nh < 2; ++nh)
#pragma unroll
                    for (int ks = 0; ks < CH / 32; ++ks) {
                        dh[nh][ks] = frag(&sD[0][nh * 16 + fr][ks * 32 + fk]);
                        dl[nh][ks] = frag(&sD[1][nh * 16 + fr][ks * 32 + fk]);
                    }
                // O^T = (gamma r_q) (Q S0)^T + d^T P^T: A = d^T, B = P^T (the P fragments, read as B)
                const float c2 = s_c[cb][2][16 * w + fr];
#pragma unroll
                for (int nh = 0; nh < 2; ++nh) {
                    f32x4 oacc;
                    oacc[0] = c2 * acc[nh][0];
                    oacc[1] = c2 * acc[nh][1];
                    oacc[2] = c2 * acc[nh][2];
                    oacc[3] = c2 * acc[nh][3];
#pragma unroll
                    for (int ks = 0; ks < CH / 32; ++ks) {
                        const bf16x8 ph = __builtin_bit_cast(bf16x8, fB[ks]), pl = __builtin_bit_cast(bf16x8, fB[2 + ks]);
                        oacc = mfma(dh[nh][ks], ph, oacc);
                        oacc = mfma(dl[nh][ks], ph, oacc);
                        oacc = mfma(dh[nh][ks], pl, oacc);
                    }
                    acc[nh] = oacc;
                }
            }
            const float gc = s_c[cb][4][0];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < CH / 32; ++ks) {
                    sacc = mfma(ka[ks][mt], eh[ks], sacc);
                    sacc = mfma(ka[ks][mt], el[ks], sacc);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) S[mt][i] = fmaf(gc, S[mt][i], sacc[i]);
                mirror(mt);
            }
            if (wv < 5) s_c[cb ^ 1][wv][lane] = __uint_as_float(psc);  // the next chunk's scalars
        }
        fence_issue();
        fetch_b(c + 1);
        fence_issue();
        store_o(c, acc);  // after the next operands are requested: a wait for those never waits for these
        fence_issue();
        __syncthreads();
    }

#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            a.ST[((size_t)h * DK + 32 * w + 16 * mt + fq + i) * DV + SLAB * slab + 16 * role + fr] = S[mt][i];
}

struct PrefillWs {
    size_t tm, p, sc, kq, total;
};
PrefillWs prefill_ws(int T, int NK, int NV) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t nch = (size_t)(T + CH - 1) / CH;
    PrefillWs l;
    l.tm = 0;
    l.p = up(nch * NV * 2 * CH * CH * 2);
    l.sc = l.p + up(nch * NV * 2 * CH * CH * 2);
    l.kq = l.sc + up(nch * NV * 5 * CH * 4);
    l.total = l.kq + up(nch * NK * 2 * CH * DK * 2);
    return l;
}

}  // namespace

// The chunk sizes a caller may name: the reference prefill's 32 (prefill/pp_prefill.py:56, :801) and this
// kernel's 64. The chunked form equals the token-by-token recurrence for every chunk size (the intra-chunk
// WY solve is exact algebra), so both run the 64-token decomposition; a 32-token one would differ from it
// only in rounding.
static bool chunk_ok(int chunk) { return chunk == CH || chunk == CH / 2; }

extern "C" size_t qs_gdn_chunk_prefill_workspace_bytes(int T, int NK, int NV, int DKa, int DVa, int chunk) {
    if (T <= 0 || NK <= 0 || NV <= 0 || NV % NK || NV / NK > MAXREP || DKa != DK || DVa != DV || !chunk_ok(chunk))
        return 0;
    return prefill_ws(T, NK, NV).total;
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
    QS_REQUIRE(NV / NK <= MAXREP, "qs_gdn_chunk_prefill: at most %d value heads per key head are built (got %d)", MAXREP,
               NV / NK);
    QS_REQUIRE(chunk_ok(chunk), "qs_gdn_chunk_prefill: chunk must be %d or %d (got %d)", CH / 2, CH, chunk);
    QS_REQUIRE((long)(T + CH) * NV * DV * 2 < (1L << 31) && (long)(T + CH) * NK * DK * 2 < (1L << 31),
               "qs_gdn_chunk_prefill: T = %d tokens exceed the 2 GB buffer range", T);
    const PrefillWs L = prefill_ws(T, NK, NV);
    char *ws = static_cast<char *>(workspace);
    PrefillArgs a{};
    a.q = q, a.k = k, a.v = v, a.g = g, a.beta = beta, a.S0 = initial_state, a.ST = final_state, a.o = o;
    a.Tm = reinterpret_cast<uint16_t *>(ws + L.tm);
    a.P = reinterpret_cast<uint16_t *>(ws + L.p);
    a.sc = reinterpret_cast<float *>(ws + L.sc);
    a.KQ = reinterpret_cast<uint16_t *>(ws + L.kq);
    a.T = T, a.NK = NK, a.NV = NV, a.nch = (T + CH - 1) / CH, a.scale = scale, a.eps = eps;
    hipStream_t st = QS_STREAM(stream);
    chunk_prep_kernel<<<a.nch * NK, 256, 0, st>>>(a);
    if (int e = qs::launch_status("qs_gdn_chunk_prefill (prep)")) return e;
    chunk_walk_kernel<<<NV * NSLAB, WALK_THREADS, 0, st>>>(a);
    return qs::launch_status("qs_gdn_chunk_prefill (walk)");
}
