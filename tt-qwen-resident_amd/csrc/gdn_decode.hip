// Gated DeltaNet decode-time state path on gfx950: conv1d update, gates, L2-norm + gated delta rule
// (decode and T-token verify) and the verify rollback.
//
// Workgroup decomposition of the delta rule. For value column v the step is column-separable:
//     delta_v = beta (v_v - e^g sum_k k_k S_kv),  S'_kv = e^g S_kv + k_k delta_v,  o_v = sum_k q_k S'_kv
// so one workgroup owns a 128 x 32 slab S[:, 32 s .. 32 s + 31] of one (user, value head): 4 slabs per head,
// B * NV * 4 workgroups of 256 threads. Thread (rg = tid / 8, cg = tid % 8) holds rows rg + 32 i (i < 4),
// columns 4 cg .. 4 cg + 3 of the slab in 16 VGPRs; one wave-wide dwordx4 load covers 8 full 128-byte rows
// of the slab. The two k-reductions (S^T k and S'^T q) run as a 3-step lane butterfly inside the wave plus
// one LDS stage across the 4 waves, in a fixed order (bit-reproducible run to run). The state is read once
// and written once per token.
#include "qs_common.h"

namespace {

constexpr int DK = 128;
constexpr int DV = 128;
constexpr int KC = 4;  // conv taps
constexpr int SLAB = 32;
constexpr int NSLAB = DV / SLAB;
constexpr int THREADS = 256;
constexpr int TMAX = 8;
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct GdnArgs {
    const uint16_t *q, *k, *v;  // q|k|v mode: [B, T, NK, DK], [B, T, NK, DK], [B, T, NV, DV]
    const uint16_t *x;          // conv mode: projection slice [B, T, C]
    const uint16_t *conv_in;    // [B, C, KC-1]
    uint16_t *conv_out;         // decode: == conv_in (in place); verify: [T, B, C, KC-1]
    const uint16_t *taps;       // [C, KC]
    uint16_t *y_out;            // nullable: conv output [B, T, C]
    const float *g, *beta;      // [B, T, NV]
    const float *s_in;          // [B, NV, DK, DV]
    float *s_out;               // decode: == s_in (in place); verify: [T, B, NV, DK, DV]
    uint16_t *o;                // [B, T, NV, DV]
    int *counters;              // decode + conv: [B, NK] self-resetting
    int B, T, NK, NV, C;
    float scale, eps;
};

// Inputs of one channel's causal conv: the K-1 history values, the K taps and the channel's x for every
// token. Loaded before the state slab so the prologue does not queue behind it.
template <int TM>
struct ConvIn {
    float h[3], w[4];
    uint32_t x[TM];
};

template <int TM>
__device__ __forceinline__ ConvIn<TM> conv_load(const GdnArgs &a, int b, int c, int T) {
    ConvIn<TM> in;
    const uint16_t *cs = a.conv_in + ((size_t)b * a.C + c) * (KC - 1);
    in.h[0] = qs::bf2f(cs[0]);
    in.h[1] = qs::bf2f(cs[1]);
    in.h[2] = qs::bf2f(cs[2]);
    const uint2 tw = *reinterpret_cast<const uint2 *>(a.taps + (size_t)c * KC);
    in.w[0] = qs::bf_lo(tw.x), in.w[1] = qs::bf_hi(tw.x), in.w[2] = qs::bf_lo(tw.y), in.w[3] = qs::bf_hi(tw.y);
#pragma unroll
    for (int t = 0; t < TM; ++t)
        if (t < T) in.x[t] = a.x[((size_t)b * T + t) * a.C + c];
    return in;
}

// Conv1d + SiLU of one channel over T tokens (window oldest first, tap 0 on the oldest input). The tap
// products of two bf16 values are exact in fp32, so fused or unfused multiply-adds round identically.
// Writes the bf16-rounded outputs (as fp32) to y[t * ystride], optionally the per-token conv-state
// snapshots (verify); leaves the final window in in.h[0..2].
template <bool SNAP, int TM>
__device__ __forceinline__ void conv_run(const GdnArgs &a, ConvIn<TM> &in, int b, int c, int T, float *y,
                                         int ystride, bool write_out) {
    float *h = in.h;
    const float *w = in.w;
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        if (t >= T) break;
        const uint32_t xr = in.x[t];
        const float xt = qs::bf2f(xr);
        float acc = h[0] * w[0];
        acc = acc + h[1] * w[1];
        acc = acc + h[2] * w[2];
        acc = acc + xt * w[3];
        const uint32_t yb = qs::f2bf(qs::silu(acc));
        y[t * ystride] = qs::bf2f(yb);
        if (write_out && a.y_out) a.y_out[((size_t)b * T + t) * a.C + c] = (uint16_t)yb;
        h[0] = h[1];
        h[1] = h[2];
        h[2] = xt;
        if (SNAP && write_out) {
            uint16_t *d = a.conv_out + (((size_t)t * a.B + b) * a.C + c) * (KC - 1);
            d[0] = (uint16_t)qs::f2bf(h[0]);
            d[1] = (uint16_t)qs::f2bf(h[1]);
            d[2] = (uint16_t)xr;
        }
    }
}

__device__ __forceinline__ void store_conv_state(const GdnArgs &a, int b, int c, const float h[3]) {
    uint16_t *d = a.conv_out + ((size_t)b * a.C + c) * (KC - 1);
    d[0] = (uint16_t)qs::f2bf(h[0]);
    d[1] = (uint16_t)qs::f2bf(h[1]);
    d[2] = (uint16_t)qs::f2bf(h[2]);
}

// Sum of p[0..3] (this thread's 4 columns) over the 32 row groups: lane butterfly over the 8 row groups of
// the wave (lane bits 3..5), then the 4 waves through LDS in a fixed order.
__device__ __forceinline__ void reduce_cols(float p[4], float (*red)[SLAB], float out[4], int lane, int w,
                                            int cg) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        p[j] += qs::dpp<0x128>(p[j]);  // xor 8 (row_ror:8)
        p[j] += __shfl_xor(p[j], 16, 64);
        p[j] += __shfl_xor(p[j], 32, 64);
    }
    if (lane < 8) {
#pragma unroll
        for (int j = 0; j < 4; ++j) red[w][lane * 4 + j] = p[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int col = cg * 4 + j;
        out[j] = (red[0][col] + red[1][col]) + (red[2][col] + red[3][col]);
    }
}

template <bool CONV, bool VERIFY>
__global__ __launch_bounds__(THREADS) void gdn_kernel(GdnArgs a) {
    const int nwg = a.B * a.NV * NSLAB;
    const int lid = qs::xcd_logical(blockIdx.x, nwg);
    const int s = lid % NSLAB;
    const int h = (lid / NSLAB) % a.NV;
    const int b = lid / (NSLAB * a.NV);
    const int rep = a.NV / a.NK;
    const int kh = h / rep;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int cg = tid & 7, rg = tid >> 3;
    const int T = VERIFY ? a.T : 1;
    const bool kq_owner = (h % rep == 0) && (s == 0);  // writes the shared q/k channel outputs

    __shared__ float s_qn[TMAX][DK];
    __shared__ float s_kn[TMAX][DK];
    __shared__ float s_v[TMAX][SLAB];
    __shared__ float s_red[2][4][SLAB];
    __shared__ int s_last;

    // 1. The small conv inputs first, then the state slab: the slab's latency overlaps the prologue.
    constexpr int TM = VERIFY ? TMAX : 1;
    const int qd = a.NK * DK;
    const bool isq = tid < DK;
    const int c = isq ? kh * DK + tid : qd + kh * DK + (tid - DK);
    const int cv = 2 * qd + h * DV + s * SLAB + tid;
    ConvIn<TM> cq, cvin;
    if (CONV) {
        cq = conv_load<TM>(a, b, c, T);
        if (tid < SLAB) cvin = conv_load<TM>(a, b, cv, T);
    }
    const size_t head = (size_t)(b * a.NV + h) * DK * DV;
    const float *sp = a.s_in + head + s * SLAB + cg * 4;
    f32x4 S[4];  // streamed once per step: nontemporal loads and stores keep it from thrashing L2 / MALL
#pragma unroll
    for (int i = 0; i < 4; ++i) S[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(sp + (size_t)(rg + 32 * i) * DV));
    // the gates of every token, requested with the rest so no load waits later in the chain
    float gdec[TM], gbeta[TM];
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        if (t < T) {
            const int gi = ((b * T) + t) * a.NV + h;
            gdec[t] = a.g[gi];
            gbeta[t] = a.beta[gi];
        }
    }

    // 2. Prologue: q, k of key head kh and the v slab, for every token.
    if (CONV) {
        conv_run<VERIFY>(a, cq, b, c, T, isq ? &s_qn[0][tid] : &s_kn[0][tid - DK], DK, kq_owner);
        if (tid < SLAB) conv_run<VERIFY>(a, cvin, b, cv, T, &s_v[0][tid], SLAB, true);
        // v channels of this slab are read by this workgroup only: shift them in place now.
        if (!VERIFY && tid < SLAB) store_conv_state(a, b, cv, cvin.h);
    } else {
        for (int t = 0; t < T; ++t) {
            const size_t qk = (((size_t)b * T + t) * a.NK + kh) * DK;
            if (tid < DK)
                s_qn[t][tid] = qs::bf2f(a.q[qk + tid]);
            else
                s_kn[t][tid - DK] = qs::bf2f(a.k[qk + tid - DK]);
            if (tid < SLAB) s_v[t][tid] = qs::bf2f(a.v[(((size_t)b * T + t) * a.NV + h) * DV + s * SLAB + tid]);
        }
    }
    __syncthreads();
    // q/k conv channels are read by the rep * NSLAB workgroups of key head kh. Each counts itself in after
    // the barrier above (its reads are consumed); the last to arrive writes the shifted state at the end
    // and re-arms the counter. The count's return is only waited for at the end.
    int arrived = 0;
    if (CONV && !VERIFY && tid == 0) arrived = atomicAdd(a.counters + b * a.NK + kh, 1);

    // 3. L2 norms (q times scale): wave w normalises vectors w, w + 4, ... of (q_0, k_0, q_1, k_1, ...).
    for (int j = w; j < 2 * T; j += 4) {
        float *vec = (j & 1) ? s_kn[j >> 1] : s_qn[j >> 1];
        const float x0 = vec[lane], x1 = vec[lane + 64];
        const float r = rsqrtf(qs::wave_sum_dpp(x0 * x0 + x1 * x1) + a.eps);
        const float f = (j & 1) ? 1.0f : a.scale;
        vec[lane] = x0 * r * f;
        vec[lane + 64] = x1 * r * f;
    }
    __syncthreads();

    // 4. Delta rule, token by token, on the slab held in registers.
    for (int t = 0; t < T; ++t) {
        const int gi = ((b * T) + t) * a.NV + h;
        const float decay = expf(gdec[t]);
        const float bt = gbeta[t];
        float kn[4], qn[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            kn[i] = s_kn[t][rg + 32 * i];
            qn[i] = s_qn[t][rg + 32 * i];
        }
        float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float kd = decay * kn[i];
            p[0] = fmaf(kd, S[i].x, p[0]);
            p[1] = fmaf(kd, S[i].y, p[1]);
            p[2] = fmaf(kd, S[i].z, p[2]);
            p[3] = fmaf(kd, S[i].w, p[3]);
        }
        float ks[4];
        reduce_cols(p, s_red[0], ks, lane, w, cg);
        float dl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) dl[j] = bt * (s_v[t][cg * 4 + j] - ks[j]);
        float po[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            S[i].x = fmaf(kn[i], dl[0], decay * S[i].x);
            S[i].y = fmaf(kn[i], dl[1], decay * S[i].y);
            S[i].z = fmaf(kn[i], dl[2], decay * S[i].z);
            S[i].w = fmaf(kn[i], dl[3], decay * S[i].w);
            po[0] = fmaf(qn[i], S[i].x, po[0]);
            po[1] = fmaf(qn[i], S[i].y, po[1]);
            po[2] = fmaf(qn[i], S[i].z, po[2]);
            po[3] = fmaf(qn[i], S[i].w, po[3]);
        }
        float* dst = VERIFY ? a.s_out + (size_t)t * a.B * a.NV * DK * DV + head + s * SLAB + cg * 4
                            : a.s_out + head + s * SLAB + cg * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) __builtin_nontemporal_store(S[i], reinterpret_cast<f32x4 *>(dst + (size_t)(rg + 32 * i) * DV));
        float ov[4];
        reduce_cols(po, s_red[1], ov, lane, w, cg);
        if (tid < 8) {
            uint2 pk;
            pk.x = qs::pack_bf2(ov[0], ov[1]);
            pk.y = qs::pack_bf2(ov[2], ov[3]);
            *reinterpret_cast<uint2 *>(a.o + (size_t)gi * DV + s * SLAB + cg * 4) = pk;
        }
    }
    if (CONV && !VERIFY) {
        if (tid == 0) {
            const int last = arrived == rep * NSLAB - 1;
            if (last) atomicExch(a.counters + b * a.NK + kh, 0);
            s_last = last;
        }
        __syncthreads();
        if (s_last) store_conv_state(a, b, c, cq.h);
    }
}

// -------------------------------------------------------------------------------------------- conv1d alone

__global__ __launch_bounds__(256) void conv1d_update_kernel(const uint16_t *x, uint16_t *cs, const uint16_t *taps,
                                                            uint16_t *y, int B, int C) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= B * C) return;
    const int c = i % C;
    uint16_t *st = cs + (size_t)i * (KC - 1);
    const float h0 = qs::bf2f(st[0]), h1 = qs::bf2f(st[1]), h2 = qs::bf2f(st[2]);
    const uint32_t xr = x[i];
    const float xt = qs::bf2f(xr);
    const uint2 tw = *reinterpret_cast<const uint2 *>(taps + (size_t)c * KC);
    float acc = h0 * qs::bf_lo(tw.x);
    acc = acc + h1 * qs::bf_hi(tw.x);
    acc = acc + h2 * qs::bf_lo(tw.y);
    acc = acc + xt * qs::bf_hi(tw.y);
    y[i] = (uint16_t)qs::f2bf(qs::silu(acc));
    st[0] = st[1];
    st[1] = st[2];
    st[2] = (uint16_t)xr;
}

// -------------------------------------------------------------------------------------------- gates

__global__ __launch_bounds__(256) void gates_kernel(const uint16_t *a, const uint16_t *bb, const float *dt,
                                                    const float *neg_a, float *g, float *beta, int B, int NV) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= B * NV) return;
    const int h = i % NV;
    const float z = qs::bf2f(a[i]) + dt[h];
    const float sp = z > 20.0f ? z : log1pf(expf(z));
    g[i] = neg_a[h] * sp;
    beta[i] = 1.0f / (1.0f + expf(-qs::bf2f(bb[i])));
}

// -------------------------------------------------------------------------------------------- rollback

// grid (chunks, B): the chunks of user b copy its state snapshot and its conv-state snapshot in 16-byte
// units (2-byte units when the conv state is not a multiple of 16 bytes); chunk 0 also sets the new
// sequence length. accept_len outside [1, T] leaves the user untouched.
__global__ __launch_bounds__(256) void rollback_kernel(const float *states_out, float *state,
                                                       const uint16_t *conv_states_out, uint16_t *conv_state,
                                                       const int *accept, int *seq_lens, const int *base_lens,
                                                       int B, int T, size_t state_f4, size_t conv_elems) {
    const int b = blockIdx.y;
    const int acc = accept[b];
    if (acc < 1 || acc > T) return;
    const size_t slot = (size_t)(acc - 1) * B + b;
    const size_t stride = (size_t)gridDim.x * 256, i0 = (size_t)blockIdx.x * 256 + threadIdx.x;
    const float4 *src = reinterpret_cast<const float4 *>(states_out) + slot * state_f4;
    float4 *dst = reinterpret_cast<float4 *>(state) + (size_t)b * state_f4;
    for (size_t i = i0; i < state_f4; i += stride) dst[i] = src[i];
    const uint16_t *cs = conv_states_out + slot * conv_elems;
    uint16_t *cd = conv_state + (size_t)b * conv_elems;
    if (conv_elems % 8 == 0) {
        const uint4 *cs4 = reinterpret_cast<const uint4 *>(cs);
        uint4 *cd4 = reinterpret_cast<uint4 *>(cd);
        for (size_t i = i0; i < conv_elems / 8; i += stride) cd4[i] = cs4[i];
    } else {
        for (size_t i = i0; i < conv_elems; i += stride) cd[i] = cs[i];
    }
    if (blockIdx.x == 0 && threadIdx.x == 0 && seq_lens) seq_lens[b] = base_lens[b] + acc;
}

int check_gdn_shapes(int B, int NK, int NV, int DKa, int DVa) {
    QS_REQUIRE(B > 0, "B must be positive (got %d)", B);
    QS_REQUIRE(DKa == DK && DVa == DV, "DK and DV must be 128 (got %d, %d)", DKa, DVa);
    QS_REQUIRE(NK > 0 && NV > 0 && NV % NK == 0, "NV (%d) must be a positive multiple of NK (%d)", NV, NK);
    QS_REQUIRE((long)B * NV * NSLAB < (1L << 31), "grid too large");
    return QS_OK;
}

}  // namespace

extern "C" int qs_conv1d_update(const uint16_t *x, uint16_t *conv_state, const uint16_t *taps, uint16_t *y, int B,
                                int C, int K, void *stream) {
    QS_REQUIRE(x && conv_state && taps && y, "qs_conv1d_update: null pointer");
    QS_REQUIRE(B > 0 && C > 0, "qs_conv1d_update: B and C must be positive (got %d, %d)", B, C);
    QS_REQUIRE(K == KC, "qs_conv1d_update: only K = 4 taps are supported (got %d)", K);
    const int n = B * C;
    conv1d_update_kernel<<<(n + 255) / 256, 256, 0, QS_STREAM(stream)>>>(x, conv_state, taps, y, B, C);
    return qs::launch_status("qs_conv1d_update");
}

extern "C" int qs_gdn_gates(const uint16_t *a, const uint16_t *b, const float *dt_bias, const float *neg_a, float *g,
                            float *beta, int B, int NV, void *stream) {
    QS_REQUIRE(a && b && dt_bias && neg_a && g && beta, "qs_gdn_gates: null pointer");
    QS_REQUIRE(B > 0 && NV > 0, "qs_gdn_gates: B and NV must be positive");
    gates_kernel<<<(B * NV + 255) / 256, 256, 0, QS_STREAM(stream)>>>(a, b, dt_bias, neg_a, g, beta, B, NV);
    return qs::launch_status("qs_gdn_gates");
}

extern "C" int qs_gdn_decode_step(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *g,
                                  const float *beta, float *state, uint16_t *o, int B, int NK, int NV, int DKa,
                                  int DVa, float scale, float eps, void *stream) {
    QS_REQUIRE(q && k && v && g && beta && state && o, "qs_gdn_decode_step: null pointer");
    if (int e = check_gdn_shapes(B, NK, NV, DKa, DVa)) return e;
    GdnArgs a{};
    a.q = q, a.k = k, a.v = v, a.g = g, a.beta = beta, a.s_in = state, a.s_out = state, a.o = o;
    a.B = B, a.T = 1, a.NK = NK, a.NV = NV, a.C = 2 * NK * DK + NV * DV, a.scale = scale, a.eps = eps;
    gdn_kernel<false, false><<<B * NV * NSLAB, THREADS, 0, QS_STREAM(stream)>>>(a);
    return qs::launch_status("qs_gdn_decode_step");
}

extern "C" size_t qs_gdn_workspace_bytes(int B, int NK) { return (size_t)(B > 0 ? B : 0) * (NK > 0 ? NK : 0) * 4; }

extern "C" int qs_gdn_decode_fused(const uint16_t *x, uint16_t *conv_state, const uint16_t *taps, const float *g,
                                   const float *beta, float *state, uint16_t *o, uint16_t *y_out, void *workspace,
                                   int B, int NK, int NV, int DKa, int DVa, int K, float scale, float eps,
                                   void *stream) {
    QS_REQUIRE(x && conv_state && taps && g && beta && state && o && workspace,
               "qs_gdn_decode_fused: null pointer");
    if (int e = check_gdn_shapes(B, NK, NV, DKa, DVa)) return e;
    QS_REQUIRE(K == KC, "qs_gdn_decode_fused: only K = 4 taps are supported (got %d)", K);
    GdnArgs a{};
    a.x = x, a.conv_in = conv_state, a.conv_out = conv_state, a.taps = taps, a.y_out = y_out;
    a.g = g, a.beta = beta, a.s_in = state, a.s_out = state, a.o = o;
    a.counters = static_cast<int *>(workspace);
    a.B = B, a.T = 1, a.NK = NK, a.NV = NV, a.C = 2 * NK * DK + NV * DV, a.scale = scale, a.eps = eps;
    gdn_kernel<true, false><<<B * NV * NSLAB, THREADS, 0, QS_STREAM(stream)>>>(a);
    return qs::launch_status("qs_gdn_decode_fused");
}

extern "C" int qs_gdn_verify_step(const uint16_t *x, const uint16_t *conv_state_in, uint16_t *conv_states_out,
                                  const uint16_t *taps, const float *g, const float *beta, const float *state_in,
                                  float *states_out, uint16_t *o, uint16_t *y_out, int B, int T, int NK, int NV,
                                  int DKa, int DVa, int K, float scale, float eps, void *stream) {
    QS_REQUIRE(x && conv_state_in && conv_states_out && taps && g && beta && state_in && states_out && o,
               "qs_gdn_verify_step: null pointer");
    if (int e = check_gdn_shapes(B, NK, NV, DKa, DVa)) return e;
    QS_REQUIRE(T >= 1 && T <= TMAX, "qs_gdn_verify_step: T must be in [1, %d] (got %d)", TMAX, T);
    QS_REQUIRE(K == KC, "qs_gdn_verify_step: only K = 4 taps are supported (got %d)", K);
    QS_REQUIRE(states_out != state_in, "qs_gdn_verify_step: states_out must not alias state_in");
    GdnArgs a{};
    a.x = x, a.conv_in = conv_state_in, a.conv_out = conv_states_out, a.taps = taps, a.y_out = y_out;
    a.g = g, a.beta = beta, a.s_in = state_in, a.s_out = states_out, a.o = o;
    a.B = B, a.T = T, a.NK = NK, a.NV = NV, a.C = 2 * NK * DK + NV * DV, a.scale = scale, a.eps = eps;
    gdn_kernel<true, true><<<B * NV * NSLAB, THREADS, 0, QS_STREAM(stream)>>>(a);
    return qs::launch_status("qs_gdn_verify_step");
}

extern "C" int qs_gdn_rollback(const float *states_out, float *state, const uint16_t *conv_states_out,
                               uint16_t *conv_state, const int *accept_len, int *seq_lens, const int *base_lens,
                               int B, int T, int NV, int DKa, int DVa, int C, int K, void *stream) {
    QS_REQUIRE(states_out && state && conv_states_out && conv_state && accept_len, "qs_gdn_rollback: null pointer");
    QS_REQUIRE(!seq_lens || base_lens, "qs_gdn_rollback: seq_lens needs base_lens");
    QS_REQUIRE(B > 0 && T >= 1 && T <= TMAX && NV > 0 && C > 0 && K == KC, "qs_gdn_rollback: bad shape");
    QS_REQUIRE(DKa == DK && DVa == DV, "qs_gdn_rollback: DK and DV must be 128");
    const size_t state_f4 = (size_t)NV * DK * DV / 4;
    const size_t conv_elems = (size_t)C * (K - 1);
    const int chunks = (int)((state_f4 + 255) / 256 < 256 ? (state_f4 + 255) / 256 : 256);
    rollback_kernel<<<dim3(chunks, B), 256, 0, QS_STREAM(stream)>>>(states_out, state, conv_states_out, conv_state,
                                                                    accept_len, seq_lens, base_lens, B, T,
                                                                    state_f4, conv_elems);
    return qs::launch_status("qs_gdn_rollback");
}
