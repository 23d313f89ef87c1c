// Gated DeltaNet decode-time state path on gfx950: conv1d update, gates, L2-norm + gated delta rule
// (decode and T-token verify) and the verify rollback.
//
// Decomposition of the delta rule. For value column v the step is column-separable:
//     delta_v = beta (v_v - e^g sum_k k_k S_kv),  S'_kv = e^g S_kv + k_k delta_v,  o_v = sum_k q_k S'_kv
// so the unit is a 128 x 32 slab S[:, 32 s .. 32 s + 31] of one (user, value head), 4 slabs per head.
// At large batch one wavefront owns a slab (the slab waves of a workgroup share the key head's q/k conv):
// lane (rg = lane / 8, cg = lane % 8) holds rows rg + 8 i (i < 16), columns 4 cg .. 4 cg + 3 in 64 VGPRs,
// each dwordx4 load or store instruction covers 8 full 128-byte rows, and the k-reductions (S^T k and
// S^T q) sum a lane's rows in registers, then the row groups (lane bits 3..5) with one DPP step and two lane
// swaps in a fixed order (bit-reproducible run to run), with no workgroup barrier. At small batch a slab's
// rows are split over 4 waves; per token each wave reduce-scatters its column sums and the waves add them
// through LDS behind one barrier. The state is read once and written once per token.
#include <mutex>

#include "qs_common.h"

namespace {

constexpr int DK = 128;
constexpr int DV = 128;
constexpr int KC = 4;  // conv taps
constexpr int TMAX = 8;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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
    int *counters;              // decode + conv: [B, NK, 2] (q, k) self-resetting
    const int *in_slot;         // verify, nullable: [B] slot of s_in / conv_in holding user b's input
    const int *lens;            // nullable: [B]; a user with lens[b] < 0 is an idle slot (decode: left untouched;
                                // verify: no token verified, slot mode carries its input slot forward)
    int n_slots;                // slots in s_in / conv_in
    const uint16_t *z;          // decode, nullable: the projection's z rows (row b at z + b ldz), for the gated
    int ldz;                    // RMSNorm epilogue o <- bf16(rmsnorm(o) norm_w silu(z)) per value head
    const float *norm_w;        // [DV]
    int B, T, NK, NV, C;
    float scale, eps;
};

// Inputs of the causal conv of two adjacent channels (c, c + 1), as loaded (bf16 bits): their K-1 history
// values (12 contiguous bytes: c's three, then c + 1's), their taps (16 bytes) and x of both for every token
// (4 bytes per token). Three wide loads per pair instead of ten narrow ones; nothing reads them until
// conv_run, so no wait sits between them and the state loads issued after.
template <int TM>
struct ConvPair {
    u32x3 h;
    uint4 tw;
    uint32_t x[TM];
};

template <int TM>
__device__ __forceinline__ ConvPair<TM> conv_load(const GdnArgs &a, const uint16_t *conv_b, int b, int c, int T) {
    ConvPair<TM> in;
    in.h = *reinterpret_cast<const u32x3 *>(conv_b + (size_t)c * (KC - 1));
    in.tw = *reinterpret_cast<const uint4 *>(a.taps + (size_t)c * KC);
#pragma unroll
    for (int t = 0; t < TM; ++t)  // tokens past T repeat token 0 (in range; their results are never used)
        in.x[t] = *reinterpret_cast<const uint32_t *>(a.x + ((size_t)b * T + (t < T ? t : 0)) * a.C + c);
    return in;
}

// The 3 + T inputs of channel e (0: c, 1: c + 1) in time order: history, then x_0 .. x_{T-1}.
template <int TM>
__device__ __forceinline__ uint32_t conv_seq(const ConvPair<TM> &in, int e, int i) {
    if (i < 3) {
        const int k = 3 * e + i;  // half-word index into the 12 history bytes
        const uint32_t w = k < 2 ? in.h.x : (k < 4 ? in.h.y : in.h.z);
        return (k & 1) ? w >> 16 : w & 0xffffu;
    }
    return e ? in.x[i - 3] >> 16 : in.x[i - 3] & 0xffffu;
}

// Conv1d + SiLU of the pair over T tokens (window oldest first, tap 0 on the oldest input). The tap
// products of two bf16 values are exact in fp32, so fused or unfused multiply-adds round identically.
// y[e][t] receives the bf16-rounded outputs as fp32, yb[t] their bits packed (c | c + 1 << 16).
template <int TM>
__device__ __forceinline__ void conv_run(const ConvPair<TM> &in, int T, float y[2][TM], uint32_t yb[TM]) {
    float sv[2][TM];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint32_t tw0 = e ? in.tw.z : in.tw.x, tw1 = e ? in.tw.w : in.tw.y;
        const float w0 = qs::bf_lo(tw0), w1 = qs::bf_hi(tw0), w2 = qs::bf_lo(tw1), w3 = qs::bf_hi(tw1);
        float h0 = qs::bf2f(conv_seq(in, e, 0)), h1 = qs::bf2f(conv_seq(in, e, 1)), h2 = qs::bf2f(conv_seq(in, e, 2));
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            const float xt = qs::bf2f(conv_seq(in, e, 3 + t));
            float acc = h0 * w0;
            acc = acc + h1 * w1;
            acc = acc + h2 * w2;
            acc = acc + xt * w3;
            sv[e][t] = qs::silu(acc);
            h0 = h1;
            h1 = h2;
            h2 = xt;
        }
    }
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        yb[t] = qs::cvt_pk_bf16(sv[0][t], sv[1][t]);
        y[0][t] = qs::bf_lo(yb[t]);
        y[1][t] = qs::bf_hi(yb[t]);
    }
}

// The pair's global outputs, issued once the state loads have been consumed: the conv outputs (y_out,
// when given and write_y) and, with write_state, every token's window (SNAP: verify snapshots, slot t of
// conv_out) or the final window in place (decode). Windows are runs of the input sequence, all bf16
// already, so they are copied as bits: window after token t = inputs t + 1 .. t + 3 of each channel.
template <bool SNAP, int TM>
__device__ __forceinline__ void conv_commit(const GdnArgs &a, const ConvPair<TM> &in, const uint32_t yb[TM], int b,
                                            int c, int T, bool write_y, bool write_state) {
    auto window = [&](int t) {
        u32x3 w;
        w.x = conv_seq(in, 0, t + 1) | (conv_seq(in, 0, t + 2) << 16);
        w.y = conv_seq(in, 0, t + 3) | (conv_seq(in, 1, t + 1) << 16);
        w.z = conv_seq(in, 1, t + 2) | (conv_seq(in, 1, t + 3) << 16);
        return w;
    };
    if constexpr (SNAP) {
        // verify: buffer stores, the lane's offset once and the token's as a scalar; a lane that writes nothing
        // stores past the descriptor's range (dropped), so no branch surrounds the stores (T y values and T
        // snapshots per lane: ~4.5 us less per 4-token verify step than global stores with their addresses)
        const int ybytes = a.y_out ? a.B * T * a.C * 2 : 0;
        const auto ry = __builtin_amdgcn_make_buffer_rsrc(a.y_out, (short)0, ybytes, 0x00020000);
        const int sbytes = T * a.B * a.C * (KC - 1) * 2;
        const auto rs = __builtin_amdgcn_make_buffer_rsrc(a.conv_out, (short)0, sbytes, 0x00020000);
        const int yo = write_y ? (b * T * a.C + c) * 2 : ybytes;
        const int so = write_state ? (b * a.C + c) * (KC - 1) * 2 : sbytes;
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            if (t >= T) break;
            __builtin_amdgcn_raw_buffer_store_b32(yb[t], ry, yo, t * a.C * 2, 0);
            __builtin_amdgcn_raw_buffer_store_b96(window(t), rs, so, t * a.B * a.C * (KC - 1) * 2, 0);
        }
    } else {  // decode: T == 1, the window after x_0
        if (write_y && a.y_out) *reinterpret_cast<uint32_t *>(a.y_out + (size_t)b * a.C + c) = yb[0];
        if (write_state) *reinterpret_cast<u32x3 *>(a.conv_out + ((size_t)b * a.C + c) * (KC - 1)) = window(0);
    }
}

// Sum over the row groups of a slab wave (lane bits log2(CG) .. 5) as a butterfly in a fixed order: every
// lane ends with bit-identical sums of its column group.
template <int CG>
__device__ __forceinline__ float sum_row_groups(float x) {
    if (CG == 4) x += __shfl_xor(x, 4, 64);
    x += qs::dpp<0x128>(x);  // xor 8 (row_ror:8)
    x = qs::xor16_sum(x);
    x = qs::xor32_sum(x);
    return x;
}

// The small-batch form's column sums (CG = 8) as a reduce-scatter, since the waves' exchange through LDS
// gathers whole columns afterwards anyway: the 8 partial sums of a lane (p and r of its 4 columns) are halved
// across lane bit 4 by v_permlane16_swap of two different values (the lower row of each pair keeps the first
// value's pair sum, the upper row the second's), then across bit 5 by v_permlane32_swap, and the last two are
// summed across bit 3 on DPP. Lane (cg, bits 3-5) ends with p and r of column 4 cg + 2 (bit 5) + (bit 4) over
// all 8 row groups, in a fixed order; 14 cross-lane operations and adds instead of 40 for full sums.
__device__ __forceinline__ float pair_sum16(float a, float b) {
    const auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(x[0]) + __uint_as_float(x[1]);
}
__device__ __forceinline__ float pair_sum32(float a, float b) {
    const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(x[0]) + __uint_as_float(x[1]);
}
__device__ __forceinline__ void scatter_sums8(const float (&p)[4], const float (&r)[4], float &ps, float &rs) {
    const float tp0 = pair_sum16(p[0], p[1]), tp1 = pair_sum16(p[2], p[3]);
    const float tr0 = pair_sum16(r[0], r[1]), tr1 = pair_sum16(r[2], r[3]);
    const float up = pair_sum32(tp0, tp1), ur = pair_sum32(tr0, tr1);
    ps = up + qs::dpp<0x128>(up);  // xor 8 (row_ror:8)
    rs = ur + qs::dpp<0x128>(ur);
}

// First state element of lane (cg, row) of slab s of value head h in user slot `user` of s_in.
template <int SLAB>
__device__ __forceinline__ const float *sp_of_t(const GdnArgs &a, size_t user, int h, int s, int cg, int row) {
    return a.s_in + (user * a.NV + h) * DK * DV + s * SLAB + cg * 4 + (size_t)row * DV;
}

// One workgroup of NW wavefronts per (user, value head, SLAB-column slab); wave w holds rows
// w * RW .. (w + 1) * RW - 1 (RW = 128 / NW) of the slab, lane (rg = lane / CG, cg = lane % CG) rows
// w * RW + rg + RG i (i < RPL), columns 4 cg .. 4 cg + 3. NW = 1 at large batch (each wave streams a
// 16 KB slab); NW = 4 when one wave per slab would leave the chip underfilled (small batch), which also
// spreads the conv prologue over three waves and cuts the serial work per token by 4, for one LDS
// exchange per token.
// Per token both column reductions are taken from the state before the update, in one pass:
//     p_v = sum_k k_k S_kv,  r_v = sum_k q_k S_kv,  delta_v = beta (v_v - e^g p_v)
//     S'_kv = e^g S_kv + k_k delta_v,  o_v = q^T S'_v = e^g r_v + (q . k) delta_v
// so the update and the stores of S' follow the reduction with no second reduction in between.
// The conv: q channels 2 lane, 2 lane + 1 of key head kh on wave WQ, the same k channels on wave WK, the
// slab's v channels 2 (lane % (SLAB / 2)), + 1 on wave WV (all wave 0 when NW = 1).
// Memory order: every load is issued first (the user's length and, in a verify step, its input slot; then the
// conv inputs, the state and the gates as scalar loads); the idle-slot exit comes after those requests; no
// global store is issued before the state loads are consumed, because vmcnt counts loads and stores
// together and a store in flight would turn each wait for a state load into a wait for everything. The
// decode's arrival count (an atomic returning its value, counted like a load) is the one exception: it
// leaves after the conv, behind the state loads, and is waited for only at the end.
// in_slot (verify only, nullable): user b's input state and conv state are slot in_slot[b] of s_in and
// conv_in ([n_slots, B, ...]); a slot outside [0, n_slots) reads slot 0.
// NORM (decode, WPG == NSLAB: a workgroup holds the 4 slabs of one value head): the gated RMSNorm epilogue of
// the mixer (model.py:274-275, the head cores' steps 7-8, kernels/gdn_head_compute.cpp:320-346) on the fp32 o
// of the head: the slabs' sums of squares meet in LDS (one barrier per token) and o receives
// bf16(o rsqrt(mean(o^2) + eps) norm_w silu(z)).
template <bool CONV, bool VERIFY, int TM, int SLAB, int NW, int WPG, bool NORM = false>
__global__ __launch_bounds__(64 * NW * WPG) void gdn_kernel(GdnArgs a) {
    constexpr int NSLAB = DV / SLAB;
    constexpr int CG = SLAB / 4;   // column groups of 4 (lane % CG)
    constexpr int RG = 64 / CG;    // row groups (lane / CG)
    constexpr int RW = DK / NW;    // rows per wave
    constexpr int RPL = RW / RG;   // rows per lane
    static_assert(RPL >= 1 && RW % RG == 0 && (VERIFY || TM == 1), "slab shape");
    static_assert(!NORM || (!VERIFY && WPG == NSLAB && CG <= 16), "the epilogue needs whole heads per workgroup");
    // conv roles by wave of the workgroup: q channels on wave 0, k on wave 1 (when there is one), the slab's v
    // channels on wave 2 (NW = 4) or on every wave for its own slab (NW = 1)
    constexpr int WK = (NW >= 4 || WPG >= 2) ? 1 : 0;
    constexpr int WV = NW >= 4 ? 2 : NW - 1;
    // the wave that writes o (and forms each token's q . k for it): the slab's last wave, which reaches each
    // token's exchange first; wave 0, which also runs the q conv, was the last with o on its path as well
    constexpr int WO = NW - 1;
    // The one-wave-per-slab form: the load addresses' kernel arguments, requested with the first batch of
    // argument loads (the compiler would otherwise request them after the index arithmetic below, a second
    // round trip before the first load; the other forms already request them in one batch, and the fence
    // measured slower there)
    if constexpr (NW == 1)
        asm volatile("" ::"s"(a.x), "s"(a.conv_in), "s"(a.taps), "s"(a.g), "s"(a.beta), "s"(a.s_in), "s"(a.lens),
                     "s"(a.in_slot), "s"(a.q), "s"(a.k), "s"(a.v));
    // WPG slab units per workgroup, NW waves each: unit = logical workgroup x WPG + gw
    const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave within the workgroup (uniform)
    const int gw = WPG > 1 ? wid / NW : 0;        // slab unit within the workgroup
    const int nwg = a.B * a.NV * NSLAB / WPG;
    const int lid = qs::xcd_logical(blockIdx.x, nwg) * WPG + gw;
    const int s = lid % NSLAB;
    const int h = (lid / NSLAB) % a.NV;
    const int b = lid / (NSLAB * a.NV);
    // The user's length (idle slots are negative) and, in a verify step, its input slot, requested together
    // before any other load (an empty range reads 0 when the array is not given): decode checks the length once
    // its other loads are requested; a verify step needs the slot for its addresses, one round trip for both.
    auto user_int = [&](const int *p) {
        return (int)__builtin_amdgcn_raw_buffer_load_b32(
            __builtin_amdgcn_make_buffer_rsrc(const_cast<int *>(p), (short)0, p ? a.B * 4 : 0, 0x00020000), b * 4, 0, 0);
    };
    const int lb = user_int(a.lens);
    const int slot_in = VERIFY ? user_int(a.in_slot) : 0;
    const int rep = a.NV / a.NK;
    const int kh = h / rep;
    const int lane = threadIdx.x & 63;
    const int w = NW > 1 ? wid % NW : 0;  // wave within the slab
    const int r = wid;
    const bool isq = r == 0, isk = r == WK, isv = NW > 1 ? w == WV : true;
    const int cg = lane % CG, rg = lane / CG;
    const int T = VERIFY ? a.T : 1;
    // the workgroup's slab units share key head kh (rep * NSLAB units per key head, a multiple of WPG); the
    // workgroup holding its first unit writes the shared q/k channel outputs
    const int u0 = lid - gw;
    const bool kq_owner = ((u0 / NSLAB) % a.NV) % rep == 0 && u0 % NSLAB == 0;
    const int slot = VERIFY && slot_in >= 0 && slot_in < a.n_slots ? slot_in : 0;
    const size_t user_in = (size_t)slot * a.B + b;  // this user's input in s_in / conv_in

    // q / k normalised per token, row r = w' RW + g + RG i stored at w' RW + g RPL + i: lane rg of wave w
    // reads its RPL rows as contiguous pieces
    __shared__ __align__(16) float s_qn[TM][DK];
    __shared__ __align__(16) float s_kn[TM][DK];
    __shared__ __align__(16) float s_v_[WPG][TM][SLAB];
    auto &s_v = s_v_[gw];
    __shared__ __align__(16) f32x4 s_red_[NW > 1 ? 2 : 1][WPG][NW][2][CG];  // per token parity: wave column sums
    __shared__ float s_nrm[2][WPG];  // NORM, per token parity: the slabs' sums of o^2
    __shared__ float s_qk_[WPG][TM];  // q . k of every token of the unit

    // the q / k conv waves of a multi-slab workgroup issue first: their conv inputs then leave ahead of the other
    // waves' state loads and the norms every slab waits for are ready sooner (the 64-layer batch-8 step:
    // 936.5 -> 928.5 us; at batch 1, with the rows of a slab split over 4 waves, it measured slower)
    if (CONV && NW == 1 && (isq || isk)) __builtin_amdgcn_s_setprio(2);
    // 1. Loads. Conv inputs (raw bits, untouched until used), this wave's state rows, the gates.
    const int qd = a.NK * DK;
    const int cq = kh * DK + 2 * lane, ck = qd + cq;                           // q, k channel pairs
    const int cv = 2 * qd + h * DV + s * SLAB + 2 * (lane & (SLAB / 2 - 1));  // v channel pair
    const uint16_t *conv_b = CONV ? a.conv_in + user_in * a.C * (KC - 1) : nullptr;
    if (VERIFY && lb < 0) {
        // An idle slot (uniform over the workgroup, whose units belong to one user): no token is verified and
        // no output written. In slot mode its input is carried unchanged into the same slot of the output
        // set, which is the set the next step reads after the acceptance left this user's slot as it was;
        // in copy mode the caller's state is not touched at all.
        if (a.in_slot && slot < a.T) {
            const size_t out_b = (size_t)slot * a.B + b;
            float *dp = a.s_out + (out_b * a.NV + h) * DK * DV + s * SLAB + cg * 4 + (size_t)(w * RW + rg) * DV;
#pragma unroll
            for (int i = 0; i < RPL; ++i)
                *reinterpret_cast<f32x4 *>(dp + (size_t)(RG * i) * DV) =
                    *reinterpret_cast<const f32x4 *>(sp_of_t<SLAB>(a, user_in, h, s, cg, w * RW + rg) + (size_t)(RG * i) * DV);
            if (CONV) {
                uint16_t *co = a.conv_out + out_b * a.C * (KC - 1);
                auto carry = [&](int c) {
                    *reinterpret_cast<u32x3 *>(co + (size_t)c * (KC - 1)) =
                        *reinterpret_cast<const u32x3 *>(conv_b + (size_t)c * (KC - 1));
                };
                if (isv && lane < SLAB / 2) carry(cv);
                if (isq && kq_owner) carry(cq);
                if (isk && kq_owner) carry(ck);
            }
        }
        return;
    }
    ConvPair<TM> inq, ink, inv;
    // Decode + conv: the waves holding the q/k channels count themselves in once their history is consumed.
    // Every wave issues the same buffer atomic, out of range on every lane but lane 0 of the q and k waves, so
    // no branch surrounds it and the compiler's waits for the state loads leave it in flight (a conditional
    // atomic makes them wait for it). The key head's workgroup holding its first unit adds 1 - N and the others
    // 1 (N arrivals), so the count is back at zero after every launch and the arrival that brings it there is
    // the last. The small-batch form counts right after the conv, so the count's round trip overlaps the state
    // loads and the first token (batch 1: 5.15 -> 4.56 us per layer); the one-wave-per-slab form after the
    // first token's reductions (counting after the conv there measured slower at batch 8).
    int arrived = 0;  // lane 0 of the q / k waves: the count before this arrival
    auto count_in = [&]() {
        const auto rc = __builtin_amdgcn_make_buffer_rsrc(qs::uniform_ptr(a.counters + (b * a.NK + kh) * 2),
                                                          (short)0, 8, 0x00020000);
        const int off = (lane == 0 && (isq || isk)) ? (isq ? 0 : 4) : 8;
        return __builtin_amdgcn_raw_ptr_buffer_atomic_add_i32(kq_owner ? 1 - rep * NSLAB / WPG : 1, rc, off, 0, 0);
    };
    if (CONV) {
        if (isq) inq = conv_load<TM>(a, conv_b, b, cq, T);
        if (isk) ink = conv_load<TM>(a, conv_b, b, ck, T);
        if (isv) inv = conv_load<TM>(a, conv_b, b, cv, T);
    }
    const size_t head = (size_t)(b * a.NV + h) * DK * DV;
    const float *sp = sp_of_t<SLAB>(a, user_in, h, s, cg, w * RW + rg);
    f32x4 S[RPL];  // streamed once per step: nontemporal loads and stores keep it from thrashing L2 / MALL
#pragma unroll
    for (int i = 0; i < RPL; ++i)
        S[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(sp + (size_t)(RG * i) * DV));
    float gdec[TM], gbeta[TM];
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        const int gi = ((b * T) + (t < T ? t : 0)) * a.NV + h;
        gdec[t] = a.g[gi];
        gbeta[t] = a.beta[gi];
    }
    // NORM: the epilogue's z and norm_w of the lane's 4 columns, requested now (used after the last token)
    uint2 z4 = make_uint2(0, 0);
    float4 w4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (NORM && w == WO && lane < CG) {
        z4 = *reinterpret_cast<const uint2 *>(a.z + (size_t)b * a.ldz + h * DV + s * SLAB + cg * 4);
        w4 = *reinterpret_cast<const float4 *>(a.norm_w + s * SLAB + cg * 4);
    }
    // An idle slot keeps its state, conv history and output as they are. The check comes once the loads are
    // requested (they only read, within the buffers), so the length's round trip overlaps them, and waits for
    // the length alone (requested first); nothing has been stored or counted yet. The workgroup's units belong
    // to one user (a user's B NV NSLAB units are a multiple of WPG), so the exit is uniform over the workgroup.
    // The fence keeps the compiler from sinking the loads below the exit (they are dead on that path), which
    // would make them wait for the length.
    asm volatile("" ::: "memory");
    if (!VERIFY && lb < 0) return;

    // 2. q, k (rows 2 lane, 2 lane + 1) and the v slab for every token; L2 norms (q times scale).
    float qv[2][TM], kv[2][TM], vv[2][TM];
    uint32_t yq[TM], yk[TM], yv[TM];
    if (CONV) {
        if (isq) conv_run<TM>(inq, T, qv, yq);
        if (isk) conv_run<TM>(ink, T, kv, yk);
        if (isv) conv_run<TM>(inv, T, vv, yv);
        if constexpr (!VERIFY && NW > 1) arrived = count_in();
    } else {
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            if (t >= T) break;
            const size_t qk0 = (((size_t)b * T + t) * a.NK + kh) * DK + 2 * lane;
            if (isq) {
                const uint32_t q2 = *reinterpret_cast<const uint32_t *>(a.q + qk0);
                qv[0][t] = qs::bf_lo(q2), qv[1][t] = qs::bf_hi(q2);
            }
            if (isk) {
                const uint32_t k2 = *reinterpret_cast<const uint32_t *>(a.k + qk0);
                kv[0][t] = qs::bf_lo(k2), kv[1][t] = qs::bf_hi(k2);
            }
            if (isv) {
                const uint32_t v2 = *reinterpret_cast<const uint32_t *>(
                    a.v + (((size_t)b * T + t) * a.NV + h) * DV + s * SLAB + 2 * (lane & (SLAB / 2 - 1)));
                vv[0][t] = qs::bf_lo(v2), vv[1][t] = qs::bf_hi(v2);
            }
        }
    }
    {
        const int r0 = 2 * lane, rr = r0 % RW;
        const int p0 = (r0 / RW) * RW + (rr % RG) * RPL + rr / RG;  // stored position of row r0 (+ RPL: r0 + 1)
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            if (t >= T) break;
            if (isq) {
                const float rq = rsqrtf(qs::wave_sum_dpp(qv[0][t] * qv[0][t] + qv[1][t] * qv[1][t]) + a.eps) * a.scale;
                s_qn[t][p0] = qv[0][t] * rq;
                s_qn[t][p0 + RPL] = qv[1][t] * rq;
            }
            if (isk) {
                const float rk = rsqrtf(qs::wave_sum_dpp(kv[0][t] * kv[0][t] + kv[1][t] * kv[1][t]) + a.eps);
                s_kn[t][p0] = kv[0][t] * rk;
                s_kn[t][p0 + RPL] = kv[1][t] * rk;
            }
            if (isv && lane < SLAB / 2)
                *reinterpret_cast<float2 *>(&s_v[t][2 * lane]) = make_float2(vv[0][t], vv[1][t]);
        }
    }
    if (NW > 1 || WPG > 1)
        __syncthreads();
    else
        __builtin_amdgcn_wave_barrier();

    if (CONV && NW == 1 && (isq || isk)) __builtin_amdgcn_s_setprio(0);
    // q . k of every token, before the token chain (it does not depend on the state): wave w of the unit
    // forms tokens w, w + NW, ..., every lane writing the wave-uniform sum. Wave WO reads them after each
    // token's exchange barrier (with one wave per slab it reads back its own writes).
    for (int t = w; t < T; t += NW) {
        const float2 q2 = *reinterpret_cast<const float2 *>(&s_qn[t][2 * lane]);
        const float2 k2 = *reinterpret_cast<const float2 *>(&s_kn[t][2 * lane]);
        s_qk_[gw][t] = qs::wave_sum_dpp(q2.x * k2.x + q2.y * k2.y);
    }
    // 3. Delta rule, token by token, on the rows held in registers.
    for (int t = 0; t < T; ++t) {
        const int gi = ((b * T) + t) * a.NV + h;
        const float decay = expf(gdec[t]);
        const float bt = gbeta[t];
        float kn[RPL], qn[RPL];
#pragma unroll
        for (int i4 = 0; i4 < (RPL + 3) / 4; ++i4) {
            const float *kp = &s_kn[t][w * RW + rg * RPL + 4 * i4];
            const float *qp = &s_qn[t][w * RW + rg * RPL + 4 * i4];
            if constexpr (RPL >= 4) {
                const float4 k4 = *reinterpret_cast<const float4 *>(kp);
                const float4 q4 = *reinterpret_cast<const float4 *>(qp);
                kn[4 * i4] = k4.x, kn[4 * i4 + 1] = k4.y, kn[4 * i4 + 2] = k4.z, kn[4 * i4 + 3] = k4.w;
                qn[4 * i4] = q4.x, qn[4 * i4 + 1] = q4.y, qn[4 * i4 + 2] = q4.z, qn[4 * i4 + 3] = q4.w;
            } else {
#pragma unroll
                for (int j = 0; j < RPL; ++j) kn[j] = kp[j], qn[j] = qp[j];
            }
        }
        const float4 v4 = *reinterpret_cast<const float4 *>(&s_v[t][cg * 4]);
        float p[4] = {0.f, 0.f, 0.f, 0.f}, r[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            p[0] = fmaf(kn[i], S[i].x, p[0]);
            p[1] = fmaf(kn[i], S[i].y, p[1]);
            p[2] = fmaf(kn[i], S[i].z, p[2]);
            p[3] = fmaf(kn[i], S[i].w, p[3]);
            r[0] = fmaf(qn[i], S[i].x, r[0]);
            r[1] = fmaf(qn[i], S[i].y, r[1]);
            r[2] = fmaf(qn[i], S[i].z, r[2]);
            r[3] = fmaf(qn[i], S[i].w, r[3]);
        }
        if constexpr (NW == 1) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                p[j] = sum_row_groups<CG>(p[j]);
                r[j] = sum_row_groups<CG>(r[j]);
            }
        } else {
            // the wave's column sums, one column component per lane (scatter_sums8), then the waves' sums
            // added in wave order by every wave (bit-identical everywhere); two buffers by token parity, so one
            // barrier per token suffices
            static_assert(NW == 1 || CG == 8, "the reduce-scatter takes 8 column groups");
            float ps, rs;
            scatter_sums8(p, r, ps, rs);
            auto &red = s_red_[t & 1][gw];
            if (((lane >> 3) & 1) == 0) {
                const int c = ((lane >> 5) & 1) * 2 + ((lane >> 4) & 1);
                reinterpret_cast<float *>(&red[w][0][cg])[c] = ps;
                reinterpret_cast<float *>(&red[w][1][cg])[c] = rs;
            }
            __syncthreads();
            f32x4 P = red[0][0][cg], R = red[0][1][cg];
#pragma unroll
            for (int ww = 1; ww < NW; ++ww) {
                P += red[ww][0][cg];
                R += red[ww][1][cg];
            }
            p[0] = P.x, p[1] = P.y, p[2] = P.z, p[3] = P.w;
            r[0] = R.x, r[1] = R.y, r[2] = R.z, r[3] = R.w;
        }
        if (CONV && t == 0) {
            // The state loads are consumed: now the conv's global outputs. v channels of this slab belong
            // to this workgroup alone (shifted in place / snapshotted here); the q/k channels are read by
            // the rep * NSLAB workgroups of key head kh, which in decode count themselves in (q and k
            // separately when different waves hold them): the last to arrive writes the shifted state at the
            // end, where the count's return is waited for.
            if (isv) conv_commit<VERIFY, TM>(a, inv, yv, b, cv, T, lane < SLAB / 2, lane < SLAB / 2);
            if (isq) conv_commit<VERIFY, TM>(a, inq, yq, b, cq, T, kq_owner, VERIFY && kq_owner);
            if (isk) conv_commit<VERIFY, TM>(a, ink, yk, b, ck, T, kq_owner, VERIFY && kq_owner);
            if constexpr (!VERIFY && NW == 1) arrived = count_in();
        }
        float dl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) dl[j] = bt * ((&v4.x)[j] - decay * p[j]);
        // the slab's new state: streamed (nt) and written through the L2 (sc1), so the launch ends with no
        // dirty state lines left to write back (measured faster than write-back stores at batch 1 and 8)
        float *slab = qs::uniform_ptr((VERIFY ? a.s_out + (size_t)t * a.B * a.NV * DK * DV : a.s_out) + head + s * SLAB);
        const auto rs = __builtin_amdgcn_make_buffer_rsrc(slab, (short)0, DK * DV * 4, 0x00020000);
        const int soff = (cg * 4 + (w * RW + rg) * DV) * 4;
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            S[i].x = fmaf(kn[i], dl[0], decay * S[i].x);
            S[i].y = fmaf(kn[i], dl[1], decay * S[i].y);
            S[i].z = fmaf(kn[i], dl[2], decay * S[i].z);
            S[i].w = fmaf(kn[i], dl[3], decay * S[i].w);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, S[i]), rs, soff + RG * i * DV * 4, 0,
                                                   qs::CP_NT | qs::CP_SC1);
        }
        if constexpr (NORM) {
            // the head's o in fp32 (lanes < CG of each slab's wave WO), its sum of squares over the 4 slabs in
            // slab order, then the gated RMSNorm, rounded once to bf16
            float po[4] = {0.f, 0.f, 0.f, 0.f};
            if (w == WO && lane < CG) {
                const float qk = s_qk_[gw][t];  // q . k of the token (past the exchange barrier)
#pragma unroll
                for (int j = 0; j < 4; ++j) po[j] = fmaf(qk, dl[j], decay * r[j]);
            }
            float ss = (po[0] * po[0] + po[1] * po[1]) + (po[2] * po[2] + po[3] * po[3]);
            // the sum over the first 16-lane row (lanes 0 .. CG - 1 hold o, the others zeros): quads by xor 1,
            // xor 2, then row_ror 4 and 8, after which every lane of the row, lane 0 included, holds the total
            ss += qs::dpp<0xB1>(ss);
            ss += qs::dpp<0x4E>(ss);
            ss += qs::dpp<0x124>(ss);
            ss += qs::dpp<0x128>(ss);
            if (w == WO && lane == 0) s_nrm[t & 1][gw] = ss;
            __syncthreads();
            if (w == WO && lane < CG) {
                float tot = s_nrm[t & 1][0];
#pragma unroll
                for (int u = 1; u < WPG; ++u) tot += s_nrm[t & 1][u];
                const float rn = rsqrtf(tot * (1.0f / DV) + a.eps);
                const int d0 = s * SLAB + cg * 4;
                const float y0 = po[0] * rn * w4.x * qs::silu(qs::bf_lo(z4.x));
                const float y1 = po[1] * rn * w4.y * qs::silu(qs::bf_hi(z4.x));
                const float y2 = po[2] * rn * w4.z * qs::silu(qs::bf_lo(z4.y));
                const float y3 = po[3] * rn * w4.w * qs::silu(qs::bf_hi(z4.y));
                *reinterpret_cast<uint2 *>(a.o + (size_t)gi * DV + d0) =
                    make_uint2(qs::cvt_pk_bf16(y0, y1), qs::cvt_pk_bf16(y2, y3));
            }
        } else if (w == WO && lane < CG) {
            const float qk = s_qk_[gw][t];  // q . k of the token (past the exchange barrier)
            float po[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) po[j] = fmaf(qk, dl[j], decay * r[j]);
            uint2 pk;
            pk.x = qs::pack_bf2(po[0], po[1]);
            pk.y = qs::pack_bf2(po[2], po[3]);
            *reinterpret_cast<uint2 *>(a.o + (size_t)gi * DV + s * SLAB + cg * 4) = pk;
        }
    }
    if (CONV && !VERIFY && (isq || isk)) {
        // one arrival per workgroup per counter: rep * NSLAB / WPG workgroups read key head kh's q/k history.
        // The increments sum to zero, so nothing is left to re-arm at the end (a store here would hold the
        // launch open for another round trip).
        const unsigned inc = kq_owner ? 1u - (unsigned)(rep * NSLAB / WPG) : 1u;
        const int last = (unsigned)__builtin_amdgcn_readfirstlane(arrived) + inc == 0u;
        if (last) {
            if (isq) conv_commit<false, TM>(a, inq, yq, b, cq, T, false, true);
            if (isk) conv_commit<false, TM>(a, ink, yk, b, ck, T, false, true);
        }
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
    y[i] = (uint16_t)(qs::cvt_pk_bf16(qs::silu(acc), 0.f) & 0xffffu);
    st[0] = st[1];
    st[1] = st[2];
    st[2] = (uint16_t)xr;
}

// -------------------------------------------------------------------------------------------- gated norm

// Gated RMSNorm of the delta rule's output, per row of DV values (torch model.py:274-275; the head cores'
// step 7-8, kernels/gdn_head_compute.cpp:320-346): out = bf16(o * rsqrt(mean(o^2) + eps) * w * silu(z)).
// One wave per row, two values per lane; the mean is a fixed-order wave reduction.
__global__ __launch_bounds__(256) void gated_norm_kernel(const uint16_t *o, const uint16_t *z, const float *w,
                                                         uint16_t *out, int rows, float eps) {
    const int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (row >= rows) return;  // the whole wave
    const int lane = threadIdx.x & 63;
    const uint32_t o2 = reinterpret_cast<const uint32_t *>(o + (size_t)row * DV)[lane];
    const uint32_t z2 = reinterpret_cast<const uint32_t *>(z + (size_t)row * DV)[lane];
    const float2 w2 = reinterpret_cast<const float2 *>(w)[lane];
    const float a = qs::bf_lo(o2), b = qs::bf_hi(o2);
    const float r = rsqrtf(qs::wave_sum_dpp(a * a + b * b) * (1.0f / DV) + eps);
    const float ya = a * r * w2.x * qs::silu(qs::bf_lo(z2));
    const float yb = b * r * w2.y * qs::silu(qs::bf_hi(z2));
    reinterpret_cast<uint32_t *>(out + (size_t)row * DV)[lane] = qs::cvt_pk_bf16(ya, yb);
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

// grid (chunks, B, layers): chunk c of user b copies 4 16-byte units per thread of its state snapshot (all
// loads issued before the stores), the chunks after the state's copy the conv-state snapshot the same way
// (2-byte units when the conv state is not a multiple of 16 bytes); chunk 0 of layer 0 also sets the new
// sequence length. Layer z's tensors start z * (its stride) elements past the given pointers. accept_len
// outside [1, T], or an idle slot (base_lens[b] < 0), leaves the user untouched.
constexpr int RB_UNITS = 4;  // 16-byte units per thread

// Units i0, i0 + 256, i0 + 512, i0 + 768 of src to dst (those below n): every load first (clamped into
// range, so nothing is indexed dynamically), then the stores.
template <typename V>
__device__ __forceinline__ void copy4(const V *__restrict__ src, V *__restrict__ dst, size_t i0, size_t n) {
    const V a0 = src[min(i0, n - 1)], a1 = src[min(i0 + 256, n - 1)];
    const V a2 = src[min(i0 + 512, n - 1)], a3 = src[min(i0 + 768, n - 1)];
    if (i0 < n) dst[i0] = a0;
    if (i0 + 256 < n) dst[i0 + 256] = a1;
    if (i0 + 512 < n) dst[i0 + 512] = a2;
    if (i0 + 768 < n) dst[i0 + 768] = a3;
}
__global__ __launch_bounds__(256) void rollback_kernel(const float *states_out, float *state,
                                                       const uint16_t *conv_states_out, uint16_t *conv_state,
                                                       const int *accept, int *seq_lens, const int *base_lens,
                                                       int B, int T, size_t state_f4, size_t conv_elems,
                                                       int state_chunks, size_t so_stride, size_t s_stride,
                                                       size_t co_stride, size_t c_stride) {
    const int b = blockIdx.y, z = blockIdx.z;
    states_out += z * so_stride;
    state += z * s_stride;
    conv_states_out += z * co_stride;
    conv_state += z * c_stride;
    const int acc = accept[b];
    if (acc < 1 || acc > T) return;
    if (base_lens && base_lens[b] < 0) return;  // an idle slot: nothing was verified, nothing to restore
    const size_t slot = (size_t)(acc - 1) * B + b;
    if ((int)blockIdx.x < state_chunks) {
        const float4 *src = reinterpret_cast<const float4 *>(states_out) + slot * state_f4;
        float4 *dst = reinterpret_cast<float4 *>(state) + (size_t)b * state_f4;
        const size_t i0 = (size_t)blockIdx.x * 256 * RB_UNITS + threadIdx.x;
        copy4(src, dst, i0, state_f4);
    } else {
        const uint16_t *cs = conv_states_out + slot * conv_elems;
        uint16_t *cd = conv_state + (size_t)b * conv_elems;
        const size_t i0 = (size_t)(blockIdx.x - state_chunks) * 256 * RB_UNITS + threadIdx.x;
        if (conv_elems % 8 == 0) {
            const uint4 *cs4 = reinterpret_cast<const uint4 *>(cs);
            uint4 *cd4 = reinterpret_cast<uint4 *>(cd);
            copy4(cs4, cd4, i0, conv_elems / 8);
        } else {
            for (size_t i = i0 * 8; i < conv_elems && i < (i0 + 1) * 8 * RB_UNITS; ++i) cd[i] = cs[i];
        }
    }
    if (blockIdx.x == 0 && z == 0 && threadIdx.x == 0 && seq_lens) seq_lens[b] = base_lens[b] + acc;
}

// 32-column slabs. One wave per slab when that gives at least 1024 waves (batch >= 6 at 48 value heads),
// grouped 6 (or 4) to a workgroup: at 3 value heads per key head, 6 consecutive slab units are half of one
// key head's 12, so the q / k conv runs once per workgroup (waves 0 and 1, shared through LDS) and 2
// workgroups count in per key head; at batch 8 that is 256 workgroups, one per CU, which streams the same
// access pattern ~5% faster than 1536 single-wave workgroups. Below 1024 units each slab's rows are split
// over 4 waves so the grid fills the chip. The choice depends on the shape only, so a one-token verify
// reproduces decode bit for bit at every batch. Verify kernels are compiled for up to 4 and up to 8 tokens.
template <bool CONV, bool VERIFY, int TM>
void launch_gdn_tm(const GdnArgs &a, hipStream_t st) {
    const int units = a.B * a.NV * (DV / 32);
    const int per_key_head = (a.NV / a.NK) * (DV / 32);  // consecutive slab units sharing one key head
    if constexpr (!VERIFY) {
        // with the gated RMSNorm epilogue a workgroup holds one value head: its 4 slabs on one wave each at
        // large batch, on 4 waves each (16 waves) below
        if (a.z) {
            if (units >= 1024)
                gdn_kernel<CONV, VERIFY, TM, 32, 1, 4, true><<<units / 4, 256, 0, st>>>(a);
            else
                gdn_kernel<CONV, VERIFY, TM, 32, 4, 4, true><<<units / 4, 1024, 0, st>>>(a);
            return;
        }
    }
    // a workgroup's slab units must lie in one key head (they share its q / k conv through LDS, and the
    // conv-state counter expects per_key_head / WPG arrivals): 6 per workgroup when 6 divides the key
    // head's units (3 value heads per key head: one workgroup per CU at batch 8), else 4 (always divides)
    if (units >= 1024 && per_key_head % 6 == 0)
        gdn_kernel<CONV, VERIFY, TM, 32, 1, 6><<<units / 6, 384, 0, st>>>(a);
    else if (units >= 1024)
        gdn_kernel<CONV, VERIFY, TM, 32, 1, 4><<<units / 4, 256, 0, st>>>(a);
    else
        gdn_kernel<CONV, VERIFY, TM, 32, 4, 1><<<units, 256, 0, st>>>(a);
}
template <bool CONV, bool VERIFY>
void launch_gdn(const GdnArgs &a, hipStream_t st) {
    if constexpr (!VERIFY)
        launch_gdn_tm<CONV, VERIFY, 1>(a, st);
    else if (a.T <= 4)
        launch_gdn_tm<CONV, VERIFY, 4>(a, st);
    else
        launch_gdn_tm<CONV, VERIFY, TMAX>(a, st);
}

// The conv reads channel pairs with 4-, 12- and 16-byte loads.
int check_conv_alignment(const void *x, const void *conv, const void *conv_out, const void *taps, const void *y_out) {
    auto al = [](const void *p, uintptr_t n) { return ((uintptr_t)p % n) == 0; };
    QS_REQUIRE(al(x, 4) && al(conv, 4) && al(conv_out, 4) && al(taps, 16) && al(y_out, 4),
               "x, conv state and y_out must be 4-byte aligned, taps 16-byte aligned");
    return QS_OK;
}

int check_gdn_shapes(int B, int NK, int NV, int DKa, int DVa) {
    QS_REQUIRE(B > 0, "B must be positive (got %d)", B);
    QS_REQUIRE(DKa == DK && DVa == DV, "DK and DV must be 128 (got %d, %d)", DKa, DVa);
    QS_REQUIRE(NK > 0 && NV > 0 && NV % NK == 0, "NV (%d) must be a positive multiple of NK (%d)", NV, NK);
    QS_REQUIRE((long)B * NV * (DV / 16) < (1L << 31), "grid too large");
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

extern "C" int qs_gdn_gated_norm(const uint16_t *o, const uint16_t *z, const float *norm_w, uint16_t *out, int rows,
                                 int DVa, float eps, void *stream) {
    QS_REQUIRE(o && z && norm_w && out, "qs_gdn_gated_norm: null pointer");
    QS_REQUIRE(rows > 0 && DVa == DV, "qs_gdn_gated_norm: need rows > 0 and DV = %d (got %d, %d)", DV, rows, DVa);
    QS_REQUIRE(eps > 0.f, "qs_gdn_gated_norm: eps must be positive");
    QS_REQUIRE(((uintptr_t)o | (uintptr_t)z | (uintptr_t)out) % 4 == 0 && (uintptr_t)norm_w % 8 == 0,
               "qs_gdn_gated_norm: o, z, out must be 4-byte and norm_w 8-byte aligned");
    gated_norm_kernel<<<(rows + 3) / 4, 256, 0, QS_STREAM(stream)>>>(o, z, norm_w, out, rows, eps);
    return qs::launch_status("qs_gdn_gated_norm");
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
    QS_REQUIRE(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) % 4 == 0, "qs_gdn_decode_step: q, k, v must be 4-byte aligned");
    if (int e = check_gdn_shapes(B, NK, NV, DKa, DVa)) return e;
    GdnArgs a{};
    a.q = q, a.k = k, a.v = v, a.g = g, a.beta = beta, a.s_in = state, a.s_out = state, a.o = o;
    a.B = B, a.T = 1, a.NK = NK, a.NV = NV, a.C = 2 * NK * DK + NV * DV, a.scale = scale, a.eps = eps;
    launch_gdn<false, false>(a, QS_STREAM(stream));
    return qs::launch_status("qs_gdn_decode_step");
}

extern "C" size_t qs_gdn_workspace_bytes(int B, int NK) { return (size_t)(B > 0 ? B : 0) * (NK > 0 ? NK : 0) * 8; }

extern "C" int qs_gdn_decode_fused(const uint16_t *x, uint16_t *conv_state, const uint16_t *taps, const float *g,
                                   const float *beta, float *state, uint16_t *o, uint16_t *y_out, const uint16_t *z,
                                   int ldz, const float *norm_w, void *workspace, const int *lens, int B, int NK,
                                   int NV, int DKa, int DVa, int K, float scale, float eps, void *stream) {
    QS_REQUIRE(x && conv_state && taps && g && beta && state && o && workspace,
               "qs_gdn_decode_fused: null pointer");
    if (int e = check_gdn_shapes(B, NK, NV, DKa, DVa)) return e;
    QS_REQUIRE(K == KC, "qs_gdn_decode_fused: only K = 4 taps are supported (got %d)", K);
    if (int e = check_conv_alignment(x, conv_state, conv_state, taps, y_out)) return e;
    QS_REQUIRE(!z == !norm_w, "qs_gdn_decode_fused: give both z and norm_w or neither");
    QS_REQUIRE(!z || (ldz >= NV * DVa && ldz % 4 == 0 && (uintptr_t)z % 8 == 0 && (uintptr_t)norm_w % 16 == 0),
               "qs_gdn_decode_fused: z rows need ldz >= NV DV, ldz %% 4 == 0, z 8-byte and norm_w 16-byte aligned "
               "(got ldz %d)", ldz);
    GdnArgs a{};
    a.x = x, a.conv_in = conv_state, a.conv_out = conv_state, a.taps = taps, a.y_out = y_out;
    a.g = g, a.beta = beta, a.s_in = state, a.s_out = state, a.o = o;
    a.z = z, a.ldz = ldz, a.norm_w = norm_w;
    a.counters = static_cast<int *>(workspace);
    a.lens = lens;
    a.B = B, a.T = 1, a.NK = NK, a.NV = NV, a.C = 2 * NK * DK + NV * DV, a.scale = scale, a.eps = eps;
    launch_gdn<true, false>(a, QS_STREAM(stream));
    return qs::launch_status("qs_gdn_decode_fused");
}

// ------------------------------------------------------------------------ allocation-free fused decode
// qs_gdn_decode_fused with its conv counters in a file-scope device array instead of a caller workspace, for
// callers that cannot allocate. Each device holds its own copy of the array until the process ends; host
// code reaches it only through the address hipGetSymbolAddress returns for the current device (the array's
// name in host code is a stand-in, not a device address). The counters self-reset like the workspace's, so
// the array stays zero between calls; it is cleared once per device by a fill kernel at the first call.
// Every call on one device shares the array: calls that overlap on a device (concurrent streams) race.
namespace {
constexpr int SCRATCH_INTS = 16384;  // 64 KB: two counters per (user, key head), B * NK <= 8192
static __device__ __align__(256) int scratch[SCRATCH_INTS];

__global__ void fill_zero_kernel(int *p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
}

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
int *g_scratch_ptr[MAX_DEVICES] = {};
bool g_scratch_cleared[MAX_DEVICES] = {};

// The current device's copy of `scratch`: its address is looked up on the first call on that device, and
// it is cleared by a fill kernel on `st` (clear = true) until a clear has run outside a graph capture. A
// clear enqueued while `st` is capturing becomes a node of the graph (it runs before the decode kernel on
// every replay, which only re-zeroes counters that are zero between calls) and the next call outside a
// capture clears again, so the array is zeroed before its first use whichever comes first.
int scratch_of_current_device(int **out, hipStream_t st, bool clear, const char *who) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        qs::set_error("%s: no usable current device (%d)", who, dev);
        return QS_EHIP;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            qs::set_error("%s: hipGetSymbolAddress failed: %s", who, hipGetErrorString(e));
            return QS_EHIP;
        }
        g_scratch_ptr[dev] = static_cast<int *>(p);
    }
    if (clear && !g_scratch_cleared[dev]) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
            qs::set_error("%s: hipStreamIsCapturing failed", who);
            return QS_EHIP;
        }
        fill_zero_kernel<<<SCRATCH_INTS / 256, 256, 0, st>>>(g_scratch_ptr[dev], SCRATCH_INTS);
        if (int rc = qs::launch_status(who)) return rc;
        if (cs == hipStreamCaptureStatusNone) g_scratch_cleared[dev] = true;
    }
    *out = g_scratch_ptr[dev];
    return QS_OK;
}

}  // namespace

extern "C" int qs_gdn_decode_fused_noalloc(const uint16_t *x, uint16_t *conv_state, const uint16_t *taps,
                                           const float *g, const float *beta, float *state, uint16_t *o,
                                           uint16_t *y_out, const int *lens, int B, int NK, int NV, int DKa,
                                           int DVa, int K, float scale, float eps, void *stream) {
    QS_REQUIRE(x && conv_state && taps && g && beta && state && o, "qs_gdn_decode_fused_noalloc: null pointer");
    if (int e = check_gdn_shapes(B, NK, NV, DKa, DVa)) return e;
    QS_REQUIRE(K == KC, "qs_gdn_decode_fused_noalloc: only K = 4 taps are supported (got %d)", K);
    QS_REQUIRE((long)B * NK * 2 <= SCRATCH_INTS, "qs_gdn_decode_fused_noalloc: B NK = %ld exceeds %d",
               (long)B * NK, SCRATCH_INTS / 2);
    if (int e = check_conv_alignment(x, conv_state, conv_state, taps, y_out)) return e;
    int *counters = nullptr;
    if (int e = scratch_of_current_device(&counters, QS_STREAM(stream), true, "qs_gdn_decode_fused_noalloc")) return e;
    GdnArgs a{};
    a.x = x, a.conv_in = conv_state, a.conv_out = conv_state, a.taps = taps, a.y_out = y_out;
    a.g = g, a.beta = beta, a.s_in = state, a.s_out = state, a.o = o;
    a.counters = counters;
    a.lens = lens;
    a.B = B, a.T = 1, a.NK = NK, a.NV = NV, a.C = 2 * NK * DK + NV * DV, a.scale = scale, a.eps = eps;
    launch_gdn<true, false>(a, QS_STREAM(stream));
    return qs::launch_status("qs_gdn_decode_fused_noalloc");
}

extern "C" int qs_gdn_noalloc_scratch_read(int *dst, int n, void *stream) {
    QS_REQUIRE(dst, "qs_gdn_noalloc_scratch_read: null pointer");
    QS_REQUIRE(n >= 1 && n <= SCRATCH_INTS, "qs_gdn_noalloc_scratch_read: n must be in [1, %d] (got %d)", SCRATCH_INTS,
               n);
    int *src = nullptr;
    if (int e = scratch_of_current_device(&src, QS_STREAM(stream), false, "qs_gdn_noalloc_scratch_read")) return e;
    const hipError_t e = hipMemcpyAsync(dst, src, (size_t)n * sizeof(int), hipMemcpyDeviceToDevice, QS_STREAM(stream));
    if (e != hipSuccess) {
        qs::set_error("qs_gdn_noalloc_scratch_read: hipMemcpyAsync failed: %s", hipGetErrorString(e));
        return QS_EHIP;
    }
    return QS_OK;
}

extern "C" int qs_gdn_verify_step(const uint16_t *x, const uint16_t *conv_state_in, uint16_t *conv_states_out,
                                  const uint16_t *taps, const float *g, const float *beta, const float *state_in,
                                  float *states_out, uint16_t *o, uint16_t *y_out, const int *lens, int B, int T,
                                  int NK, int NV, int DKa, int DVa, int K, float scale, float eps, void *stream) {
    QS_REQUIRE(x && conv_state_in && conv_states_out && taps && g && beta && state_in && states_out && o,
               "qs_gdn_verify_step: null pointer");
    if (int e = check_gdn_shapes(B, NK, NV, DKa, DVa)) return e;
    QS_REQUIRE(T >= 1 && T <= TMAX, "qs_gdn_verify_step: T must be in [1, %d] (got %d)", TMAX, T);
    QS_REQUIRE(K == KC, "qs_gdn_verify_step: only K = 4 taps are supported (got %d)", K);
    if (int e = check_conv_alignment(x, conv_state_in, conv_states_out, taps, y_out)) return e;
    QS_REQUIRE(states_out != state_in, "qs_gdn_verify_step: states_out must not alias state_in");
    GdnArgs a{};
    a.x = x, a.conv_in = conv_state_in, a.conv_out = conv_states_out, a.taps = taps, a.y_out = y_out;
    a.g = g, a.beta = beta, a.s_in = state_in, a.s_out = states_out, a.o = o;
    a.lens = lens;
    a.B = B, a.T = T, a.NK = NK, a.NV = NV, a.C = 2 * NK * DK + NV * DV, a.scale = scale, a.eps = eps;
    launch_gdn<true, true>(a, QS_STREAM(stream));
    return qs::launch_status("qs_gdn_verify_step");
}

extern "C" int qs_gdn_verify_step_slots(const uint16_t *x, const uint16_t *conv_states_in, uint16_t *conv_states_out,
                                        const uint16_t *taps, const float *g, const float *beta,
                                        const float *states_in, float *states_out, const int *in_slot, int n_slots,
                                        uint16_t *o, uint16_t *y_out, const int *lens, int B, int T, int NK, int NV,
                                        int DKa, int DVa, int K, float scale, float eps, void *stream) {
    QS_REQUIRE(x && conv_states_in && conv_states_out && taps && g && beta && states_in && states_out && in_slot && o,
               "qs_gdn_verify_step_slots: null pointer");
    if (int e = check_gdn_shapes(B, NK, NV, DKa, DVa)) return e;
    QS_REQUIRE(T >= 1 && T <= TMAX, "qs_gdn_verify_step_slots: T must be in [1, %d] (got %d)", TMAX, T);
    QS_REQUIRE(n_slots >= 1, "qs_gdn_verify_step_slots: n_slots must be positive (got %d)", n_slots);
    QS_REQUIRE(K == KC, "qs_gdn_verify_step_slots: only K = 4 taps are supported (got %d)", K);
    if (int e = check_conv_alignment(x, conv_states_in, conv_states_out, taps, y_out)) return e;
    QS_REQUIRE(states_out != states_in && conv_states_out != conv_states_in,
               "qs_gdn_verify_step_slots: outputs must not alias the input slots");
    GdnArgs a{};
    a.x = x, a.conv_in = conv_states_in, a.conv_out = conv_states_out, a.taps = taps, a.y_out = y_out;
    a.g = g, a.beta = beta, a.s_in = states_in, a.s_out = states_out, a.o = o;
    a.in_slot = in_slot, a.n_slots = n_slots;
    a.lens = lens;
    a.B = B, a.T = T, a.NK = NK, a.NV = NV, a.C = 2 * NK * DK + NV * DV, a.scale = scale, a.eps = eps;
    launch_gdn<true, true>(a, QS_STREAM(stream));
    return qs::launch_status("qs_gdn_verify_step_slots");
}

// Acceptance by slot selection: slot[b] <- accept[b] - 1 and seq_lens[b] <- base_lens[b] + accept[b] for
// accept[b] in [1, T]; other users are left untouched and reported (QS_STATUS_ACCEPT) when status is given.
// An idle slot (base_lens[b] < 0: the step's advance left its length negative) keeps its slot and length
// whatever its accept length.
__global__ void verify_accept_kernel(const int *accept, int *slot, int *seq_lens, const int *base_lens, int B, int T,
                                     int *status) {
    const int b = blockIdx.x * 64 + threadIdx.x;
    if (b >= B) return;
    if (base_lens && base_lens[b] < 0) return;
    const int acc = accept[b];
    if (acc < 1 || acc > T) {
        if (status) atomicOr(status, QS_STATUS_ACCEPT);
        return;
    }
    slot[b] = acc - 1;
    if (seq_lens) seq_lens[b] = base_lens[b] + acc;
}

extern "C" int qs_verify_accept(const int *accept_len, int *slot, int *seq_lens, const int *base_lens, int B, int T,
                                int *status, void *stream) {
    QS_REQUIRE(accept_len && slot, "qs_verify_accept: null pointer");
    QS_REQUIRE(!seq_lens || base_lens, "qs_verify_accept: seq_lens needs base_lens");
    QS_REQUIRE(B > 0 && T >= 1 && T <= TMAX, "qs_verify_accept: bad shape (B %d, T %d)", B, T);
    verify_accept_kernel<<<(B + 63) / 64, 64, 0, QS_STREAM(stream)>>>(accept_len, slot, seq_lens, base_lens, B, T,
                                                                      status);
    return qs::launch_status("qs_verify_accept");
}

static int rollback_launch(const float *states_out, size_t so_stride, float *state, size_t s_stride,
                           const uint16_t *conv_states_out, size_t co_stride, uint16_t *conv_state, size_t c_stride,
                           const int *accept_len, int *seq_lens, const int *base_lens, int L, int B, int T, int NV,
                           int DKa, int DVa, int C, int K, void *stream, const char *who) {
    QS_REQUIRE(states_out && state && conv_states_out && conv_state && accept_len, "%s: null pointer", who);
    QS_REQUIRE(!seq_lens || base_lens, "%s: seq_lens needs base_lens", who);
    QS_REQUIRE(L >= 1 && L <= 65535 && B > 0 && B <= 65535 && T >= 1 && T <= TMAX && NV > 0 && C > 0 && K == KC,
               "%s: bad shape", who);
    QS_REQUIRE(DKa == DK && DVa == DV, "%s: DK and DV must be 128", who);
    const size_t state_f4 = (size_t)NV * DK * DV / 4;
    const size_t conv_elems = (size_t)C * (K - 1);
    const size_t per_chunk = 256 * RB_UNITS;  // 16-byte units per workgroup
    const size_t conv_units = conv_elems % 8 == 0 ? conv_elems / 8 : (conv_elems + 7) / 8;
    const int state_chunks = (int)((state_f4 + per_chunk - 1) / per_chunk);
    const int conv_chunks = (int)((conv_units + per_chunk - 1) / per_chunk);
    QS_REQUIRE((long)state_chunks + conv_chunks < (1L << 31), "%s: state too large", who);
    rollback_kernel<<<dim3(state_chunks + conv_chunks, B, L), 256, 0, QS_STREAM(stream)>>>(
        states_out, state, conv_states_out, conv_state, accept_len, seq_lens, base_lens, B, T, state_f4, conv_elems,
        state_chunks, so_stride, s_stride, co_stride, c_stride);
    return qs::launch_status(who);
}

extern "C" int qs_gdn_rollback(const float *states_out, float *state, const uint16_t *conv_states_out,
                               uint16_t *conv_state, const int *accept_len, int *seq_lens, const int *base_lens,
                               int B, int T, int NV, int DKa, int DVa, int C, int K, void *stream) {
    return rollback_launch(states_out, 0, state, 0, conv_states_out, 0, conv_state, 0, accept_len, seq_lens, base_lens,
                           1, B, T, NV, DKa, DVa, C, K, stream, "qs_gdn_rollback");
}

extern "C" int qs_gdn_rollback_layers(const float *states_out, size_t states_out_layer_stride, float *state,
                                      size_t state_layer_stride, const uint16_t *conv_states_out,
                                      size_t conv_states_out_layer_stride, uint16_t *conv_state,
                                      size_t conv_state_layer_stride, const int *accept_len, int *seq_lens,
                                      const int *base_lens, int L, int B, int T, int NV, int DKa, int DVa, int C,
                                      int K, void *stream) {
    return rollback_launch(states_out, states_out_layer_stride, state, state_layer_stride, conv_states_out,
                           conv_states_out_layer_stride, conv_state, conv_state_layer_stride, accept_len, seq_lens,
                           base_lens, L, B, T, NV, DKa, DVa, C, K, stream, "qs_gdn_rollback_layers");
}
