// Causal depthwise conv1d + SiLU over a prefill prompt of T tokens, with the conv carry in and out.
//
// Window of channel c: w = [carry_0, carry_1, carry_2, x_0, x_1, ..., x_{T-1}] (oldest first, carry zero
// when none is given); y_t = bf16(silu(w_t tap_0 + w_{t+1} tap_1 + w_{t+2} tap_2 + w_{t+3} tap_3)) and the new
// carry is w_T, w_{T+1}, w_{T+2}: the last three inputs, bits unchanged. The tap sum runs in the order of
// the decode update (tap 0 first, one rounding per addition; each product of two bf16 values is exact in
// fp32), so y equals T successive decode conv steps bit for bit, and the carry is the decode conv state
// those steps leave.
//
// One thread per 8 adjacent channels (16-byte rows) and R = 8 tokens: it loads the 11 window rows it needs
// (the 3 before its block from x, or from the carry for the first block), then writes 8 output rows into
// the q, k or v plane its channels belong to (channels [0, CQ) -> q, [CQ, 2 CQ) -> k, [2 CQ, 2 CQ + CV) -> v).
// The threads of the first token block also write the new carry; they are the only readers of the carry
// in, so the carry may be updated in place. Lanes run over channel groups, so every row access is a
// contiguous 1 KB per wave. Measured at 8192 tokens x 10240 channels with the prompts rotating past the
// Infinity Cache: ~66.5 us, 5.05 TB/s of algorithmic bytes, HBM reads 1.10x the input (the halo rows of
// wave 0).
#include "qs_common.h"

namespace {

constexpr int KC = 4;  // conv taps
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int R = 8;  // tokens per thread (4, 16, 24, 32, or 4 blocks of 16 in sequence measured slower)

struct ConvPrefillArgs {
    const uint16_t *x;       // [T, ldx], conv channels in columns [0, 2 CQ + CV)
    const uint16_t *st_in;   // [C, 3] or null (zeros)
    const uint16_t *taps;    // [C, 4]
    uint16_t *q, *k, *v;     // [T, CQ], [T, CQ], [T, CV]
    uint16_t *st_out;        // [C, 3], may equal st_in
    int ldx, T, CQ, CV, ngroups, ntb;
};

__device__ __forceinline__ uint32_t half_of(const uint4 &r, int c) {
    const uint32_t w = c < 2 ? r.x : c < 4 ? r.y : c < 6 ? r.z : r.w;
    return (c & 1) ? w >> 16 : w & 0xffffu;
}

__global__ __launch_bounds__(256) void conv_prefill_kernel(ConvPrefillArgs a) {
    // workgroup = 64 channel groups (lanes) x 4 consecutive token blocks (waves): the 3 rows before the
    // block of waves 1-3 are rows the wave before loads, so only wave 0's come from another workgroup;
    // consecutive workgroups run across the channel spans, so the running ones stream whole rows
    const int nspan = (a.ngroups + 63) / 64;
    const int span = (int)blockIdx.x % nspan, quad = (int)blockIdx.x / nspan;
    const int cg = span * 64 + (int)(threadIdx.x & 63), tb = quad * 4 + (int)(threadIdx.x >> 6);
    if (tb >= a.ntb || cg >= a.ngroups) return;
    const int c0 = cg * 8, t0 = tb * R;

    uint4 tw[4];  // taps of channels c0 .. c0 + 7, 4 per channel
#pragma unroll
    for (int i = 0; i < 4; ++i) tw[i] = reinterpret_cast<const uint4 *>(a.taps + (size_t)c0 * KC)[i];

    // carry of channels c0 .. c0 + 7 ([c][j], 24 values), read only by the first token block
    uint32_t sw[12];
#pragma unroll
    for (int i = 0; i < 12; ++i) sw[i] = 0;
    if (tb == 0 && a.st_in) {
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const uint4 s = reinterpret_cast<const uint4 *>(a.st_in + (size_t)c0 * (KC - 1))[i];
            sw[4 * i] = s.x, sw[4 * i + 1] = s.y, sw[4 * i + 2] = s.z, sw[4 * i + 3] = s.w;
        }
    }
    auto carry = [&](int c, int j) -> uint32_t {  // c, j compile-time
        const int e = c * (KC - 1) + j;
        return (e & 1) ? sw[e >> 1] >> 16 : sw[e >> 1] & 0xffffu;
    };
    auto carry_rt = [&](int c, int j) -> uint32_t {  // j in [0, 3) known only at run time
        return j == 0 ? carry(c, 0) : j == 1 ? carry(c, 1) : carry(c, 2);
    };

    // window rows t0 - 3 .. t0 + R - 1
    uint4 w[R + 3];
#pragma unroll
    for (int i = 0; i < R + 3; ++i) {
        const int t = t0 - 3 + i;
        if (t >= 0 && t < a.T) {
            w[i] = *reinterpret_cast<const uint4 *>(a.x + (size_t)t * a.ldx + c0);
        } else if (i < 3 && t < 0) {  // first block only: the carry row j = t + 3 = i
            uint32_t p[4];
#pragma unroll
            for (int c = 0; c < 8; c += 2) p[c >> 1] = carry(c, i) | (carry(c + 1, i) << 16);
            w[i] = make_uint4(p[0], p[1], p[2], p[3]);
        } else {
            w[i] = make_uint4(0, 0, 0, 0);
        }
    }

    uint16_t *dst;
    int ld;
    if (c0 < a.CQ) dst = a.q + c0, ld = a.CQ;
    else if (c0 < 2 * a.CQ) dst = a.k + (c0 - a.CQ), ld = a.CQ;
    else dst = a.v + (c0 - 2 * a.CQ), ld = a.CV;

#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int t = t0 + r;
        if (t >= a.T) break;
        float y[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint4 &tc = tw[c >> 1];
            const uint32_t t01 = (c & 1) ? tc.z : tc.x, t23 = (c & 1) ? tc.w : tc.y;
            float acc = qs::bf2f(half_of(w[r], c)) * qs::bf_lo(t01);
            acc = acc + qs::bf2f(half_of(w[r + 1], c)) * qs::bf_hi(t01);
            acc = acc + qs::bf2f(half_of(w[r + 2], c)) * qs::bf_lo(t23);
            acc = acc + qs::bf2f(half_of(w[r + 3], c)) * qs::bf_hi(t23);
            y[c] = qs::silu(acc);
        }
        // streamed out (nontemporal): 66.5 against 70 us per prompt with write-back stores; nontemporal loads
        // of x measured slower (75 us), the halo rows are then re-read from memory
        const u32x4 yo = {qs::cvt_pk_bf16(y[0], y[1]), qs::cvt_pk_bf16(y[2], y[3]), qs::cvt_pk_bf16(y[4], y[5]),
                          qs::cvt_pk_bf16(y[6], y[7])};
        __builtin_nontemporal_store(yo, reinterpret_cast<u32x4 *>(dst + (size_t)t * ld));
    }

    if (tb == 0) {
        // new carry row j = window position T + j: carry row T + j while T + j < 3, else input T - 3 + j
        uint4 nr[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int t = a.T - 3 + j;
            if (t >= 0) {
                nr[j] = *reinterpret_cast<const uint4 *>(a.x + (size_t)t * a.ldx + c0);
            } else {
                uint32_t p[4];
#pragma unroll
                for (int c = 0; c < 8; c += 2) p[c >> 1] = carry_rt(c, a.T + j) | (carry_rt(c + 1, a.T + j) << 16);
                nr[j] = make_uint4(p[0], p[1], p[2], p[3]);
            }
        }
        uint32_t o[12];
#pragma unroll
        for (int i = 0; i < 12; ++i) {
            const int e0 = 2 * i, e1 = 2 * i + 1;  // element e = c * 3 + j
            o[i] = half_of(nr[e0 % 3], e0 / 3) | (half_of(nr[e1 % 3], e1 / 3) << 16);
        }
#pragma unroll
        for (int i = 0; i < 3; ++i)
            reinterpret_cast<uint4 *>(a.st_out + (size_t)c0 * (KC - 1))[i] =
                make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
    }
}

}  // namespace

extern "C" int qs_conv1d_prefill(const uint16_t *x, int ldx, const uint16_t *conv_state_in, const uint16_t *taps,
                                 uint16_t *q, uint16_t *k, uint16_t *v, uint16_t *conv_state_out, int T, int CQ,
                                 int CV, int K, void *stream) {
    QS_REQUIRE((T == 0 || (x && q && k && v)) && taps && conv_state_out, "qs_conv1d_prefill: null pointer");
    QS_REQUIRE(K == KC, "qs_conv1d_prefill: only K = 4 taps are supported (got %d)", K);
    QS_REQUIRE(T >= 0, "qs_conv1d_prefill: T must be non-negative (got %d)", T);
    QS_REQUIRE(CQ > 0 && CV > 0 && CQ % 8 == 0 && CV % 8 == 0,
               "qs_conv1d_prefill: CQ and CV must be positive multiples of 8 (got %d, %d)", CQ, CV);
    const int C = 2 * CQ + CV;
    QS_REQUIRE(ldx >= C && ldx % 8 == 0, "qs_conv1d_prefill: ldx (%d) must be a multiple of 8 and >= %d", ldx, C);
    QS_REQUIRE(((uintptr_t)x | (uintptr_t)taps | (uintptr_t)q | (uintptr_t)k | (uintptr_t)v |
                (uintptr_t)conv_state_out | (uintptr_t)conv_state_in) % 16 == 0,
               "qs_conv1d_prefill: every buffer must be 16-byte aligned");
    ConvPrefillArgs a{};
    a.x = x, a.st_in = conv_state_in, a.taps = taps, a.q = q, a.k = k, a.v = v, a.st_out = conv_state_out;
    a.ldx = ldx, a.T = T, a.CQ = CQ, a.CV = CV, a.ngroups = C / 8, a.ntb = T > 0 ? (T + R - 1) / R : 1;
    const long wgs = (long)((a.ngroups + 63) / 64) * ((a.ntb + 3) / 4);
    QS_REQUIRE(wgs < (1L << 31), "qs_conv1d_prefill: T = %d tokens are too many for one launch", T);
    conv_prefill_kernel<<<(unsigned)wgs, 256, 0, QS_STREAM(stream)>>>(a);
    return qs::launch_status("qs_conv1d_prefill");
}
