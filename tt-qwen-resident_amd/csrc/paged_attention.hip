// Paged GQA decode attention on gfx950 (HD 256, block 64): split-K over block-table pages, online softmax,
// an ordered merge of the splits, optional fused append of the step's new K/V rows (and the mixer edges).
//
// Grid: one workgroup per (user, KV head, split); a split is `pps` (<= 64) consecutive block-table entries.
// Every K/V byte is loaded once for all G query heads of the KV head (GQA reuse) and, in a verify step, for
// all query tokens of the step. Two kernels walk the pages:
//   attn_wave_kernel  up to 16 query rows per KV head (every one-token decode): MFMA scores and P V, each
//                     wave on its own 16-row slices with no barrier in the page loop, one or two pages in
//                     flight per workgroup;
//   attn_mfma_kernel  17 to 32 query rows (verify steps up to T = 5 at G = 6): MFMA, the 4 waves on the same
//                     page, each wave owning a quarter of the head dims in P V;
//   attn_kernel       more query rows: VALU dot products, the 4 waves on the same page.
// The step's new rows are loaded with the query rows and attended without a round trip through the pool:
// the one-token kernel (up to two tokens) holds them in registers and patches them over the page rows they
// replace (K through a one-row LDS copy when the page goes straight into the score operand), the MFMA kernel
// (up to 8) stages them in LDS; both store them to the pool after the page loop. With the mixer or more
// tokens they are appended first, by the wave that reads them back from the pool.
// The splits' partials (m, l, unnormalised O per query row) go to the workspace and are merged in split order
// (the leader side of the reference: global max, rescale, sum, normalise, kernels/attn_leader_writer.cpp:
// 86-106 and kernels/attn_leader_compute.cpp:42-79) by the last workgroup of the (user, KV head) to finish
// when there are at most 16 splits, else by a separate merge launch, so results are identical run to run.
#include "qs_common.h"

namespace {

constexpr int HD = 256;
constexpr int BLK = 64;
// cache policy of the K / V page loads: nontemporal (each page is read once per step; measured ~5% faster
// than the default policy at batch 8 / 4096 positions and at batch 1 / 32768)
constexpr int NT = 2;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                           false);
}

struct AttnArgs {
    const uint16_t *q;                  // [B, T, NQ, HD]
    const uint16_t *k_new, *v_new;      // nullable [B, T, NKV, HD]
    uint16_t *k_cache, *v_cache;        // [num_blocks, NKV, BLK, HD]
    const int *block_table;             // [B, max_blocks]
    const int *seq_lens;                // [B]
    uint16_t *o;                        // [B, T, NQ, HD]
    float *part_o;                      // [B, NKV, nsplit, T G, HD]: split partials (unnormalised O)
    float *part_ml;                     // [B, NKV, nsplit, T G, 2]: their (max, sum), log2 domain
    int *cnt;                           // [B, NKV] arrival counters of the in-launch merge (kept zero)
    int *status;                        // nullable: QS_STATUS_* bits of invalid lengths / table entries
    int B, T, NQ, NKV, max_blocks, num_blocks, pps, nsplit;
    float scale;
    // mixer edges (qs_attn_mixer_decode; null / 0 for plain attention): q and the new k rows are
    // RMS-normalised times wq / wk [HD] and rotated on their first rot dims with rcos / rsin
    // [B, T, rot / 2]; the output is multiplied by sigmoid(gate [B, T, NQ, HD])
    const uint16_t *gate;
    const float *wq, *wk, *rcos, *rsin;
    int rot;
    float eps;
};

// Mixer prologue of one 8-element chunk (raw bf16 bits, chunk ch of a 256-dim row whose 32 chunks sit in 32
// consecutive, fully active lanes): y = x * rsqrt(mean(x^2) + eps) * w, then the rotary embedding on the
// first rot dims with the halves paired as at model.py:135-140 (d < rot/2 with d + rot/2:
// y_d c - y_{d+h} s and y_{d+h} c + y_d s). fp32 throughout (model.py:86-89, :237-238).
__device__ __forceinline__ void mixer_chunk(const uint4 raw, int ch, const float *w, const float *cs,
                                            const float *sn, int rot, float eps, float y[8]) {
    const uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        y[2 * e] = qs::bf_lo(wd[e]);
        y[2 * e + 1] = qs::bf_hi(wd[e]);
        ss = fmaf(y[2 * e], y[2 * e], ss);
        ss = fmaf(y[2 * e + 1], y[2 * e + 1], ss);
    }
    ss += qs::dpp<0xB1>(ss);
    ss += qs::dpp<0x4E>(ss);
    ss += qs::dpp<0x124>(ss);
    ss += qs::dpp<0x128>(ss);
    ss = qs::xor16_sum(ss);  // the 32 lanes of the row
    const float r = rsqrtf(ss * (1.0f / HD) + eps);
    const float4 w0 = *reinterpret_cast<const float4 *>(w + ch * 8), w1 = *reinterpret_cast<const float4 *>(w + ch * 8 + 4);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = y[i] * r * wv[i];
    if (rot > 0) {
        const int half = rot / 2, hc = half / 8;  // dims / chunks per half
        float yp[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) yp[i] = __shfl_xor(y[i], hc, 64);
        if (ch < 2 * hc) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int d = (ch * 8 + i) % half;
                y[i] = ch < hc ? y[i] * cs[d] - yp[i] * sn[d] : y[i] * cs[d] + yp[i] * sn[d];
            }
        }
    }
}
__device__ __forceinline__ uint4 pack8(const float y[8]) {
    return make_uint4(qs::cvt_pk_bf16(y[0], y[1]), qs::cvt_pk_bf16(y[2], y[3]), qs::cvt_pk_bf16(y[4], y[5]),
                      qs::cvt_pk_bf16(y[6], y[7]));
}
// The rounding residues y - bf16(y) of 8 values as bf16 (hi = pack8(y)): hi + lo carries y to ~2^-17 relative,
// so products against exact bf16 operands (K rows) keep the fp32 value of a normalised, rotated q.
__device__ __forceinline__ uint4 pack8_lo(const float y[8], uint4 hi) {
    const uint32_t h[4] = {hi.x, hi.y, hi.z, hi.w};
    uint32_t lo[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) lo[e] = qs::cvt_pk_bf16(y[2 * e] - qs::bf_lo(h[e]), y[2 * e + 1] - qs::bf_hi(h[e]));
    return make_uint4(lo[0], lo[1], lo[2], lo[3]);
}
__device__ __forceinline__ float sigm(float g) { return 1.0f / (1.0f + expf(-g)); }

// A user's length n (positions valid after this step's T rows) is usable when T <= n <= max_blocks * BLK.
// n < T marks an idle slot (nothing appended or attended, zero output); n past the block table is an error
// (reported in the status word) and the user is treated as idle, never clamped onto other positions.
__device__ __forceinline__ bool user_active(const AttnArgs &a, int n, bool report) {
    if (n > a.max_blocks * BLK) {
        if (report && a.status) atomicOr(a.status, QS_STATUS_LENGTH);
        return false;
    }
    return n >= a.T;
}
__device__ __forceinline__ void report_page(const AttnArgs &a) {
    if (a.status) atomicOr(a.status, QS_STATUS_PAGE);
}
// Zero output rows of an inactive user for KV head g (all T G query rows; threads of one workgroup).
template <int G, int NTH = 256>
__device__ __forceinline__ void zero_rows(const AttnArgs &a, int b, int g, int tid) {
    for (int idx = tid; idx < a.T * G * 32; idx += NTH) {
        const int qr = idx >> 5, ch = idx & 31;
        *reinterpret_cast<uint4 *>(a.o + (((size_t)b * a.T + qr / G) * a.NQ + g * G + qr % G) * HD + ch * 8) =
            make_uint4(0, 0, 0, 0);
    }
}

// Workspace layout (bytes): arrival counters | part_ml | part_o, each 256-byte aligned. The counters sit in
// a fixed block at the head, so a workspace reused for another shape never finds partial data where its
// counters are (they must read zero).
constexpr size_t CNT_BYTES = 65536;  // room for B NKV <= 16384 counters
struct WsLayout {
    size_t cnt, ml, po, total;
};
__host__ __device__ inline WsLayout ws_layout(int B, int T, int NKV, int G, int nsplit) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    WsLayout l;
    l.cnt = 0;
    l.ml = CNT_BYTES;
    l.po = l.ml + up((size_t)B * T * NKV * nsplit * G * 2 * 4);
    l.total = l.po + up((size_t)B * T * NKV * nsplit * G * HD * 4);
    return l;
}
// Row of the partial of query row qr (= t G + h) of split sp for user b, KV head g: one workgroup's rows
// are contiguous.
__device__ __forceinline__ size_t prow(const AttnArgs &a, int G, int b, int g, int sp, int qr) {
    return (((size_t)b * a.NKV + g) * a.nsplit + sp) * (size_t)(a.T * G) + qr;
}

// The MFMA kernels' first requests, each one buffer load with no branch around it (lanes outside the range
// read zeros without a memory access), so the compiler's waits stay exact: the first page's loads, issued
// next, need only the block-table entries, and nothing waits for the query rows until they are staged.
// Block-table entry p0 + lane of user b (zero past the split or the table; only entries below
// min(max_blocks, p0 + pps) are ever read back).
__device__ __forceinline__ int split_entries(const AttnArgs &a, int b, int p0, int lane) {
    const int cnt = max(0, min(a.max_blocks, p0 + a.pps) - p0);
    const auto r = __builtin_amdgcn_make_buffer_rsrc(
        qs::uniform_ptr(const_cast<int *>(a.block_table) + (size_t)b * a.max_blocks + min(p0, a.max_blocks)), (short)0,
        cnt * 4, 0x00020000);
    return (int)__builtin_amdgcn_raw_buffer_load_b32(r, lane * 4, 0, 0);
}
// 16-byte chunk ch of query row qr = t G + hh of user b, KV head g (zeros for qr >= T G)
__device__ __forceinline__ uint4 q_chunk(const AttnArgs &a, int G, int b, int g, int qr, int ch) {
    const int T = a.T;
    const auto r = __builtin_amdgcn_make_buffer_rsrc(
        qs::uniform_ptr(const_cast<uint16_t *>(a.q) + ((size_t)b * T * a.NQ + (size_t)g * G) * HD), (short)0,
        ((T - 1) * a.NQ + G) * HD * 2, 0x00020000);
    const int off = qr < T * G ? ((qr / G) * a.NQ + qr % G) * HD * 2 + ch * 16 : 0x7ffffff0;
    const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(x[0], x[1], x[2], x[3]);
}
// 16-byte chunk ch of the new K or V row of token t of user b, KV head g (rows [B, T, NKV, HD]; zeros for
// t >= T, ch < 0 or a null pointer)
__device__ __forceinline__ u32x4 new_chunk(const AttnArgs &a, const uint16_t *rows, int b, int g, int t, int ch) {
    const auto r = __builtin_amdgcn_make_buffer_rsrc(
        qs::uniform_ptr(const_cast<uint16_t *>(rows ? rows : a.q) + (size_t)b * a.T * a.NKV * HD), (short)0,
        rows ? a.T * a.NKV * HD * 2 : 0, 0x00020000);
    const int off = t < a.T && ch >= 0 ? ((t * a.NKV + g) * HD + ch * 8) * 2 : 0x7ffffff0;
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// One workgroup per (user, KV head, split); the 4 waves work on the same page at a time, wave w owning
// rows 16 w .. 16 w + 15, so a page's K and V (16 KB per wave) are requested in one round trip:
//   K   lane = (row 16 w + lane / 4, piece c = lane % 4): dims 32 i + 8 c .. + 7 for i < 8, 8 x 16-byte loads
//   V   lane = head dims 4 lane .. 4 lane + 3, the wave's 16 rows (one 512-byte row per load instruction)
// and the loaded page is reused for every query token of the group (TT tokens: the verify rows).
template <int G, int TT, bool MIX>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
    constexpr int GP = (G + 3) & ~3;
    const int nwg = a.B * a.NKV * a.nsplit;
    const int lid = qs::xcd_logical(blockIdx.x, nwg);
    const int split = lid % a.nsplit;
    const int g = (lid / a.nsplit) % a.NKV;
    const int b = lid / (a.nsplit * a.NKV);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int T = a.T;

    __shared__ __align__(16) uint16_t s_q[TT][G][HD];
    __shared__ __align__(16) uint16_t s_ql[MIX ? TT : 1][G][HD];  // mixer: bf16 residues of the fp32 q
    __shared__ __align__(16) uint32_t s_pp[4][8][GP];
    __shared__ __align__(16) float s_acc[4][G][HD];
    __shared__ float s_m[4][G], s_l[4][G];
    __shared__ float s_w[4][G], s_L[G], s_M[G];

    const int n = a.seq_lens[b];
    if (!user_active(a, n, split == 0 && g == 0 && tid == 0)) {  // uniform over the user's workgroups
        if (split == 0) zero_rows<G>(a, b, g, tid);
        return;
    }
    const int base = n - T;  // first new position
    const int npages = (n + BLK - 1) / BLK;
    const int p0 = split * a.pps;
    const int p1 = min(npages, p0 + a.pps);
    const int *bt = a.block_table + (size_t)b * a.max_blocks;
    // The split's block-table entries (at most 64), one per lane, read once up front: the page walk takes
    // each page index with a readlane and never waits on a table read (a wait for one load would also
    // wait for the K/V loads in flight).
    const int bt_pre = p0 + lane < min(a.max_blocks, p0 + a.pps) ? bt[p0 + lane] : -1;  // issued before n is known
    auto page_at = [&](int pi) {
        const int pg = __builtin_amdgcn_readlane(bt_pre, pi - p0);
        return (pg >= 0 && pg < a.num_blocks) ? pg : -1;
    };
    if (tid == 0)
        for (int pi = p0; pi < p1; ++pi)
            if (page_at(pi) < 0) report_page(a);

    // Fused append, first: the new rows that fall in this split's pages go into the pools, and the stores
    // complete before the barrier that precedes the page walk, so the walk reads every row - new ones
    // included - from the pool. No other workgroup reads these pages.
    if (a.k_new && p0 <= (n - 1) / BLK && base / BLK < p1) {
        for (int idx = tid; idx < T * 64; idx += 256) {  // whole waves: T * 64 is a multiple of 64
            const int t = idx >> 6, kv = (idx >> 5) & 1, ch = idx & 31;
            const int pos = base + t, pi = pos / BLK;
            const size_t src = (((size_t)b * T + t) * a.NKV + g) * HD + ch * 8;
            uint4 u = *reinterpret_cast<const uint4 *>((kv ? a.v_new : a.k_new) + src);
            if (a.wk) {  // k rows normalised and rotated (all lanes take part in the row reductions)
                float y[8];
                const size_t rc = ((size_t)b * T + t) * (a.rot / 2);
                mixer_chunk(u, ch, a.wk, a.rcos + rc, a.rsin + rc, a.rot, a.eps, y);
                if (!kv) u = pack8(y);
            }
            if (pi < p0 || pi >= p1) continue;
            const int pg = bt[pi];  // per thread: the new rows may straddle two pages
            if (pg < 0 || pg >= a.num_blocks) continue;  // reported with the split's pages above
            const size_t dst = (((size_t)pg * a.NKV + g) * BLK + (pos % BLK)) * HD + ch * 8;
            *reinterpret_cast<uint4 *>((kv ? a.v_cache : a.k_cache) + dst) = u;
        }
        qs::wait_vmem();
        __syncthreads();  // the rows are read by the wave that owns their 16-row slice (the branch is uniform)
    }

    const int kq = lane & 3;               // K: this lane's 16-byte piece of each 64-byte run of the row
    const int krw = 16 * w + (lane >> 2);  // K: row of the page this lane scores
    const size_t pstride = (size_t)a.NKV * BLK * HD;  // elements per page
    const float sl2 = a.scale * 1.4426950408889634f;  // scores in the log2 domain: p = 2^(s scale log2e - m)
    const int kvo = krw * HD * 2 + kq * 16;           // bytes: this lane's K piece in a head tile
    const int vvo = 16 * w * HD * 2 + lane * 8;       // bytes: this lane's V dims in the wave's first row

    // Page loads through a buffer descriptor based at the page's head tile (the per-page address work is
    // scalar). A K buffer holds the wave's 16 K rows (4 lanes per row, 8 x 16 bytes per lane); a V buffer
    // its 16 V rows, 4 dims per lane, rows 2 j and 2 j + 1 in entry j (.xy, .zw). Loads only issue here.
    auto load_k = [&](int pg, uint4 (&kb)[8]) {
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(
            qs::uniform_ptr(const_cast<uint16_t *>(a.k_cache + (size_t)pg * pstride + (size_t)g * BLK * HD)), (short)0,
            BLK * HD * 2, 0x00020000);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rk, kvo, i * 64, NT);
            kb[i] = make_uint4(x[0], x[1], x[2], x[3]);
        }
    };
    auto load_v = [&](int pg, uint4 (&vb)[8]) {
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(
            qs::uniform_ptr(const_cast<uint16_t *>(a.v_cache + (size_t)pg * pstride + (size_t)g * BLK * HD)), (short)0,
            BLK * HD * 2, 0x00020000);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const u32x2 x0 = __builtin_amdgcn_raw_buffer_load_b64(rv, vvo, (2 * j) * HD * 2, NT);
            const u32x2 x1 = __builtin_amdgcn_raw_buffer_load_b64(rv, vvo, (2 * j + 1) * HD * 2, NT);
            vb[j] = make_uint4(x0[0], x0[1], x1[0], x1[1]);
        }
    };

    for (int tg = 0; tg < T; tg += TT) {
        const int nt = min(TT, T - tg);
        const int vend = base + tg + nt;  // rows at or past vend are invalid for every token of the group
        const int pe = min(p1, (vend + BLK - 1) / BLK);
        // q of the token group: loaded into registers, then stored to LDS (normalised and rotated for the mixer)
        constexpr int QCH = (TT * G * 32 + 255) / 256;
        uint4 qreg[QCH];
#pragma unroll
        for (int k = 0; k < QCH; ++k) {
            const int idx = tid + 256 * k;
            const int tt = idx / (G * 32), hh = (idx / 32) % G, ch = idx & 31;
            qreg[k] = make_uint4(0, 0, 0, 0);
            if (idx < TT * G * 32 && tt < nt)
                qreg[k] = *reinterpret_cast<const uint4 *>(a.q + (((size_t)b * T + tg + tt) * a.NQ + g * G + hh) * HD + ch * 8);
        }
        auto store_q = [&]() {
            __syncthreads();  // the previous group's readers of s_q are done
#pragma unroll
            for (int k = 0; k < QCH; ++k) {
                const int idx = tid + 256 * k;
                const int tt = idx / (G * 32), hh = (idx / 32) % G, ch = idx & 31;
                uint4 u = qreg[k];
                if constexpr (MIX) {  // normalised and rotated q (all lanes take part in the row reductions)
                    float y[8];
                    const size_t rc = ((size_t)b * T + min(tg + tt, T - 1)) * (a.rot / 2);
                    mixer_chunk(u, ch, a.wq, a.rcos + rc, a.rsin + rc, a.rot, a.eps, y);
                    u = pack8(y);
                    if (idx < TT * G * 32) *reinterpret_cast<uint4 *>(&s_ql[tt][hh][ch * 8]) = pack8_lo(y, u);
                }
                if (idx < TT * G * 32) *reinterpret_cast<uint4 *>(&s_q[tt][hh][ch * 8]) = u;
            }
            __syncthreads();
        };
        store_q();

        // m: running max (log2 domain, wave-uniform); lp: every lane adds its row's rounded probability (so
        // the wave sum is 4x the row sum), reduced over the wave once per split
        float m[TT][G], lp[TT][G], acc[TT][G][4];
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
            for (int h = 0; h < G; ++h) {
                m[tt][h] = -INFINITY;
                lp[tt][h] = 0.f;
                acc[tt][h][0] = acc[tt][h][1] = acc[tt][h][2] = acc[tt][h][3] = 0.f;
            }

        // zero the V rows past every token's window (a stale row times a zero probability could be NaN)
        auto mask_v = [&](int pi, uint4 (&vb)[8]) {
            const int rbase = pi * BLK + 16 * w;
            if (rbase + 15 >= vend) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (rbase + 2 * j >= vend) vb[j].x = vb[j].y = 0;
                    if (rbase + 2 * j + 1 >= vend) vb[j].z = vb[j].w = 0;
                }
            }
        };
        // scores of page pi for token tg + tt, online softmax update, probabilities to s_pp
        auto scores_tt = [&](int pi, int tt, const uint4 (&kv)[8]) {
            const int P = pi * BLK + krw;
            const bool okr = P < base + tg + tt + 1;  // token tg + tt sees positions 0 .. base + tg + tt
            // this lane's row over its 64 dims, then across the row's 4 lanes (the q reads of the 4 lanes
            // are 64 contiguous bytes; all 16 rows read the same q)
            float sc[G];
#pragma unroll
            for (int h = 0; h < G; ++h) sc[h] = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    const uint4 qv = *reinterpret_cast<const uint4 *>(&s_q[tt][h][i * 32 + kq * 8]);
                    float d = sc[h];
                    d = dot2(kv[i].x, qv.x, d);
                    d = dot2(kv[i].y, qv.y, d);
                    d = dot2(kv[i].z, qv.z, d);
                    d = dot2(kv[i].w, qv.w, d);
                    if constexpr (MIX) {
                        const uint4 ql = *reinterpret_cast<const uint4 *>(&s_ql[tt][h][i * 32 + kq * 8]);
                        d = dot2(kv[i].x, ql.x, d);
                        d = dot2(kv[i].y, ql.y, d);
                        d = dot2(kv[i].z, ql.z, d);
                        d = dot2(kv[i].w, ql.w, d);
                    }
                    sc[h] = d;
                }
            }
#pragma unroll
            for (int h = 0; h < G; ++h) {
                sc[h] += qs::dpp<0xB1>(sc[h]);
                sc[h] += qs::dpp<0x4E>(sc[h]);
            }
            // online softmax over the wave's 16 rows (log2 domain; the max is taken on the raw scores, the
            // scale being positive); probabilities rounded to bf16 (the running sum adds the rounded values,
            // so the normalisation matches what P V uses) and packed two rows per dword for P V
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float mn = fmaxf(m[tt][h], qs::wave_max_bcast(okr ? sc[h] : -INFINITY) * sl2);
                const float e = okr ? __builtin_amdgcn_exp2f(fmaf(sc[h], sl2, -mn)) : 0.f;
                const uint32_t pk = qs::cvt_pk_bf16(e, qs::dpp<0x104>(e));  // this row | the next row
                if (mn != m[tt][h]) {  // wave-uniform: rescale only when the running max moved
                    const float alpha = m[tt][h] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[tt][h] - mn);
                    lp[tt][h] *= alpha;
                    acc[tt][h][0] *= alpha;
                    acc[tt][h][1] *= alpha;
                    acc[tt][h][2] *= alpha;
                    acc[tt][h][3] *= alpha;
                    m[tt][h] = mn;
                }
                lp[tt][h] += __uint_as_float(pk << 16);
                if ((lane & 7) == 0) s_pp[w][lane >> 3][h] = pk;
            }
            __builtin_amdgcn_wave_barrier();
        };
        // P V of the page for token tg + tt: two rows per v_dot2 (interleaved with v_perm)
        auto pv_tt = [&](int tt, const uint4 (&vb)[8]) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t x0 = __builtin_amdgcn_perm(vb[j].z, vb[j].x, 0x05040100u);
                const uint32_t x1 = __builtin_amdgcn_perm(vb[j].z, vb[j].x, 0x07060302u);
                const uint32_t x2 = __builtin_amdgcn_perm(vb[j].w, vb[j].y, 0x05040100u);
                const uint32_t x3 = __builtin_amdgcn_perm(vb[j].w, vb[j].y, 0x07060302u);
                uint32_t pr[GP];
#pragma unroll
                for (int h4 = 0; h4 < GP; h4 += 4) {
                    const uint4 p4 = *reinterpret_cast<const uint4 *>(&s_pp[w][j][h4]);
                    pr[h4] = p4.x, pr[h4 + 1] = p4.y, pr[h4 + 2] = p4.z, pr[h4 + 3] = p4.w;
                }
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    acc[tt][h][0] = dot2(pr[h], x0, acc[tt][h][0]);
                    acc[tt][h][1] = dot2(pr[h], x1, acc[tt][h][1]);
                    acc[tt][h][2] = dot2(pr[h], x2, acc[tt][h][2]);
                    acc[tt][h][3] = dot2(pr[h], x3, acc[tt][h][3]);
                }
            }
            __builtin_amdgcn_wave_barrier();
        };

        // the accumulators of TT tokens leave no registers for pages in flight
        for (int pi = p0; pi < pe; ++pi) {
            const int pg = page_at(pi);
            if (pg < 0) continue;
            uint4 X[8], Y[8];
            load_k(pg, X);
            load_v(pg, Y);
            mask_v(pi, Y);
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) {
                if (tt >= nt) break;
                scores_tt(pi, tt, X);
                pv_tt(tt, Y);
            }
        }

        // ---- merge the 4 waves, token by token; one partial (or the output) per token and split
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
            if (tt >= nt) break;
            const int t = tg + tt;
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float lw = 0.25f * qs::wave_sum_dpp(lp[tt][h]);
                *reinterpret_cast<float4 *>(&s_acc[w][h][lane * 4]) =
                    make_float4(acc[tt][h][0], acc[tt][h][1], acc[tt][h][2], acc[tt][h][3]);
                if (lane == 0) {
                    s_m[w][h] = m[tt][h];
                    s_l[w][h] = lw;
                }
            }
            __syncthreads();
            if (tid < G) {
                float M = -INFINITY;
                for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, s_m[ww][tid]);
                float L = 0.f;
                for (int ww = 0; ww < 4; ++ww) {
                    const float e = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[ww][tid] - M);
                    s_w[ww][tid] = e;
                    L += e * s_l[ww][tid];
                }
                s_M[tid] = M;
                s_L[tid] = L;
            }
            __syncthreads();
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float O = s_w[0][h] * s_acc[0][h][tid] + s_w[1][h] * s_acc[1][h][tid] +
                                s_w[2][h] * s_acc[2][h][tid] + s_w[3][h] * s_acc[3][h][tid];
                if (a.nsplit == 1) {
                    const size_t oi = (((size_t)b * T + t) * a.NQ + g * G + h) * HD + tid;
                    const float gt = a.gate ? sigm(qs::bf2f(a.gate[oi])) : 1.0f;
                    a.o[oi] = (uint16_t)qs::f2bf(O / s_L[h] * gt);
                }
                else
                    a.part_o[prow(a, G, b, g, split, t * G + h) * HD + tid] = O;
            }
            if (a.nsplit > 1 && tid < G) {
                float *ml = a.part_ml + prow(a, G, b, g, split, t * G + tid) * 2;
                ml[0] = s_M[tid];
                ml[1] = s_L[tid];
            }
            __syncthreads();
        }
    }
}

// ------------------------------------------------------------------------------ shared by the MFMA kernels
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int QPAD = HD + 8;   // s_q row pitch (bf16): 16-byte skew between rows
constexpr int VPAD = HD + 16;  // K / V slice row pitch (bf16): 32-byte skew between rows
constexpr int PPAD = 16 + 4;   // s_p row pitch (bf16)

// Split merge inside the attention launch (nsplit <= MERGE_MAX). Every workgroup of (user b, KV head g) has
// stored its partial with agent-coherent stores (sc1: written through the XCD's L2); each thread waits for
// its stores to complete, then one thread counts the workgroup in (the count wraps to zero at the last
// arrival). The workgroup that completes the count merges: wave w of NWV takes query rows w, w + NWV, ...
// (two at a time), lane l owns head dims 4 l .. 4 l + 3, and every split's partial and (m, l) are read with agent-coherent loads in one round
// trip. Global max M (log2 domain) and sum L over the splits, weights 2^(m_s - M), O = sum_s w_s O_s / L in
// split order, so the result does not depend on which workgroup finished last. No L2-wide writeback or
// invalidate is needed because only sc1 accesses touch the shared data. (The leader side of the
// reference: kernels/attn_leader_writer.cpp:86-106, kernels/attn_leader_compute.cpp:42-79.)
constexpr int MERGE_MAX = 16;
template <int G, int NWV = 4>
__device__ __forceinline__ void merge_in_launch(const AttnArgs &a, int b, int g, int tid) {
    __shared__ int s_last;
    qs::wait_vmem();
    __syncthreads();
    if (tid == 0) {
        // an increment modulo the splits: the last arrival leaves the count at zero for the next launch
        unsigned *c = reinterpret_cast<unsigned *>(a.cnt) + (size_t)b * a.NKV + g;
        const unsigned ns1 = (unsigned)a.nsplit - 1;
        s_last = __builtin_amdgcn_atomic_inc32(c, ns1, __ATOMIC_RELAXED, "agent") == ns1;
    }
    __syncthreads();
    if (!s_last) return;
    asm volatile("" ::: "memory");
    const int lane = tid & 63, w = tid >> 6;
    const int T = a.T, R = T * G, ns = a.nsplit;
    const auto ro = __builtin_amdgcn_make_buffer_rsrc(qs::uniform_ptr(a.part_o + prow(a, G, b, g, 0, 0) * HD),
                                                      (short)0, ns * R * HD * 4, 0x00020000);
    const auto rm = __builtin_amdgcn_make_buffer_rsrc(qs::uniform_ptr(a.part_ml + prow(a, G, b, g, 0, 0) * 2),
                                                      (short)0, ns * R * 8, 0x00020000);
    for (int r0 = w; r0 < R; r0 += 2 * NWV) {
        f32x4_t x[2][MERGE_MAX];
        float2 ml[2];
        uint2 gw[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int qr = r0 + NWV * j;
            if (qr >= R) continue;
#pragma unroll
            for (int sp = 0; sp < MERGE_MAX; ++sp)
                if (sp < ns)
                    x[j][sp] = __builtin_bit_cast(
                        f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(ro, ((sp * R + qr) * HD + 4 * lane) * 4, 0,
                                                                        qs::CP_SC1));
            ml[j] = make_float2(-INFINITY, 0.f);
            if (lane < ns) {
                const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(rm, (lane * R + qr) * 8, 0, qs::CP_SC1);
                ml[j] = make_float2(__uint_as_float(u[0]), __uint_as_float(u[1]));
            }
            if (a.gate)
                gw[j] = *reinterpret_cast<const uint2 *>(
                    a.gate + (((size_t)b * T + qr / G) * a.NQ + g * G + qr % G) * HD + 4 * lane);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int qr = r0 + NWV * j;
            if (qr >= R) continue;
            const float M = qs::wave_max_bcast(ml[j].x);
            const float e = ml[j].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml[j].x - M);
            const float L = qs::wave_sum_dpp(e * ml[j].y);
            f32x4_t O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int sp = 0; sp < MERGE_MAX; ++sp)
                if (sp < ns) O += qs::lane_val(e, sp) * x[j][sp];
            O *= 1.0f / L;
            if (a.gate) {
                O[0] *= sigm(qs::bf_lo(gw[j].x)), O[1] *= sigm(qs::bf_hi(gw[j].x));
                O[2] *= sigm(qs::bf_lo(gw[j].y)), O[3] *= sigm(qs::bf_hi(gw[j].y));
            }
            *reinterpret_cast<uint2 *>(a.o + (((size_t)b * T + qr / G) * a.NQ + g * G + qr % G) * HD + 4 * lane) =
                make_uint2(qs::cvt_pk_bf16(O[0], O[1]), qs::cvt_pk_bf16(O[2], O[3]));
        }
    }
}

// ------------------------------------------------------------------------------ MFMA kernel (verify rows)
// For T query tokens the T * G query rows of a KV head form a dense [T G x 256] x [256 x rows] product, so
// the multi-token (verify) step runs it on MFMA. One workgroup per (user, KV head, split of pps pages),
// walking its pages in order. Per page, in two phases separated by a barrier:
//   scores  wave w takes rows 16 w .. 16 w + 15 (a 16-row slice): S^T [16 rows x 16 q] = K Q^T on 8
//           v_mfma_f32_16x16x32_bf16 per 16-query-row tile (lane l holds K row l % 16, dims 32 j + 8 (l / 16)
//           .. + 7: one 16-byte load per j), the slice's own max m_s per query row (log2 domain), P^T =
//           2^(s - m_s) rounded to bf16 and its row sums l_s into LDS; the slice's V rows into LDS;
//   P V     every wave adds the 4 slices in order to O^T [its 64 head dims x 16 q] on
//           v_mfma_f32_16x16x16_bf16 (V^T read from LDS with the transposing ds_read_b64_tr_b16, P^T as
//           written), scaled by 2^(m_s - M) against the running max M; M moves only when a slice max exceeds
//           it by 2^8, so the accumulators are rarely rescaled.
// All waves see the same slice maxima in the same order, so M and the sum L agree across waves, and the
// 4 waves' head dims are disjoint: the split's partial needs no cross-wave merge.
template <int G, int QT, bool MIX>
__global__ __launch_bounds__(256) void attn_mfma_kernel(AttnArgs a) {
    constexpr int NQR = 16 * QT;
    const int nwg = a.B * a.NKV * a.nsplit;
    const int lid = qs::xcd_logical(blockIdx.x, nwg);
    const int split = lid % a.nsplit;
    const int g = (lid / a.nsplit) % a.NKV;
    const int b = lid / (a.nsplit * a.NKV);
    // the wave index through readfirstlane: the compiler then knows the wave's page and slice tests are uniform
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, lg = lane >> 4;
    const int T = a.T;

    __shared__ __align__(16) uint16_t s_q[NQR][QPAD];
    __shared__ __align__(16) uint16_t s_ql[MIX ? NQR : 1][QPAD];  // mixer: bf16 residues of the fp32 q
    __shared__ __align__(16) uint16_t s_v[4][16][VPAD];     // the page's V rows, slice by slice
    __shared__ __align__(16) uint16_t s_p[4][QT][16][PPAD];  // P^T of each slice: [query row][slice row]
    __shared__ float s_m[4][NQR], s_l[4][NQR];              // slice max (log2 domain) and row sum
    // Fused append from registers and LDS (up to TN tokens, no mixer): the new rows are requested with the
    // query rows, staged in LDS with them, written over the page's rows as those are used (K in the registers
    // of the score operand, V as it is staged) and stored to the pool after the page loop, so nothing waits for
    // a store and no page is read twice.
    constexpr int TN = MIX ? 0 : (32 / G < 8 ? 32 / G : 8);
    __shared__ __align__(16) uint16_t s_new[TN > 0 ? TN : 1][2][HD];  // token t's new K and V rows

    // Issued first, in this order: the split's block-table entries, the user's length and the query rows.
    // The first page's K / V loads then wait only for the table entries, not for the length.
    const int p0 = split * a.pps;
    const int *bt = a.block_table + (size_t)b * a.max_blocks;
    const int bt_pre = split_entries(a, b, p0, lane);
    int n = a.seq_lens[b];
    // query rows qr = t G + hh (zero past T G): loaded into registers now, stored to LDS once the first
    // page's loads are in flight
    constexpr int QCH = NQR * 32 / 256;
    uint4 qreg[QCH];
#pragma unroll
    for (int k = 0; k < QCH; ++k) {
        const int idx = tid + 256 * k;
        qreg[k] = q_chunk(a, G, b, g, idx >> 5, idx & 31);
    }
    // the new rows, chunk tid % 32 of token tid / 32 (zeros past T, or with more than TN tokens)
    const bool fresh = a.k_new && T <= TN;
    u32x4 nkc = {0u, 0u, 0u, 0u}, nvc = {0u, 0u, 0u, 0u};
    if constexpr (TN > 0) {
        nkc = new_chunk(a, fresh ? a.k_new : nullptr, b, g, tid >> 5, tid & 31);
        nvc = new_chunk(a, fresh ? a.v_new : nullptr, b, g, tid >> 5, tid & 31);
    }

    auto page_at = [&](int pi) {
        const int pg = __builtin_amdgcn_readlane(bt_pre, pi - p0);
        return (pg >= 0 && pg < a.num_blocks) ? pg : -1;
    };
    const size_t pstride = (size_t)a.NKV * BLK * HD;  // elements per page

    // a page of -1 is an empty range: the loads still issue (no branch around them, so the compiler's waits
    // stay exact) and read zeros without touching memory
    auto load_k = [&](int pg, uint4 (&kb)[8]) {
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(
            qs::uniform_ptr(const_cast<uint16_t *>(a.k_cache + (size_t)max(pg, 0) * pstride + (size_t)g * BLK * HD)),
            (short)0, pg >= 0 ? BLK * HD * 2 : 0, 0x00020000);
        const int off = (16 * w + l16) * HD * 2 + lg * 16;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rk, off, j * 64, NT);
            kb[j] = make_uint4(x[0], x[1], x[2], x[3]);
        }
    };
    auto load_v = [&](int pg, uint4 (&vb)[8]) {
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(
            qs::uniform_ptr(const_cast<uint16_t *>(a.v_cache + (size_t)max(pg, 0) * pstride + (size_t)g * BLK * HD)),
            (short)0, pg >= 0 ? BLK * HD * 2 : 0, 0x00020000);
        const int off = (16 * w + (lane >> 5)) * HD * 2 + (lane & 31) * 16;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rv, off, k * 1024, NT);
            vb[k] = make_uint4(x[0], x[1], x[2], x[3]);
        }
    };

    // the first page's rows, before the length is known: a page in the pool's range that turns out to lie
    // past the user's length is simply not used
    uint4 KA[8], VA[8];
    const int pg0 = p0 < a.max_blocks ? page_at(p0) : -1;
    load_k(pg0, KA);
    load_v(pg0, VA);

    if (!user_active(a, n, split == 0 && g == 0 && tid == 0)) {  // uniform over the user's workgroups
        if (split == 0) zero_rows<G>(a, b, g, tid);
        return;
    }
    const int base = n - T;  // first new position
    const int npages = (n + BLK - 1) / BLK;
    const int p1 = min(npages, p0 + a.pps);
    // an entry of the split's pages outside the pool (lane pi - p0 checks entry pi) is reported after the
    // page loop: an atomic here, inside a branch, would make the compiler wait for every load at the next use
    const bool bad_pages = __any(lane < p1 - p0 && (bt_pre < 0 || bt_pre >= a.num_blocks));

    // Fused append otherwise (more tokens, or the mixer's normalised and rotated k rows), first: wave w writes
    // the new rows of its 16-row slices in this split's pages and waits for them, so its slice loads read them
    // back from the pool. No other wave reads these slices.
    if (a.k_new && !fresh && p0 < p1 && base / BLK < p1 && (n - 1) / BLK >= p0) {
        for (int idx = lane; idx < T * 64; idx += 64) {
            const int t = idx >> 6, kv = (idx >> 5) & 1, ch = idx & 31;
            const int pos = base + t, pi = pos / BLK;
            const size_t src = (((size_t)b * T + t) * a.NKV + g) * HD + ch * 8;
            uint4 u = *reinterpret_cast<const uint4 *>((kv ? a.v_new : a.k_new) + src);
            if (a.wk) {  // k rows normalised and rotated (all lanes take part in the row reductions)
                float y[8];
                const size_t rc = ((size_t)b * T + t) * (a.rot / 2);
                mixer_chunk(u, ch, a.wk, a.rcos + rc, a.rsin + rc, a.rot, a.eps, y);
                if (!kv) u = pack8(y);
            }
            if (pi < p0 || pi >= p1 || (pos % BLK) / 16 != w) continue;
            const int pg = bt[pi];
            if (pg < 0 || pg >= a.num_blocks) continue;  // reported with the split's pages above
            const size_t dst = (((size_t)pg * a.NKV + g) * BLK + (pos % BLK)) * HD + ch * 8;
            *reinterpret_cast<uint4 *>((kv ? a.v_cache : a.k_cache) + dst) = u;
        }
        qs::wait_vmem();
        if (pg0 >= 0 && base / BLK <= p0) {  // new rows landed in the first page: read it again
            load_k(pg0, KA);
            load_v(pg0, VA);
        }
    }

    const float sl2 = a.scale * 1.4426950408889634f;  // log2 domain
    int lim[QT];  // the lane's causal limit per query-row tile: token qr / G sees positions <= base + token
#pragma unroll
    for (int nt = 0; nt < QT; ++nt) {
        const int qr = l16 + 16 * nt;
        lim[nt] = qr < T * G ? base + qr / G : -1;
    }

    f32x4_t oacc[QT][4];  // O^T of head dims 64 w + 16 dd + 4 lg + i (dd < 4), query row l16 + 16 nt
    float M[QT], L[QT];
#pragma unroll
    for (int nt = 0; nt < QT; ++nt) {
        M[nt] = -INFINITY;
        L[nt] = 0.f;
#pragma unroll
        for (int dd = 0; dd < 4; ++dd) oacc[nt][dd] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    // Q^T fragments (query row l16 + 16 nt, dims 32 j + 8 lg .. + 7), held in registers for the split once
    // the query rows are staged (with the mixer, whose residues double them, they are read from LDS per page)
    bf16x8_t qbr[MIX ? 1 : QT][MIX ? 1 : 8];

    // one page: scores of this wave's slice into LDS, barrier, every slice's P V into this wave's dims,
    // barrier. kb / vb hold the page's K and V rows; each is refilled with the next page's rows as soon as
    // it has been consumed (V after staging, K after the score MFMAs), so one buffer of each suffices.
    auto page = [&](int pi, uint4 (&kb)[8], uint4 (&vb)[8]) {
        const int pgn = pi + 1 < p1 ? page_at(pi + 1) : -1;
        const bool ok = page_at(pi) >= 0;
        const int r0w = pi * BLK + 16 * w;  // first position of this wave's slice
        // V rows (zero where the page is invalid or past the user's length: a stale row times a zero
        // probability could be NaN)
        // new rows in this wave's slice of the page (uniform): token pos - base at slice row pos - r0w; their
        // LDS reads are issued together, ahead of the staging
        const bool has_new = TN > 0 && fresh && ok && r0w + 16 > base && r0w < n;
        auto stage_v = [&](const u32x4 (&x)[8], bool patch) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int row = 2 * k + (lane >> 5), pos = r0w + row;
                const bool live = ok && pos < n;
                u32x4 v = {live ? vb[k].x : 0u, live ? vb[k].y : 0u, live ? vb[k].z : 0u, live ? vb[k].w : 0u};
                if (patch) v = live && pos >= base ? x[k] : v;
                *reinterpret_cast<u32x4 *>(&s_v[w][row][(lane & 31) * 8]) = v;
            }
        };
        if (TN > 0 && has_new) {
            u32x4 x[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int t = r0w + 2 * k + (lane >> 5) - base;
                x[k] = *reinterpret_cast<const u32x4 *>(&s_new[min(max(t, 0), TN > 0 ? TN - 1 : 0)][1][(lane & 31) * 8]);
            }
            stage_v(x, true);
        } else {
            const u32x4 x[8] = {};
            stage_v(x, false);
        }
        load_v(pgn, vb);
        if constexpr (TN > 0)
            if (has_new) {  // the new K row at this lane's row l16 of the slice, over the pool's (dims 32 j + 8 lg)
                const int t = r0w + l16 - base;
                const bool kp = t >= 0 && r0w + l16 < n;
                u32x4 x[8];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    x[j] = *reinterpret_cast<const u32x4 *>(&s_new[min(max(t, 0), TN - 1)][0][32 * j + 8 * lg]);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    kb[j].x = kp ? x[j][0] : kb[j].x;
                    kb[j].y = kp ? x[j][1] : kb[j].y;
                    kb[j].z = kp ? x[j][2] : kb[j].z;
                    kb[j].w = kp ? x[j][3] : kb[j].w;
                }
            }
        f32x4_t sacc[QT];
#pragma unroll
        for (int nt = 0; nt < QT; ++nt) sacc[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bf16x8_t ak = __builtin_bit_cast(bf16x8_t, kb[j]);
#pragma unroll
            for (int nt = 0; nt < QT; ++nt) {
                bf16x8_t bq;
                if constexpr (MIX)
                    bq = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(&s_q[l16 + 16 * nt][32 * j + 8 * lg]));
                else
                    bq = qbr[nt][j];
                sacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, bq, sacc[nt], 0, 0, 0);
                if constexpr (MIX) {
                    const bf16x8_t bl = __builtin_bit_cast(
                        bf16x8_t, *reinterpret_cast<const uint4 *>(&s_ql[l16 + 16 * nt][32 * j + 8 * lg]));
                    sacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, bl, sacc[nt], 0, 0, 0);
                }
            }
        }
        load_k(pgn, kb);
#pragma unroll
        for (int nt = 0; nt < QT; ++nt) {
            float sc[4];
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sc[i] = ok && r0w + 4 * lg + i <= lim[nt] ? sacc[nt][i] : -INFINITY;
                mx = fmaxf(mx, sc[i]);
            }
            mx = qs::xor32_max(qs::xor16_max(mx));
            const float ms = mx * sl2;  // -inf when no row of the slice is visible to this query row
            float e[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) e[i] = sc[i] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(fmaf(sc[i], sl2, -ms));
            const uint32_t p01 = qs::cvt_pk_bf16(e[0], e[1]), p23 = qs::cvt_pk_bf16(e[2], e[3]);
            *reinterpret_cast<uint2 *>(&s_p[w][nt][l16][4 * lg]) = make_uint2(p01, p23);
            float ls = (qs::bf_lo(p01) + qs::bf_hi(p01)) + (qs::bf_lo(p23) + qs::bf_hi(p23));
            ls = qs::xor32_sum(qs::xor16_sum(ls));
            if (lg == 0) {
                s_m[w][l16 + 16 * nt] = ms;
                s_l[w][l16 + 16 * nt] = ls;
            }
        }
        __syncthreads();
        // P V: the 4 slices in order into this wave's head dims
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            i16x4_t av[4];
#pragma unroll
            for (int dd = 0; dd < 4; ++dd)
                av[dd] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t *)&s_v[q][4 * lg + (l16 >> 2)][16 * (4 * w + dd) + 4 * (l16 & 3)]);
#pragma unroll
            for (int nt = 0; nt < QT; ++nt) {
                const float ms = s_m[q][l16 + 16 * nt], ls = s_l[q][l16 + 16 * nt];
                const bool move = M[nt] == -INFINITY ? ms != -INFINITY : ms > M[nt] + 8.0f;
                const float Mn = move ? ms : M[nt];
                if (__any(move)) {
                    const float alpha = M[nt] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M[nt] - Mn);
                    L[nt] *= alpha;
#pragma unroll
                    for (int dd = 0; dd < 4; ++dd) oacc[nt][dd] *= alpha;
                }
                M[nt] = Mn;
                const float es = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - Mn);
                L[nt] = fmaf(es, ls, L[nt]);
                const i16x4_t pb = __builtin_bit_cast(i16x4_t, *reinterpret_cast<const uint2 *>(&s_p[q][nt][l16][4 * lg]));
#pragma unroll
                for (int dd = 0; dd < 4; ++dd) {
                    const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
                    const f32x4_t pv = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av[dd], pb, z, 0, 0, 0);
                    oacc[nt][dd] += es * pv;
                }
            }
        }
        __syncthreads();  // the next page's scores overwrite s_v, s_p, s_m, s_l
    };

#pragma unroll
    for (int k = 0; k < QCH; ++k) {
        const int idx = tid + 256 * k, qr = idx >> 5, ch = idx & 31;
        uint4 u = qreg[k];
        if constexpr (MIX) {  // normalised and rotated q (all lanes take part in the row reductions)
            float y[8];
            const size_t rc = ((size_t)b * T + min(qr / G, T - 1)) * (a.rot / 2);
            mixer_chunk(u, ch, a.wq, a.rcos + rc, a.rsin + rc, a.rot, a.eps, y);
            u = pack8(y);
            *reinterpret_cast<uint4 *>(&s_ql[qr][ch * 8]) = pack8_lo(y, u);
        }
        *reinterpret_cast<uint4 *>(&s_q[qr][ch * 8]) = u;
    }
    if constexpr (TN > 0)
        if (tid < TN * 32) {
            *reinterpret_cast<u32x4 *>(&s_new[tid >> 5][0][(tid & 31) * 8]) = nkc;
            *reinterpret_cast<u32x4 *>(&s_new[tid >> 5][1][(tid & 31) * 8]) = nvc;
        }
    __syncthreads();
    if constexpr (!MIX)
#pragma unroll
        for (int nt = 0; nt < QT; ++nt)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                qbr[nt][j] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(&s_q[l16 + 16 * nt][32 * j + 8 * lg]));
    for (int pi = p0; pi < p1; ++pi) page(pi, KA, VA);
    if (bad_pages && tid == 0) report_page(a);
    if constexpr (TN > 0)
        if (fresh)  // the new rows of this wave's slices into the pool (lanes < 32 the K row, the others the V row)
#pragma unroll
            for (int t = 0; t < TN; ++t) {
                const int pos = base + t, pi = pos / BLK;
                if (t >= T || pi < p0 || pi >= p1 || (pos % BLK) / 16 != w) continue;
                const int pg = page_at(pi);
                if (pg < 0) continue;  // reported with the split's pages
                const size_t row = (((size_t)pg * a.NKV + g) * BLK + pos % BLK) * HD + (lane & 31) * 8;
                *reinterpret_cast<u32x4 *>((lane < 32 ? a.k_cache : a.v_cache) + row) =
                    *reinterpret_cast<const u32x4 *>(&s_new[t][lane >> 5][(lane & 31) * 8]);
            }

    // this wave's head dims of the split's partial (or of the output); the partials are written through
    // to the agent-coherent level (sc1), where another workgroup of this launch or the merge launch reads them
    const auto rpo = __builtin_amdgcn_make_buffer_rsrc(a.part_o + prow(a, G, b, g, split, 0) * HD, (short)0,
                                                       T * G * HD * 4, 0x00020000);
    const auto rpm = __builtin_amdgcn_make_buffer_rsrc(a.part_ml + prow(a, G, b, g, split, 0) * 2, (short)0,
                                                       T * G * 8, 0x00020000);
#pragma unroll
    for (int nt = 0; nt < QT; ++nt) {
        const int qr = l16 + 16 * nt;
        if (qr >= T * G) continue;
        const int t = qr / G, hh = qr % G;
        if (a.nsplit == 1) {
            const float inv = 1.0f / L[nt];
            const size_t oi = (((size_t)b * T + t) * a.NQ + g * G + hh) * HD + 64 * w + 4 * lg;
#pragma unroll
            for (int dd = 0; dd < 4; ++dd) {
                f32x4_t v = oacc[nt][dd] * inv;
                if (a.gate) {
                    const uint2 gw = *reinterpret_cast<const uint2 *>(a.gate + oi + 16 * dd);
                    v[0] *= sigm(qs::bf_lo(gw.x)), v[1] *= sigm(qs::bf_hi(gw.x));
                    v[2] *= sigm(qs::bf_lo(gw.y)), v[3] *= sigm(qs::bf_hi(gw.y));
                }
                *reinterpret_cast<uint2 *>(a.o + oi + 16 * dd) =
                    make_uint2(qs::cvt_pk_bf16(v[0], v[1]), qs::cvt_pk_bf16(v[2], v[3]));
            }
        } else {
#pragma unroll
            for (int dd = 0; dd < 4; ++dd)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, oacc[nt][dd]), rpo,
                                                       (qr * HD + 64 * w + 16 * dd + 4 * lg) * 4, 0, qs::CP_SC1);
            if (w == 0 && lg == 0)
                __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(M[nt]), __float_as_uint(L[nt])}, rpm,
                                                      qr * 8, 0, qs::CP_SC1);
        }
    }
    if (a.nsplit > 1 && a.nsplit <= MERGE_MAX) merge_in_launch<G>(a, b, g, tid);
}

// ------------------------------------------------------------------- MFMA kernel, independent waves
// Up to 16 query rows per KV head (every one-token decode, and verify steps with T G <= 16). One workgroup per
// (user, KV head, split of pps pages) with 4 WPP waves: wave w owns rows
// 16 (w % 4) .. + 15 of pages p0 + w / 4, p0 + w / 4 + WPP, ... of the split (WPP pages in flight per
// workgroup) and walks them on its own, with no workgroup barrier inside the page loop:
//   scores  S^T [16 rows x 16 q] = K Q^T on 8 v_mfma_f32_16x16x32_bf16 (K rows loaded as whole 512-byte rows
//           and turned into the A operand through the wave's LDS slice; with one page per workgroup, whose
//           chain nothing overlaps, loaded straight in the operand's layout; Q^T held in registers);
//   softmax per query row against the wave's running max M (log2 domain): P = 2^(s - M) rounded to bf16
//           lands, lane for lane, in the B-operand layout of the P V product, so P never leaves the
//           registers; M moves only when a slice max exceeds it by 2^8 (the accumulators are then rescaled),
//           so P <= 2^8;
//   P V     O^T [256 dims x 16 q] += V^T P on 16 v_mfma_f32_16x16x16_bf16, accumulated by the MFMA itself,
//           V^T read from the same LDS slice (now holding the page's 16 V rows) with the transposing
//           ds_read_b64_tr_b16.
// Each wave keeps one page of K and V in flight (refilled as soon as consumed). At the end of the split the
// waves' (max, sum) meet in LDS and their O, scaled to the common max, is summed through LDS in a fixed order
// ((w + 4) pairs first when WPP = 2), every wave summing and storing a share of the head dims; the split's
// partial, or with one split the output, has the layout the in-launch and separate merges read.
constexpr int OPAD = HD + 4;  // fp32 row pitch of the waves' O rows in LDS
template <int G, int WPP, bool MIX>
__global__ __launch_bounds__(256 * WPP, WPP == 1 ? 2 : 1) void attn_wave_kernel(AttnArgs a) {
    constexpr int QT = 1, NQR = 16;
    constexpr int NWV = 4 * WPP, NTH = 64 * NWV;
    const int nwg = a.B * a.NKV * a.nsplit;
    const int lid = qs::xcd_logical(blockIdx.x, nwg);
    const int split = lid % a.nsplit;
    const int g = (lid / a.nsplit) % a.NKV;
    const int b = lid / (a.nsplit * a.NKV);
    // the wave index through readfirstlane: the compiler then knows every page index and page address
    // derived from it is uniform over the wave (else each page load becomes a loop over the lanes' addresses)
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sl = w & 3, ph = w >> 2;  // the wave's 16-row slice and page phase
    const int l16 = lane & 15, lg = lane >> 4;
    const int T = a.T;

    // LDS: the q rows (and the mixer's residues) and the waves' K / V slices during the page loop; after it
    // the same bytes hold 4 waves' scaled O rows
    constexpr int QB = NQR * QPAD * 2, QLB = (MIX ? NQR : 1) * QPAD * 2, KVB = NWV * 16 * VPAD * 2;
    constexpr int OB = 4 * NQR * OPAD * 4;
    constexpr int LB = QB + QLB + KVB > OB ? QB + QLB + KVB : OB;
    __shared__ __align__(16) unsigned char s_raw[LB];
    auto s_q = reinterpret_cast<uint16_t (*)[QPAD]>(s_raw);
    auto s_ql = reinterpret_cast<uint16_t (*)[QPAD]>(s_raw + QB);
    auto s_kv = reinterpret_cast<uint16_t (*)[16][VPAD]>(s_raw + QB + QLB);
    auto s_o = reinterpret_cast<float (*)[NQR][OPAD]>(s_raw);
    __shared__ float s_ml[NWV][NQR][2];
    __shared__ __align__(16) uint16_t s_nk[WPP == 1 && !MIX ? 2 : 1][HD];  // WPP = 1: the new K rows, for the score operand

    const int p0 = split * a.pps;
    const int *bt = a.block_table + (size_t)b * a.max_blocks;
    const int bt_pre = split_entries(a, b, p0, lane);
    const int n = a.seq_lens[b];
    constexpr int QCH = (NQR * 32 + NTH - 1) / NTH;
    uint4 qreg[QCH];
#pragma unroll
    for (int k = 0; k < QCH; ++k) {
        const int idx = tid + NTH * k;
        qreg[k] = q_chunk(a, G, b, g, idx >> 5, idx & 31);  // rows past NQR are never staged
    }
    // The step's new K / V rows (up to TN tokens, which registers allow: two, none with the mixer; more go
    // through the pool below): token t's chunk lane % 32 of the K row (lanes < 32) or of the V row, requested
    // before the pages like the query rows
    constexpr int TN = MIX ? 0 : 2;
    u32x4 nk[TN > 0 ? TN : 1], nv[TN > 0 ? TN : 1];  // vector types (not uint4): selects stay in registers
#pragma unroll
    for (int t = 0; t < TN; ++t) {
        nk[t] = new_chunk(a, a.k_new, b, g, t, lane < 32 ? lane : -1);
        nv[t] = new_chunk(a, a.v_new, b, g, t, lane < 32 ? -1 : lane - 32);
    }
    auto page_at = [&](int pi) {
        const int pg = __builtin_amdgcn_readlane(bt_pre, pi - p0);
        return (pg >= 0 && pg < a.num_blocks) ? pg : -1;
    };
    const size_t pstride = (size_t)a.NKV * BLK * HD;
    // K and V rows load alike, two whole 512-byte rows per instruction (lane: row 2 k + lane / 32, 16 bytes at
    // (lane % 32) 16): a gather of 16-byte pieces of 16 rows per instruction streams ~20% slower
    // (a page of -1 is an empty range: the loads still issue, with no branch around them, so the compiler's
    // waits stay exact, and read zeros without touching memory)
    auto load_rows = [&](const uint16_t *pool, int pg, uint4 (&rb)[8]) {
        const auto r = __builtin_amdgcn_make_buffer_rsrc(
            qs::uniform_ptr(const_cast<uint16_t *>(pool + (size_t)max(pg, 0) * pstride + (size_t)g * BLK * HD)),
            (short)0, pg >= 0 ? BLK * HD * 2 : 0, 0x00020000);
        const int off = (16 * sl + (lane >> 5)) * HD * 2 + (lane & 31) * 16;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, off, k * 1024, NT);
            rb[k] = make_uint4(x[0], x[1], x[2], x[3]);
        }
    };
    // one page per workgroup (WPP = 1): K straight into the score operand's layout (lane: row 16 sl + l16,
    // dims 32 j + 8 lg .. + 7), no staging through LDS
    auto load_kfrag = [&](int pg, uint4 (&rb)[8]) {
        const auto r = __builtin_amdgcn_make_buffer_rsrc(
            qs::uniform_ptr(const_cast<uint16_t *>(a.k_cache + (size_t)max(pg, 0) * pstride + (size_t)g * BLK * HD)),
            (short)0, pg >= 0 ? BLK * HD * 2 : 0, 0x00020000);
        const int off = (16 * sl + l16) * HD * 2 + lg * 16;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, off, j * 64, NT);
            rb[j] = make_uint4(x[0], x[1], x[2], x[3]);
        }
    };
    uint4 KA[8], VA[8];
    const int pf = p0 + ph;  // this wave's first page
    const int pg0 = pf < min(a.max_blocks, p0 + a.pps) ? page_at(pf) : -1;
    if constexpr (WPP == 1)
        load_kfrag(pg0, KA);
    else
        load_rows(a.k_cache, pg0, KA);
    load_rows(a.v_cache, pg0, VA);

    if (!user_active(a, n, split == 0 && g == 0 && tid == 0)) {  // uniform over the user's workgroups
        if (split == 0) zero_rows<G, NTH>(a, b, g, tid);
        return;
    }
    const int base = n - T;
    const int npages = (n + BLK - 1) / BLK;
    const int p1 = min(npages, p0 + a.pps);
    // an entry of the split's pages outside the pool (lane pi - p0 checks entry pi) is reported after the
    // page loop: an atomic here, inside a branch, would make the compiler wait for every load at the next use
    const bool bad_pages = __any(lane < p1 - p0 && (bt_pre < 0 || bt_pre >= a.num_blocks));

    // Fused append. Up to TN tokens: the new rows stay in registers (nk, nv), the page loop writes them over
    // the staged rows of this wave's slices, and they go to the pool after the loop, so no store is in flight
    // while pages load (the compiler would then wait for every load at each use), nothing waits for the
    // stores, and no page is read twice. More tokens: each wave writes the new rows of its own slices to the
    // pool and waits for them before its pages are read (it alone reads them back).
    const bool fresh = a.k_new && T <= TN;
    auto owned = [&](int pos) {  // a new row this wave attends: in one of its pages and in its slice
        const int pi = pos / BLK;
        return pi >= p0 && pi < p1 && (pos % BLK) / 16 == sl && (pi - p0) % WPP == ph;
    };
    if (a.k_new && !fresh && p0 < p1 && base / BLK < p1 && (n - 1) / BLK >= p0) {
        for (int idx = lane; idx < T * 64; idx += 64) {
            const int t = idx >> 6, kv = (idx >> 5) & 1, ch = idx & 31;
            const int pos = base + t, pi = pos / BLK;
            const size_t src = (((size_t)b * T + t) * a.NKV + g) * HD + ch * 8;
            uint4 u = *reinterpret_cast<const uint4 *>((kv ? a.v_new : a.k_new) + src);
            if (a.wk) {
                float y[8];
                const size_t rc = ((size_t)b * T + t) * (a.rot / 2);
                mixer_chunk(u, ch, a.wk, a.rcos + rc, a.rsin + rc, a.rot, a.eps, y);
                if (!kv) u = pack8(y);
            }
            if (!owned(pos)) continue;
            const int pg = bt[pi];
            if (pg < 0 || pg >= a.num_blocks) continue;  // reported with the split's pages above
            const size_t dst = (((size_t)pg * a.NKV + g) * BLK + (pos % BLK)) * HD + ch * 8;
            *reinterpret_cast<uint4 *>((kv ? a.v_cache : a.k_cache) + dst) = u;
        }
        qs::wait_vmem();
        if (pg0 >= 0 && base / BLK <= pf) {  // new rows landed in this wave's first page: read it again
            load_rows(a.k_cache, pg0, KA);
            load_rows(a.v_cache, pg0, VA);
        }
    }

    // q rows (normalised and rotated for the mixer) through LDS into B-operand registers, kept for the split
#pragma unroll
    for (int k = 0; k < QCH; ++k) {
        const int idx = tid + NTH * k, qr = idx >> 5, ch = idx & 31;
        if (qr >= NQR) continue;
        uint4 u = qreg[k];
        if constexpr (MIX) {
            float y[8];
            const size_t rc = ((size_t)b * T + min(qr / G, T - 1)) * (a.rot / 2);
            mixer_chunk(u, ch, a.wq, a.rcos + rc, a.rsin + rc, a.rot, a.eps, y);
            u = pack8(y);
            *reinterpret_cast<uint4 *>(&s_ql[qr][ch * 8]) = pack8_lo(y, u);
        }
        *reinterpret_cast<uint4 *>(&s_q[qr][ch * 8]) = u;
    }
    if constexpr (WPP == 1 && TN > 0)
        if (w == 0 && lane < 32)
#pragma unroll
            for (int t = 0; t < TN; ++t) *reinterpret_cast<u32x4 *>(&s_nk[t][lane * 8]) = nk[t];
    __syncthreads();
    // Q^T fragments, held in registers for the split
    bf16x8_t qb[QT][8], qlo[QT][MIX ? 8 : 1];
#pragma unroll
    for (int nt = 0; nt < QT; ++nt)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            qb[nt][j] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(&s_q[16 * nt + l16][32 * j + 8 * lg]));
            if constexpr (MIX)
                qlo[nt][j] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(&s_ql[16 * nt + l16][32 * j + 8 * lg]));
        }

    const float sl2 = a.scale * 1.4426950408889634f;
    int lim[QT];  // this lane's query row of tile nt sees positions <= lim[nt]
    f32x4_t oacc[QT][16];  // O^T of head dims 16 t + 4 lg + i, query row 16 nt + l16
    float M[QT], L[QT];
#pragma unroll
    for (int nt = 0; nt < QT; ++nt) {
        const int qr = 16 * nt + l16;
        lim[nt] = qr < T * G ? base + qr / G : -1;
        M[nt] = -INFINITY;
        L[nt] = 0.f;
#pragma unroll
        for (int t = 0; t < 16; ++t) oacc[nt][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    for (int pi = pf; pi < p1; pi += WPP) {
        const int pgn = pi + WPP < p1 ? page_at(pi + WPP) : -1;
        const bool ok = page_at(pi) >= 0;
        const int r0w = pi * BLK + 16 * sl;
        f32x4_t sacc[QT];
        if constexpr (WPP == 1) {  // K already in the operand's layout; the new rows patched from LDS
            if (TN > 0 && fresh && base + T > r0w && base < r0w + 16) {  // new rows in this slice (uniform)
                const int t = r0w + l16 - base;
                const bool kp = t >= 0 && t < T;
                u32x4 x[8];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    x[j] = *reinterpret_cast<const u32x4 *>(&s_nk[min(max(t, 0), TN > 0 ? TN - 1 : 0)][32 * j + 8 * lg]);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    KA[j].x = kp ? x[j][0] : KA[j].x;
                    KA[j].y = kp ? x[j][1] : KA[j].y;
                    KA[j].z = kp ? x[j][2] : KA[j].z;
                    KA[j].w = kp ? x[j][3] : KA[j].w;
                }
            }
#pragma unroll
            for (int nt = 0; nt < QT; ++nt) {
                sacc[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const bf16x8_t kb = __builtin_bit_cast(bf16x8_t, KA[j]);
                    sacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, qb[nt][j], sacc[nt], 0, 0, 0);
                    if constexpr (MIX)
                        sacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, qlo[nt][j], sacc[nt], 0, 0, 0);
                }
            }
            load_kfrag(pgn, KA);
        } else {
        // K rows through the wave's LDS slice into the A operand (row l16, dims 32 j + 8 lg .. + 7); the next
        // page's K is requested as soon as the rows are in LDS. Scores of masked rows are replaced below.
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
            *reinterpret_cast<uint4 *>(&s_kv[w][2 * kk + (lane >> 5)][(lane & 31) * 8]) = KA[kk];
        if (fresh)  // the step's new K rows over the staged ones (whatever the pool held there)
#pragma unroll
            for (int t = 0; t < TN; ++t)
                if (t < T && base + t >= r0w && base + t < r0w + 16 && lane < 32)
                    *reinterpret_cast<u32x4 *>(&s_kv[w][base + t - r0w][lane * 8]) = nk[t];
        load_rows(a.k_cache, pgn, KA);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        // K fragments (row l16, dims 32 j + 8 lg .. + 7), each used by every query tile
        constexpr int KG = 8;
#pragma unroll
        for (int nt = 0; nt < QT; ++nt) sacc[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j0 = 0; j0 < 8; j0 += KG) {
            bf16x8_t kb[KG];
#pragma unroll
            for (int j = 0; j < KG; ++j)
                kb[j] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(&s_kv[w][l16][32 * (j0 + j) + 8 * lg]));
#pragma unroll
            for (int nt = 0; nt < QT; ++nt)
#pragma unroll
                for (int j = 0; j < KG; ++j) {
                    sacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb[j], qb[nt][j0 + j], sacc[nt], 0, 0, 0);
                    if constexpr (MIX)
                        sacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb[j], qlo[nt][j0 + j], sacc[nt], 0, 0, 0);
                }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the K reads are done before V overwrites the slice
        }
        // this page's V rows into the slice (zero where invalid or past the length: a stale row times a zero
        // probability could be NaN), then the next page's V into the registers
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            const int row = 2 * kk + (lane >> 5);
            const uint4 v = ok && r0w + row < n ? VA[kk] : make_uint4(0, 0, 0, 0);
            *reinterpret_cast<uint4 *>(&s_kv[w][row][(lane & 31) * 8]) = v;
        }
        if (fresh && ok)  // the new V rows
#pragma unroll
            for (int t = 0; t < TN; ++t)
                if (t < T && base + t >= r0w && base + t < r0w + 16 && lane >= 32)
                    *reinterpret_cast<u32x4 *>(&s_kv[w][base + t - r0w][(lane - 32) * 8]) = nv[t];
        load_rows(a.v_cache, pgn, VA);
        i16x4_t pb[QT];
#pragma unroll
        for (int nt = 0; nt < QT; ++nt) {
            float sc[4], mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sc[i] = ok && r0w + 4 * lg + i <= lim[nt] ? sacc[nt][i] : -INFINITY;
                mx = fmaxf(mx, sc[i]);
            }
            mx = qs::xor32_max(qs::xor16_max(mx));
            const float ms = mx * sl2;  // -inf when no row of the slice is visible to this query row
            const bool move = M[nt] == -INFINITY ? ms != -INFINITY : ms > M[nt] + 8.0f;
            if (__any(move)) {
                const float Mn = move ? ms : M[nt];
                const float alpha = M[nt] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M[nt] - Mn);
                L[nt] *= alpha;
#pragma unroll
                for (int t = 0; t < 16; ++t) oacc[nt][t] *= alpha;
                M[nt] = Mn;
            }
            float e[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) e[i] = sc[i] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(fmaf(sc[i], sl2, -M[nt]));
            const uint32_t p01 = qs::cvt_pk_bf16(e[0], e[1]), p23 = qs::cvt_pk_bf16(e[2], e[3]);
            float ls = (qs::bf_lo(p01) + qs::bf_hi(p01)) + (qs::bf_lo(p23) + qs::bf_hi(p23));
            L[nt] += qs::xor32_sum(qs::xor16_sum(ls));
            pb[nt] = __builtin_bit_cast(i16x4_t, make_uint2(p01, p23));
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the V staging has landed in LDS
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const i16x4_t av = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4_t *)&s_kv[w][4 * lg + (l16 >> 2)][16 * t + 4 * (l16 & 3)]);
#pragma unroll
            for (int nt = 0; nt < QT; ++nt)
                oacc[nt][t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, pb[nt], oacc[nt][t], 0, 0, 0);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the reads are done before the next page's staging
    }

    if (bad_pages && tid == 0) report_page(a);
    if (fresh)  // the new rows this wave attended into the pool (lanes < 32 the K row, the others the V row)
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            const int pos = base + t;
            if (t >= T || !owned(pos)) continue;
            const int pg = page_at(pos / BLK);
            if (pg < 0) continue;  // reported with the split's pages
            const size_t dst = (((size_t)pg * a.NKV + g) * BLK + (pos % BLK)) * HD + (lane & 31) * 8;
            *reinterpret_cast<u32x4 *>((lane < 32 ? a.k_cache : a.v_cache) + dst) = lane < 32 ? nk[t] : nv[t];
        }
    // the waves' (max, sum) per query row; the barrier also frees the q and K / V bytes for the O rows
    if (lg == 0)
#pragma unroll
        for (int nt = 0; nt < QT; ++nt) {
            s_ml[w][16 * nt + l16][0] = M[nt];
            s_ml[w][16 * nt + l16][1] = L[nt];
        }
    __syncthreads();
    auto row_ml = [&](int r, float &Mr, float &Lr) {
        Mr = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < NWV; ++ww) Mr = fmaxf(Mr, s_ml[ww][r][0]);
        Lr = 0.f;
#pragma unroll
        for (int ww = 0; ww < NWV; ++ww) {
            const float mw = s_ml[ww][r][0];
            Lr += (mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - Mr)) * s_ml[ww][r][1];
        }
    };
    const int R = T * G;  // live query rows
    // each wave's O scaled to the common max: waves 4 .. 7 store theirs, then waves 0 .. 3 add their own
    // (WPP = 2); with WPP = 1 every wave stores
#pragma unroll
    for (int stage = 0; stage < WPP; ++stage) {
        if (ph == WPP - 1 - stage) {
#pragma unroll
            for (int nt = 0; nt < QT; ++nt) {
                const int qr = 16 * nt + l16;
                if (qr >= R) continue;
                float Ms, Ls;
                row_ml(qr, Ms, Ls);
                const float sw = M[nt] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M[nt] - Ms);
                f32x4_t *dst = reinterpret_cast<f32x4_t *>(&s_o[sl][qr][4 * lg]);  // + 4 t: head dims 16 t + ..
                if (stage == 0) {
#pragma unroll
                    for (int t = 0; t < 16; ++t) dst[4 * t] = oacc[nt][t] * sw;
                } else {  // every read first, then every write: one LDS round trip, not one per piece
                    f32x4_t prev[16];
#pragma unroll
                    for (int t = 0; t < 16; ++t) prev[t] = dst[4 * t];
#pragma unroll
                    for (int t = 0; t < 16; ++t) dst[4 * t] = oacc[nt][t] * sw + prev[t];
                }
            }
        }
        __syncthreads();
    }
    // wave w: head dims (64 / WPP) w .. of every live row summed over the 4 slots in order
    constexpr int DPW = HD / NWV;      // head dims per wave
    constexpr int PPR = DPW / 4 / 4;   // 16-byte pieces per lane per row (4 lanes per row of a 16-row tile)
    const auto rpo = __builtin_amdgcn_make_buffer_rsrc(a.part_o + prow(a, G, b, g, split, 0) * HD, (short)0,
                                                       R * HD * 4, 0x00020000);
#pragma unroll
    for (int nt = 0; nt < QT; ++nt) {
        const int qr = 16 * nt + l16;
        if (qr >= R) continue;
        const int tt = qr / G, hh = qr % G;
        float Ls = 0.f;
        if (a.nsplit == 1) {
            float Ms;
            row_ml(qr, Ms, Ls);
        }
#pragma unroll
        for (int k = 0; k < PPR; ++k) {
            const int d = DPW * w + 4 * (lg + 4 * k);
            f32x4_t v = *reinterpret_cast<const f32x4_t *>(&s_o[0][qr][d]);
            v += *reinterpret_cast<const f32x4_t *>(&s_o[1][qr][d]);
            v += *reinterpret_cast<const f32x4_t *>(&s_o[2][qr][d]);
            v += *reinterpret_cast<const f32x4_t *>(&s_o[3][qr][d]);
            if (a.nsplit == 1) {
                const size_t oi = (((size_t)b * T + tt) * a.NQ + g * G + hh) * HD + d;
                v *= 1.0f / Ls;
                if (a.gate) {
                    const uint2 gw = *reinterpret_cast<const uint2 *>(a.gate + oi);
                    v[0] *= sigm(qs::bf_lo(gw.x)), v[1] *= sigm(qs::bf_hi(gw.x));
                    v[2] *= sigm(qs::bf_lo(gw.y)), v[3] *= sigm(qs::bf_hi(gw.y));
                }
                *reinterpret_cast<uint2 *>(a.o + oi) = make_uint2(qs::cvt_pk_bf16(v[0], v[1]), qs::cvt_pk_bf16(v[2], v[3]));
            } else {
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rpo, (qr * HD + d) * 4, 0,
                                                       qs::CP_SC1);
            }
        }
    }
    if (a.nsplit > 1 && tid < R) {
        const auto rpm = __builtin_amdgcn_make_buffer_rsrc(a.part_ml + prow(a, G, b, g, split, 0) * 2, (short)0,
                                                           R * 8, 0x00020000);
        float Mr, Lr;
        row_ml(tid, Mr, Lr);
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(Mr), __float_as_uint(Lr)}, rpm, tid * 8, 0,
                                              qs::CP_SC1);
    }
    if (a.nsplit > 1 && a.nsplit <= MERGE_MAX) merge_in_launch<G, NWV>(a, b, g, tid);
}

// Merge of the splits of one output row (user, token, query head) in one memory round trip: wave w sums
// splits w, w + 4, w + 8, ... (lane l owns head dims 4 l .. 4 l + 3), and every wave finds the global max M
// (log2 domain, as the partials store it) and the sum L from all splits' (m, l), whose loads are in flight
// together with the partials. The 4 waves' sums are added in wave order through LDS; every reduction runs
// in a fixed order, so the result is identical run to run. (The leader side of the reference: global max,
// rescale, sum, normalise, kernels/attn_leader_writer.cpp:86-106, kernels/attn_leader_compute.cpp:42-79.)
constexpr int MAX_SPLITS = 1024;
constexpr int MCH = 16;  // splits per wave per batch of loads (64 splits in one round trip)
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnArgs a, int G) {
    __shared__ float4 s_part[4][64];
    const int rowh = blockIdx.x;  // ((b * T + t) * NKV + g) * G + h
    const int h = rowh % G, row = rowh / G;
    const int g = row % a.NKV, bt = row / a.NKV;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ns = a.nsplit, R = a.T * G;
    const int n = a.seq_lens[bt / a.T];
    // The row's partials are requested before the length is checked: their addresses do not depend on it and
    // lie in the workspace either way, so the launch waits for one round trip, not two. Buffer loads, with a
    // wave's split offset in a scalar register and the lane's 16 bytes as the vector offset, need no per-load
    // address arithmetic; the (m, l) of splits past ns lie past the descriptor's range and read zeros.
    const size_t pr = prow(a, G, bt / a.T, g, 0, (bt % a.T) * G + h);
    const int sbytes = R * HD * 4;  // bytes between consecutive splits of one row's O
    const auto rpo = __builtin_amdgcn_make_buffer_rsrc(qs::uniform_ptr(a.part_o + pr * HD), (short)0, ns * sbytes,
                                                       0x00020000);
    const auto rml = __builtin_amdgcn_make_buffer_rsrc(qs::uniform_ptr(a.part_ml + pr * 2), (short)0, ns * R * 8,
                                                       0x00020000);
    auto load_split = [&](int sp, float4 &v, float &m) {  // sp wave-uniform, < ns
        const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(rpo, lane * 16, sp * sbytes, 0);
        v = make_float4(__uint_as_float(u[0]), __uint_as_float(u[1]), __uint_as_float(u[2]), __uint_as_float(u[3]));
        m = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rml, 0, sp * R * 8, 0));
    };
    float4 x[MCH];
    float mw[MCH];
#pragma unroll
    for (int k = 0; k < MCH; ++k) load_split(min(w + 4 * k, ns - 1), x[k], mw[k]);
    // global max and sum over all splits: lane l covers splits l, l + 64, ...
    float M = -INFINITY;
    float2 mg[MAX_SPLITS / 64];
#pragma unroll
    for (int j = 0; j < MAX_SPLITS / 64; ++j) {
        const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(rml, (lane + 64 * j) * R * 8, 0, 0);
        mg[j] = lane + 64 * j < ns ? make_float2(__uint_as_float(u[0]), __uint_as_float(u[1]))
                                   : make_float2(-INFINITY, 0.f);
        M = fmaxf(M, mg[j].x);
    }
    if (n < a.T || n > a.max_blocks * BLK) {  // inactive user (reported by the attention launch): zero row
        if (w == 0)
            *reinterpret_cast<uint2 *>(a.o + ((size_t)bt * a.NQ + g * G + h) * HD + 4 * lane) = make_uint2(0, 0);
        return;
    }
    M = qs::wave_max_bcast(M);
    float L = 0.f;
#pragma unroll
    for (int j = 0; j < MAX_SPLITS / 64; ++j)
        if (mg[j].x != -INFINITY) L += __builtin_amdgcn_exp2f(mg[j].x - M) * mg[j].y;
    L = qs::wave_sum_dpp(L);
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    auto acc = [&](int sp, const float4 &v, float m) {
        if (sp < ns && m != -INFINITY) {
            const float e = __builtin_amdgcn_exp2f(m - M);
            O.x += e * v.x, O.y += e * v.y, O.z += e * v.z, O.w += e * v.w;
        }
    };
#pragma unroll
    for (int k = 0; k < MCH; ++k) acc(w + 4 * k, x[k], mw[k]);
    for (int s0 = 4 * MCH; s0 < ns; s0 += 4 * MCH) {  // further splits, a batch of loads at a time
#pragma unroll
        for (int k = 0; k < MCH; ++k) load_split(min(s0 + w + 4 * k, ns - 1), x[k], mw[k]);
#pragma unroll
        for (int k = 0; k < MCH; ++k) acc(s0 + w + 4 * k, x[k], mw[k]);
    }
    s_part[w][lane] = O;
    __syncthreads();
    if (w != 0) return;
    const float4 p1 = s_part[1][lane], p2 = s_part[2][lane], p3 = s_part[3][lane];
    const float inv = 1.0f / L;
    const float r0 = (((O.x + p1.x) + p2.x) + p3.x) * inv, r1 = (((O.y + p1.y) + p2.y) + p3.y) * inv;
    const float r2 = (((O.z + p1.z) + p2.z) + p3.z) * inv, r3 = (((O.w + p1.w) + p2.w) + p3.w) * inv;
    const size_t oi = ((size_t)bt * a.NQ + g * G + h) * HD + 4 * lane;
    float o0 = r0, o1 = r1, o2 = r2, o3 = r3;
    if (a.gate) {
        const uint2 gw = *reinterpret_cast<const uint2 *>(a.gate + oi);
        o0 *= sigm(qs::bf_lo(gw.x)), o1 *= sigm(qs::bf_hi(gw.x)), o2 *= sigm(qs::bf_lo(gw.y)), o3 *= sigm(qs::bf_hi(gw.y));
    }
    *reinterpret_cast<uint2 *>(a.o + oi) = make_uint2(qs::cvt_pk_bf16(o0, o1), qs::cvt_pk_bf16(o2, o3));
}

int nsplit_of(int max_blocks, int pps) { return (max_blocks + pps - 1) / pps; }
// Pages a workgroup of the independent-wave kernel walks at once (4 waves each): two when the split has more
// than one page (batch 8 at 4096 positions: 26.8 against 27.7 us; batch 1 at 32768: 29.8 against 30.4).
int attn_wpp(int pps) { return pps >= 2 ? 2 : 1; }

}  // namespace

extern "C" size_t qs_paged_attention_workspace_bytes(int B, int T, int NQ, int NKV, int HDa, int max_blocks,
                                                     int pages_per_split) {
    if (B <= 0 || T <= 0 || NKV <= 0 || NQ % NKV || HDa != HD || max_blocks <= 0 || pages_per_split <= 0) return 0;
    const int ns = nsplit_of(max_blocks, pages_per_split);
    return ws_layout(B, T, NKV, NQ / NKV, ns).total;
}

static int attn_launch(AttnArgs a, void *workspace, int HDa, int block, const char *who, void *stream) {
    const int B = a.B, T = a.T, NQ = a.NQ, NKV = a.NKV, max_blocks = a.max_blocks, pages_per_split = a.pps;
    QS_REQUIRE(a.q && a.k_cache && a.v_cache && a.block_table && a.seq_lens && a.o, "%s: null pointer", who);
    QS_REQUIRE((a.k_new == nullptr) == (a.v_new == nullptr), "%s: give both k_new and v_new or neither", who);
    QS_REQUIRE(HDa == HD, "%s: HD must be %d (got %d)", who, HD, HDa);
    QS_REQUIRE(block == BLK, "%s: block must be %d (got %d)", who, BLK, block);
    QS_REQUIRE(B > 0 && T >= 1 && T <= 16, "%s: need B > 0 and 1 <= T <= 16", who);
    QS_REQUIRE(NKV > 0 && NQ > 0 && NQ % NKV == 0, "%s: NQ (%d) must be a multiple of NKV (%d)", who, NQ, NKV);
    QS_REQUIRE(max_blocks > 0 && a.num_blocks > 0, "%s: bad page counts", who);
    QS_REQUIRE(pages_per_split > 0 && pages_per_split <= 64, "%s: pages_per_split must be in [1, 64] (got %d)", who,
               pages_per_split);
    const int G = NQ / NKV;
    const int ns = nsplit_of(max_blocks, pages_per_split);
    QS_REQUIRE(ns == 1 || workspace, "%s: %d splits need a workspace", who, ns);
    QS_REQUIRE(ns <= MAX_SPLITS, "%s: %d splits exceed %d (raise pages_per_split)", who, ns, MAX_SPLITS);
    QS_REQUIRE((long)B * NKV * ns < (1L << 31), "%s: grid too large", who);
    QS_REQUIRE((size_t)B * NKV * sizeof(int) <= CNT_BYTES, "%s: B NKV = %d exceeds %d", who, B * NKV,
               (int)(CNT_BYTES / sizeof(int)));
    a.nsplit = ns;
    if (workspace) {
        const WsLayout L = ws_layout(B, T, NKV, G, ns);
        char *ws = static_cast<char *>(workspace);
        a.cnt = reinterpret_cast<int *>(ws + L.cnt);
        a.part_ml = reinterpret_cast<float *>(ws + L.ml);
        a.part_o = reinterpret_cast<float *>(ws + L.po);
    }
    const dim3 grid(B * NKV * ns);
    hipStream_t st = QS_STREAM(stream);
    // up to 32 query rows per KV head (every one-token decode, and verify steps with T G <= 32) run on MFMA;
    // more rows take the VALU kernel, two query tokens per pass over the pages
    if (T * G <= 32) {
        const int QT = (T * G + 15) / 16;
        // two pages in flight per workgroup (8 waves) when the split has more than one page
        const int wpp = attn_wpp(pages_per_split);
#define QS_WAVE(GG, W, MX) attn_wave_kernel<GG, W, MX><<<grid, 256 * W, 0, st>>>(a)
#define QS_MFMA_LAUNCH(GG)                                                              \
    if (a.wq) {                                                                         \
        if (QT == 1) { if (wpp == 1) QS_WAVE(GG, 1, true); else QS_WAVE(GG, 2, true); }  \
        else attn_mfma_kernel<GG, 2, true><<<grid, 256, 0, st>>>(a);                    \
    } else {                                                                            \
        if (QT == 1) { if (wpp == 1) QS_WAVE(GG, 1, false); else QS_WAVE(GG, 2, false); } \
        else attn_mfma_kernel<GG, 2, false><<<grid, 256, 0, st>>>(a);                   \
    }
        switch (G) {
            case 1: QS_MFMA_LAUNCH(1) break;
            case 2: QS_MFMA_LAUNCH(2) break;
            case 4: QS_MFMA_LAUNCH(4) break;
            case 6: QS_MFMA_LAUNCH(6) break;
            case 8: QS_MFMA_LAUNCH(8) break;
            default: QS_REQUIRE(false, "%s: group size NQ/NKV = %d not in {1, 2, 4, 6, 8}", who, G);
        }
#undef QS_MFMA_LAUNCH
#undef QS_WAVE
        if (int e = qs::launch_status(who)) return e;
        if (ns > MERGE_MAX) {  // fewer splits are merged inside the attention launch
            attn_merge_kernel<<<B * T * NKV * G, 256, 0, st>>>(a, G);
            return qs::launch_status(who);
        }
        return QS_OK;
    }
#define QS_ATTN_LAUNCH(GG)                                \
    if (a.wq) attn_kernel<GG, 2, true><<<grid, 256, 0, st>>>(a); \
    else attn_kernel<GG, 2, false><<<grid, 256, 0, st>>>(a);
    switch (G) {
        case 1: QS_ATTN_LAUNCH(1) break;
        case 2: QS_ATTN_LAUNCH(2) break;
        case 4: QS_ATTN_LAUNCH(4) break;
        case 6: QS_ATTN_LAUNCH(6) break;
        case 8: QS_ATTN_LAUNCH(8) break;
        default: QS_REQUIRE(false, "%s: group size NQ/NKV = %d not in {1, 2, 4, 6, 8}", who, G);
    }
#undef QS_ATTN_LAUNCH
    if (int e = qs::launch_status(who)) return e;
    if (ns > 1) {
        attn_merge_kernel<<<B * T * NKV * G, 256, 0, st>>>(a, G);
        return qs::launch_status(who);
    }
    return QS_OK;
}

extern "C" int qs_paged_gqa_decode(const uint16_t *q, const uint16_t *k_new, const uint16_t *v_new,
                                   uint16_t *k_cache, uint16_t *v_cache, const int *block_table, const int *seq_lens,
                                   uint16_t *o, void *workspace, int B, int T, int NQ, int NKV, int HDa, int block,
                                   int max_blocks, int num_blocks, int pages_per_split, float scale, int *status,
                                   void *stream) {
    AttnArgs a{};
    a.status = status;
    a.q = q, a.k_new = k_new, a.v_new = v_new, a.k_cache = k_cache, a.v_cache = v_cache;
    a.block_table = block_table, a.seq_lens = seq_lens, a.o = o;
    a.B = B, a.T = T, a.NQ = NQ, a.NKV = NKV, a.max_blocks = max_blocks, a.num_blocks = num_blocks;
    a.pps = pages_per_split, a.scale = scale;
    return attn_launch(a, workspace, HDa, block, "qs_paged_gqa_decode", stream);
}

extern "C" int qs_attn_mixer_decode(const uint16_t *q, const uint16_t *k_new, const uint16_t *v_new,
                                    const uint16_t *gate, const float *wq, const float *wk, const float *rope_cos,
                                    const float *rope_sin, int rot, uint16_t *k_cache, uint16_t *v_cache,
                                    const int *block_table, const int *seq_lens, uint16_t *o, void *workspace, int B,
                                    int T, int NQ, int NKV, int HDa, int block, int max_blocks, int num_blocks,
                                    int pages_per_split, float eps, int *status, void *stream) {
    QS_REQUIRE(k_new && v_new && gate && wq && wk, "qs_attn_mixer_decode: null pointer");
    QS_REQUIRE(rot == 0 || (rope_cos && rope_sin), "qs_attn_mixer_decode: rot > 0 needs rope_cos and rope_sin");
    QS_REQUIRE(rot == 0 || rot == 16 || rot == 32 || rot == 64 || rot == 128 || rot == 256,
               "qs_attn_mixer_decode: rot must be 0, 16, 32, 64, 128 or 256 (got %d)", rot);
    QS_REQUIRE(eps > 0.f, "qs_attn_mixer_decode: eps must be positive");
    QS_REQUIRE(((uintptr_t)wq | (uintptr_t)wk) % 16 == 0, "qs_attn_mixer_decode: wq and wk must be 16-byte aligned");
    AttnArgs a{};
    a.q = q, a.k_new = k_new, a.v_new = v_new, a.k_cache = k_cache, a.v_cache = v_cache;
    a.block_table = block_table, a.seq_lens = seq_lens, a.o = o;
    a.B = B, a.T = T, a.NQ = NQ, a.NKV = NKV, a.max_blocks = max_blocks, a.num_blocks = num_blocks;
    a.pps = pages_per_split, a.scale = 1.0f;  // the softmax scale is folded into wq (model.py:237)
    a.gate = gate, a.wq = wq, a.wk = wk, a.rcos = rope_cos, a.rsin = rope_sin, a.rot = rot, a.eps = eps;
    a.status = status;
    return attn_launch(a, workspace, HDa, block, "qs_attn_mixer_decode", stream);
}
