// Paged GQA decode attention on gfx950 (HD 256, block 64): split-K over block-table pages, online softmax
// per wavefront, ordered in-kernel merge, optional fused append of the step's new K/V rows.
//
// Grid: one workgroup per (user, KV head, split); a split is `pps` consecutive block-table entries. The 4
// waves of a workgroup stream pages p0 + w, p0 + w + 4, ... independently (no workgroup barrier inside the
// page loop), each keeping its own running max m, sum l and o for the G query heads of the KV head (GQA
// reuse: every K/V byte is loaded once for all G heads):
//   scores  8 lanes per position, 32 dims per lane (16-byte loads at 128-byte row offsets, so one load
//           instruction reads eight whole 128-byte lines), packed bf16 dot products (v_dot2_f32_bf16),
//           3-step lane butterfly; scores and probabilities staged in the wave's LDS slice
//   softmax one position per lane: wave max / sum, rescale of the running state
//   P V     4 head dims per lane (one 512-byte V row per load instruction), fp32 FMA
// The waves are merged in LDS; splits are merged through a fan-in-8 tree of self-resetting counters: the
// last workgroup to finish a group of 8 merges it in a fixed order (the reference's fan-in-8 reduction
// tree, kernels/attn_compute_common.hpp:123-151), so results are identical run to run.
#include "qs_common.h"

namespace {

constexpr int HD = 256;
constexpr int BLK = 64;
constexpr int FANIN = 8;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

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
    float *part_o;                      // [B, T, NKV, slots, G, HD]
    float *part_ml;                     // [B, T, NKV, slots, G, 2]
    int *counters;                      // [B, NKV, slots]
    int B, T, NQ, NKV, max_blocks, num_blocks, pps, nsplit, slots;
    float scale;
};

// Workspace layout (bytes): counters | part_ml | part_o, each 256-byte aligned.
struct WsLayout {
    size_t cnt, ml, po, total;
};
__host__ __device__ inline WsLayout ws_layout(int B, int T, int NKV, int G, int slots) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    WsLayout l;
    l.cnt = 0;
    l.ml = up((size_t)B * NKV * slots * 4);
    l.po = l.ml + up((size_t)B * T * NKV * slots * G * 2 * 4);
    l.total = l.po + up((size_t)B * T * NKV * slots * G * HD * 4);
    return l;
}

template <int G>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
    constexpr int GP = (G + 3) & ~3;
    const int nwg = a.B * a.NKV * a.nsplit;
    const int lid = qs::xcd_logical(blockIdx.x, nwg);
    const int split = lid % a.nsplit;
    const int g = (lid / a.nsplit) % a.NKV;
    const int b = lid / (a.nsplit * a.NKV);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int T = a.T;

    __shared__ __align__(16) uint16_t s_q[G][HD];
    __shared__ __align__(16) float s_p[4][BLK][GP];
    __shared__ __align__(16) float s_acc[4][G][HD];
    __shared__ float s_m[4][G], s_l[4][G];
    __shared__ float s_w[FANIN][G], s_L[G], s_M[G];
    __shared__ int s_last;

    int n = a.seq_lens[b];
    n = n < T ? T : (n > a.max_blocks * BLK ? a.max_blocks * BLK : n);
    const int base = n - T;  // first new position
    const int npages = (n + BLK - 1) / BLK;
    const int p0 = split * a.pps;
    const int p1 = min(npages, p0 + a.pps);
    const int *bt = a.block_table + (size_t)b * a.max_blocks;
    auto page_of = [&](int pi) {
        const int pg = bt[pi];
        return (pg >= 0 && pg < a.num_blocks) ? pg : -1;
    };

    // Fused append: the new rows that fall in this split's pages go into the pools. Attention below reads
    // those rows from k_new / v_new, never from the pool, so there is no write-read hazard.
    if (a.k_new) {
        for (int idx = tid; idx < T * 64; idx += 256) {
            const int t = idx >> 6, kv = (idx >> 5) & 1, ch = idx & 31;
            const int pos = base + t, pi = pos / BLK;
            if (pi < p0 || pi >= p1) continue;
            const int pg = page_of(pi);
            if (pg < 0) continue;
            const size_t dst = (((size_t)pg * a.NKV + g) * BLK + (pos % BLK)) * HD + ch * 8;
            const size_t src = (((size_t)b * T + t) * a.NKV + g) * HD + ch * 8;
            const uint16_t *s = kv ? a.v_new : a.k_new;
            uint16_t *d = kv ? a.v_cache : a.k_cache;
            *reinterpret_cast<uint4 *>(d + dst) = *reinterpret_cast<const uint4 *>(s + src);
        }
    }

    const int c = lane & 7, r = lane >> 3;
    for (int t = 0; t < T; ++t) {
        const int valid = base + t + 1;  // positions 0 .. valid-1
        const int pe = min(p1, (valid + BLK - 1) / BLK);
        __syncthreads();
        for (int idx = tid; idx < G * 32; idx += 256) {
            const int hh = idx >> 5, ch = idx & 31;
            *reinterpret_cast<uint4 *>(&s_q[hh][ch * 8]) = *reinterpret_cast<const uint4 *>(
                a.q + (((size_t)b * T + t) * a.NQ + g * G + hh) * HD + ch * 8);
        }
        __syncthreads();

        float m[G], l[G], acc[G][4];
#pragma unroll
        for (int h = 0; h < G; ++h) {
            m[h] = -INFINITY;
            l[h] = 0.f;
            acc[h][0] = acc[h][1] = acc[h][2] = acc[h][3] = 0.f;
        }

        for (int pi = p0 + w; pi < pe; pi += 4) {
            const int pg = page_of(pi);
            if (pg < 0) continue;
            const uint16_t *kp = a.k_cache + ((size_t)pg * a.NKV + g) * BLK * HD;
            const uint16_t *vp = a.v_cache + ((size_t)pg * a.NKV + g) * BLK * HD;
            const int pbase = pi * BLK;
            auto krow = [&](int pp) -> const uint16_t * {
                const int P = pbase + pp;
                if (a.k_new && P >= base) return a.k_new + (((size_t)b * T + (P - base)) * a.NKV + g) * HD;
                return kp + (size_t)pp * HD;
            };
            auto vrow = [&](int pp) -> const uint16_t * {
                const int P = pbase + pp;
                if (a.v_new && P >= base) return a.v_new + (((size_t)b * T + (P - base)) * a.NKV + g) * HD;
                return vp + (size_t)pp * HD;
            };

            // ---- scores: 8 passes of 8 positions, 4 passes' loads in flight at a time
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                uint4 kv[4][4];
#pragma unroll
                for (int ps = 0; ps < 4; ++ps) {
                    const int pp = (half * 4 + ps) * 8 + r;
                    const uint16_t *src = krow(pp) + c * 8;
                    const bool ok = pbase + pp < valid;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        kv[ps][i] = ok ? *reinterpret_cast<const uint4 *>(src + 64 * i) : make_uint4(0, 0, 0, 0);
                }
#pragma unroll
                for (int ps = 0; ps < 4; ++ps) {
                    const int pp = (half * 4 + ps) * 8 + r;
                    float d[G];
#pragma unroll
                    for (int h = 0; h < G; ++h) d[h] = 0.f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
#pragma unroll
                        for (int h = 0; h < G; ++h) {
                            const uint4 qv = *reinterpret_cast<const uint4 *>(&s_q[h][c * 8 + 64 * i]);
                            d[h] = dot2(kv[ps][i].x, qv.x, d[h]);
                            d[h] = dot2(kv[ps][i].y, qv.y, d[h]);
                            d[h] = dot2(kv[ps][i].z, qv.z, d[h]);
                            d[h] = dot2(kv[ps][i].w, qv.w, d[h]);
                        }
                    }
#pragma unroll
                    for (int h = 0; h < G; ++h) {
                        d[h] += __shfl_xor(d[h], 1, 64);
                        d[h] += __shfl_xor(d[h], 2, 64);
                        d[h] += __shfl_xor(d[h], 4, 64);
                    }
                    if (c == 0) {
                        const bool ok = pbase + pp < valid;
#pragma unroll
                        for (int h = 0; h < G; ++h) s_p[w][pp][h] = ok ? d[h] * a.scale : -INFINITY;
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();

            // ---- online softmax: lane = position
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float x = s_p[w][lane][h];
                const float mn = fmaxf(m[h], qs::wave_max(x));
                const float e = x == -INFINITY ? 0.f : expf(x - mn);
                const float alpha = m[h] == -INFINITY ? 0.f : expf(m[h] - mn);
                l[h] = l[h] * alpha + qs::wave_sum(e);
                m[h] = mn;
                s_p[w][lane][h] = e;
                acc[h][0] *= alpha;
                acc[h][1] *= alpha;
                acc[h][2] *= alpha;
                acc[h][3] *= alpha;
            }
            __builtin_amdgcn_wave_barrier();

            // ---- P V: 16 rows' loads in flight at a time
            const int np = min(BLK, valid - pbase);
            for (int j0 = 0; j0 < np; j0 += 16) {
                uint2 vv[16];
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    vv[j] = (j0 + j < np) ? *reinterpret_cast<const uint2 *>(vrow(j0 + j) + lane * 4)
                                          : make_uint2(0, 0);
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const float v0 = qs::bf_lo(vv[j].x), v1 = qs::bf_hi(vv[j].x);
                    const float v2 = qs::bf_lo(vv[j].y), v3 = qs::bf_hi(vv[j].y);
                    float pr[GP];
#pragma unroll
                    for (int h4 = 0; h4 < GP; h4 += 4) {
                        const float4 p4 = *reinterpret_cast<const float4 *>(&s_p[w][j0 + j][h4]);
                        pr[h4] = p4.x, pr[h4 + 1] = p4.y, pr[h4 + 2] = p4.z, pr[h4 + 3] = p4.w;
                    }
#pragma unroll
                    for (int h = 0; h < G; ++h) {
                        acc[h][0] += pr[h] * v0;
                        acc[h][1] += pr[h] * v1;
                        acc[h][2] += pr[h] * v2;
                        acc[h][3] += pr[h] * v3;
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
        }

        // ---- merge the 4 waves of this workgroup
#pragma unroll
        for (int h = 0; h < G; ++h) {
            *reinterpret_cast<float4 *>(&s_acc[w][h][lane * 4]) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
            if (lane == 0) {
                s_m[w][h] = m[h];
                s_l[w][h] = l[h];
            }
        }
        __syncthreads();
        if (tid < G) {
            float M = -INFINITY;
            for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, s_m[ww][tid]);
            float L = 0.f;
            for (int ww = 0; ww < 4; ++ww) {
                const float e = M == -INFINITY ? 0.f : expf(s_m[ww][tid] - M);
                s_w[ww][tid] = e;
                L += e * s_l[ww][tid];
            }
            s_M[tid] = M;
            s_L[tid] = L;
        }
        __syncthreads();
        const size_t row = ((size_t)b * T + t) * a.NKV + g;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float O = s_w[0][h] * s_acc[0][h][tid] + s_w[1][h] * s_acc[1][h][tid] +
                            s_w[2][h] * s_acc[2][h][tid] + s_w[3][h] * s_acc[3][h][tid];
            if (a.nsplit == 1) {
                a.o[(((size_t)b * T + t) * a.NQ + g * G + h) * HD + tid] = (uint16_t)qs::f2bf(O / s_L[h]);
            } else {
                a.part_o[((row * a.slots + split) * G + h) * HD + tid] = O;
            }
        }
        if (a.nsplit > 1 && tid < G) {
            float *ml = a.part_ml + ((row * a.slots + split) * G + tid) * 2;
            ml[0] = s_M[tid];
            ml[1] = s_L[tid];
        }
    }
    if (a.nsplit == 1) return;

    // ---- fan-in-8 merge tree over the splits of (b, g)
    int idx = split, off = 0, cnt_n = a.nsplit;
    while (cnt_n > 1) {
        const int grp = idx / FANIN, nxt = off + cnt_n, nn = (cnt_n + FANIN - 1) / FANIN;
        const int members = min(FANIN, cnt_n - grp * FANIN);
        __threadfence();
        __syncthreads();
        if (tid == 0) {
            int *cnt = a.counters + ((size_t)b * a.NKV + g) * a.slots + nxt + grp;
            const int old = atomicAdd(cnt, 1);
            const int last = old == members - 1;
            if (last) atomicExch(cnt, 0);
            s_last = last;
        }
        __syncthreads();
        if (!s_last) return;
        __threadfence();
        for (int t = 0; t < T; ++t) {
            const size_t row = ((size_t)b * T + t) * a.NKV + g;
            const size_t src0 = row * a.slots + off + grp * FANIN;
            if (tid < G) {
                float M = -INFINITY;
                for (int i = 0; i < members; ++i) M = fmaxf(M, a.part_ml[((src0 + i) * G + tid) * 2]);
                float L = 0.f;
                for (int i = 0; i < members; ++i) {
                    const float *ml = a.part_ml + ((src0 + i) * G + tid) * 2;
                    const float e = M == -INFINITY ? 0.f : expf(ml[0] - M);
                    s_w[i][tid] = e;
                    L += e * ml[1];
                }
                s_M[tid] = M;
                s_L[tid] = L;
            }
            __syncthreads();
#pragma unroll
            for (int h = 0; h < G; ++h) {
                float O = 0.f;
                for (int i = 0; i < members; ++i) O += s_w[i][h] * a.part_o[((src0 + i) * G + h) * HD + tid];
                if (nn == 1)
                    a.o[(((size_t)b * T + t) * a.NQ + g * G + h) * HD + tid] = (uint16_t)qs::f2bf(O / s_L[h]);
                else
                    a.part_o[((row * a.slots + nxt + grp) * G + h) * HD + tid] = O;
            }
            if (nn > 1 && tid < G) {
                float *ml = a.part_ml + ((row * a.slots + nxt + grp) * G + tid) * 2;
                ml[0] = s_M[tid];
                ml[1] = s_L[tid];
            }
            __syncthreads();
        }
        idx = grp;
        off = nxt;
        cnt_n = nn;
    }
}

int nsplit_of(int max_blocks, int pps) { return (max_blocks + pps - 1) / pps; }
int slots_of(int nsplit) {
    int s = 0, n = nsplit;
    while (n > 1) {
        s += n;
        n = (n + FANIN - 1) / FANIN;
    }
    return s + 1;
}

}  // namespace

extern "C" size_t qs_paged_attention_workspace_bytes(int B, int T, int NQ, int NKV, int HDa, int max_blocks,
                                                     int pages_per_split) {
    if (B <= 0 || T <= 0 || NKV <= 0 || NQ % NKV || HDa != HD || max_blocks <= 0 || pages_per_split <= 0) return 0;
    const int ns = nsplit_of(max_blocks, pages_per_split);
    return ws_layout(B, T, NKV, NQ / NKV, slots_of(ns)).total;
}

extern "C" int qs_paged_gqa_decode(const uint16_t *q, const uint16_t *k_new, const uint16_t *v_new,
                                   uint16_t *k_cache, uint16_t *v_cache, const int *block_table, const int *seq_lens,
                                   uint16_t *o, void *workspace, int B, int T, int NQ, int NKV, int HDa, int block,
                                   int max_blocks, int num_blocks, int pages_per_split, float scale, void *stream) {
    QS_REQUIRE(q && k_cache && v_cache && block_table && seq_lens && o, "qs_paged_gqa_decode: null pointer");
    QS_REQUIRE((k_new == nullptr) == (v_new == nullptr), "qs_paged_gqa_decode: give both k_new and v_new or neither");
    QS_REQUIRE(HDa == HD, "qs_paged_gqa_decode: HD must be %d (got %d)", HD, HDa);
    QS_REQUIRE(block == BLK, "qs_paged_gqa_decode: block must be %d (got %d)", BLK, block);
    QS_REQUIRE(B > 0 && T >= 1 && T <= 16, "qs_paged_gqa_decode: need B > 0 and 1 <= T <= 16");
    QS_REQUIRE(NKV > 0 && NQ > 0 && NQ % NKV == 0, "qs_paged_gqa_decode: NQ (%d) must be a multiple of NKV (%d)",
               NQ, NKV);
    QS_REQUIRE(max_blocks > 0 && num_blocks > 0 && pages_per_split > 0, "qs_paged_gqa_decode: bad page counts");
    const int G = NQ / NKV;
    const int ns = nsplit_of(max_blocks, pages_per_split);
    QS_REQUIRE(ns == 1 || workspace, "qs_paged_gqa_decode: %d splits need a workspace", ns);
    QS_REQUIRE((long)B * NKV * ns < (1L << 31), "qs_paged_gqa_decode: grid too large");
    AttnArgs a{};
    a.q = q, a.k_new = k_new, a.v_new = v_new, a.k_cache = k_cache, a.v_cache = v_cache;
    a.block_table = block_table, a.seq_lens = seq_lens, a.o = o;
    a.B = B, a.T = T, a.NQ = NQ, a.NKV = NKV, a.max_blocks = max_blocks, a.num_blocks = num_blocks;
    a.pps = pages_per_split, a.nsplit = ns, a.slots = slots_of(ns), a.scale = scale;
    if (workspace) {
        const WsLayout L = ws_layout(B, T, NKV, G, a.slots);
        char *ws = static_cast<char *>(workspace);
        a.counters = reinterpret_cast<int *>(ws + L.cnt);
        a.part_ml = reinterpret_cast<float *>(ws + L.ml);
        a.part_o = reinterpret_cast<float *>(ws + L.po);
    }
    const dim3 grid(B * NKV * ns);
    hipStream_t st = QS_STREAM(stream);
    switch (G) {
        case 1: attn_kernel<1><<<grid, 256, 0, st>>>(a); break;
        case 2: attn_kernel<2><<<grid, 256, 0, st>>>(a); break;
        case 4: attn_kernel<4><<<grid, 256, 0, st>>>(a); break;
        case 6: attn_kernel<6><<<grid, 256, 0, st>>>(a); break;
        case 8: attn_kernel<8><<<grid, 256, 0, st>>>(a); break;
        default: QS_REQUIRE(false, "qs_paged_gqa_decode: group size NQ/NKV = %d not in {1, 2, 4, 6, 8}", G);
    }
    return qs::launch_status("qs_paged_gqa_decode");
}
