// Bandwidth probes of the MI355X memory system (measurement only; no counterpart in the reference): the
// ceilings the state-path kernels are compared against, each the bare access pattern of one kernel family.
//   read    a wave per 16 KB chunk, 16 nontemporal 1 KB buffer loads in flight (64 lanes x 16 bytes each, whole
//           128-byte lines), chunks grid-strided over the buffer: the streaming-read ceiling (the attention's
//           K / V pages, the projections' weights);
//   copy    the same chunk loads, then the chunk stored with the GDN state's policy (nontemporal, written
//           through the L2), in place or to a second buffer: the read + write ceiling (the GDN state);
//   gather  the paged attention's access pattern without its compute: one workgroup per (user, KV head, split
//           of pps block-table pages), 8 waves, each streaming 16-row slices (two whole 512-byte rows per load
//           instruction) of the K and V tiles of its pages through one register buffer, as attn_wave_kernel
//           loads them.
// Every loaded value is folded into a per-thread checksum that decides a store to `sink` (the store happens
// only when the checksum hits a fixed pattern, but the compiler cannot know that), so no load can be dropped.
#include "qs_common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int CHUNK = 16384;  // bytes per wave per step
constexpr int NCU = 256, WAVES_PER_CU = 32;

__device__ __forceinline__ uint32_t fold(u32x4 v) { return v[0] ^ v[1] ^ v[2] ^ v[3]; }

__global__ __launch_bounds__(1024) void read_kernel(const char *src, size_t nchunks, uint32_t *sink) {
    const int lane = threadIdx.x & 63, wpb = blockDim.x >> 6;
    const size_t wave = (size_t)blockIdx.x * wpb + (threadIdx.x >> 6);
    const size_t nwaves = (size_t)gridDim.x * wpb;
    uint32_t acc = 0;
    for (size_t c = wave; c < nchunks; c += nwaves) {
        const auto r = __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(qs::uniform_ptr(src + c * CHUNK)),
                                                         (short)0, CHUNK, 0x00020000);
        u32x4 v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16, k * 1024, qs::CP_NT);
#pragma unroll
        for (int k = 0; k < 16; ++k) acc ^= fold(v[k]);
    }
    if (acc == 0x9e3779b9u) sink[wave] = acc;
}

__global__ __launch_bounds__(1024) void copy_kernel(const char *src, char *dst, size_t nchunks) {
    const int lane = threadIdx.x & 63, wpb = blockDim.x >> 6;
    const size_t wave = (size_t)blockIdx.x * wpb + (threadIdx.x >> 6);
    const size_t nwaves = (size_t)gridDim.x * wpb;
    for (size_t c = wave; c < nchunks; c += nwaves) {
        const auto r = __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(qs::uniform_ptr(src + c * CHUNK)),
                                                         (short)0, CHUNK, 0x00020000);
        const auto w = __builtin_amdgcn_make_buffer_rsrc(qs::uniform_ptr(dst + c * CHUNK), (short)0, CHUNK, 0x00020000);
        u32x4 v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16, k * 1024, qs::CP_NT);
#pragma unroll
        for (int k = 0; k < 16; ++k)
            __builtin_amdgcn_raw_buffer_store_b128(v[k], w, lane * 16, k * 1024, qs::CP_NT | qs::CP_SC1);
    }
}

constexpr int BLK = 64, HD = 256;
// One workgroup per (user b, KV head g, split of pps pages); wave w streams rows 16 (w % 4) .. + 15 of pages
// p0 + w / 4, p0 + w / 4 + 2, ... of the split, the next page's K and V requested while the current one is
// consumed (the attention kernel's load schedule, the block-table entries read once per split into a
// register, without its LDS staging and MFMA work). An entry outside the pool reads zeros.
__global__ __launch_bounds__(512) void gather_kernel(const uint16_t *k_cache, const uint16_t *v_cache,
                                                     const int *block_table, int B, int NKV, int max_blocks,
                                                     int npages, int num_blocks, int pps, int nsplit, uint32_t *sink) {
    const int lid = qs::xcd_logical(blockIdx.x, B * NKV * nsplit);
    const int split = lid % nsplit, g = (lid / nsplit) % NKV, b = lid / (nsplit * NKV);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, sl = w & 3, ph = w >> 2;
    const int p0 = split * pps, p1 = min(npages, p0 + pps);
    const int bt_pre = p0 + lane < p1 ? block_table[(size_t)b * max_blocks + p0 + lane] : -1;
    const size_t pstride = (size_t)NKV * BLK * HD;
    const int off = (16 * sl + (lane >> 5)) * HD * 2 + (lane & 31) * 16;
    auto load = [&](const uint16_t *pool, int pi, u32x4 (&x)[8]) {
        const int pg = __builtin_amdgcn_readlane(bt_pre, pi - p0);
        const bool ok = pg >= 0 && pg < num_blocks;
        const auto r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t *>(pool + (ok ? (size_t)pg * pstride + (size_t)g * BLK * HD : 0)), (short)0,
            ok ? BLK * HD * 2 : 0, 0x00020000);
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = __builtin_amdgcn_raw_buffer_load_b128(r, off, k * 1024, qs::CP_NT);
    };
    uint32_t acc = 0;
    u32x4 K[8], V[8];
    int pi = p0 + ph;
    if (pi < p1) {
        load(k_cache, pi, K);
        load(v_cache, pi, V);
    }
    for (; pi < p1; pi += 2) {
        const bool more = pi + 2 < p1;
#pragma unroll
        for (int k = 0; k < 8; ++k) acc ^= fold(K[k]);
        if (more) load(k_cache, pi + 2, K);
#pragma unroll
        for (int k = 0; k < 8; ++k) acc ^= fold(V[k]);
        if (more) load(v_cache, pi + 2, V);
    }
    if (acc == 0x9e3779b9u) sink[blockIdx.x * 8 + w] = acc;
}

// Waves spread evenly over the 256 CUs: one workgroup per CU of nchunks / 256 waves (at most 16) when that
// divides, else 4-wave workgroups, a chunk per wave up to WAVES_PER_CU waves per CU and grid-strided beyond.
struct ProbeGrid {
    int blocks, threads;
};
ProbeGrid probe_grid(size_t nchunks) {
    if (nchunks % NCU == 0 && nchunks / NCU <= 16) return {NCU, (int)(nchunks / NCU) * 64};
    const size_t waves = nchunks < (size_t)NCU * WAVES_PER_CU ? nchunks : (size_t)NCU * WAVES_PER_CU;
    return {(int)((waves + 3) / 4), 256};
}

}  // namespace

extern "C" size_t qs_probe_sink_words(size_t bytes) {
    const ProbeGrid g = probe_grid((bytes + CHUNK - 1) / CHUNK);
    return (size_t)g.blocks * (g.threads / 64);
}

extern "C" int qs_probe_read(const void *src, size_t bytes, uint32_t *sink, void *stream) {
    QS_REQUIRE(src && sink, "qs_probe_read: null pointer");
    QS_REQUIRE(bytes >= CHUNK && bytes % CHUNK == 0, "qs_probe_read: bytes must be a positive multiple of %d", CHUNK);
    const size_t n = bytes / CHUNK;
    const ProbeGrid g = probe_grid(n);
    read_kernel<<<g.blocks, g.threads, 0, QS_STREAM(stream)>>>(static_cast<const char *>(src), n, sink);
    return qs::launch_status("qs_probe_read");
}

extern "C" int qs_probe_copy(const void *src, void *dst, size_t bytes, void *stream) {
    QS_REQUIRE(src && dst, "qs_probe_copy: null pointer");
    QS_REQUIRE(bytes >= CHUNK && bytes % CHUNK == 0, "qs_probe_copy: bytes must be a positive multiple of %d", CHUNK);
    const size_t n = bytes / CHUNK;
    const ProbeGrid g = probe_grid(n);
    copy_kernel<<<g.blocks, g.threads, 0, QS_STREAM(stream)>>>(static_cast<const char *>(src), static_cast<char *>(dst), n);
    return qs::launch_status("qs_probe_copy");
}

extern "C" size_t qs_probe_gather_sink_words(int B, int NKV, int max_blocks, int pps) {
    if (B <= 0 || NKV <= 0 || max_blocks <= 0 || pps <= 0) return 0;
    return (size_t)B * NKV * ((max_blocks + pps - 1) / pps) * 8;
}

extern "C" int qs_probe_gather(const uint16_t *k_cache, const uint16_t *v_cache, const int *block_table, int B,
                               int NKV, int max_blocks, int npages, int num_blocks, int pps, uint32_t *sink,
                               void *stream) {
    QS_REQUIRE(k_cache && v_cache && block_table && sink, "qs_probe_gather: null pointer");
    QS_REQUIRE(B > 0 && NKV > 0 && max_blocks > 0 && num_blocks > 0 && npages > 0 && npages <= max_blocks &&
                   pps > 0 && pps <= 64,
               "qs_probe_gather: bad shape");
    const int nsplit = (max_blocks + pps - 1) / pps;
    QS_REQUIRE((long)B * NKV * nsplit < (1L << 31), "qs_probe_gather: grid too large");
    gather_kernel<<<B * NKV * nsplit, 512, 0, QS_STREAM(stream)>>>(k_cache, v_cache, block_table, B, NKV, max_blocks,
                                                                    npages, num_blocks, pps, nsplit, sink);
    return qs::launch_status("qs_probe_gather");
}
