// Paged KV-cache movement on gfx950: decode append (T rows per user through the block table), prefill
// fill (paged_fill_cache) and its inverse, the gather of a sequence's pages into contiguous rows, and the
// step's length advance. Pure byte copies in 16-byte units; page indices read from device memory are
// range-checked in the kernel (a row whose page is out of range is skipped, never written out of bounds,
// and reported in the caller's status word when one is given).
#include "qs_common.h"

namespace {

// thread i copies 16-byte chunk (i % cpr) of row (i / cpr); rows are ordered (b, t, kv head)
__global__ __launch_bounds__(256) void append_kernel(const uint16_t *k, const uint16_t *v, uint16_t *kc,
                                                     uint16_t *vc, const int *block_table, const int *positions,
                                                     int B, int T, int NKV, int HD, int block, int max_blocks,
                                                     int num_blocks, int *status) {
    const int cpr = HD / 8;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    const long total = (long)B * T * NKV * cpr;
    if (i >= total) return;
    const int ch = (int)(i % cpr);
    const long r = i / cpr;
    const int hk = (int)(r % NKV);
    const long bt = r / NKV;
    const int t = (int)(bt % T);
    const int b = (int)(bt / T);
    if (positions[b] < 0) return;  // idle slot
    const int p = positions[b] + t;
    const int bi = p / block;
    const bool report = ch == 0 && hk == 0;  // one report per row
    if (bi >= max_blocks) {
        if (report && status) atomicOr(status, QS_STATUS_LENGTH);
        return;
    }
    const int page = block_table[(long)b * max_blocks + bi];
    if (page < 0 || page >= num_blocks) {
        if (report && status) atomicOr(status, QS_STATUS_PAGE);
        return;
    }
    const size_t dst = (((size_t)page * NKV + hk) * block + p % block) * HD + ch * 8;
    const size_t src = (size_t)r * HD + ch * 8;
    if (k) *reinterpret_cast<uint4 *>(kc + dst) = *reinterpret_cast<const uint4 *>(k + src);
    if (v) *reinterpret_cast<uint4 *>(vc + dst) = *reinterpret_cast<const uint4 *>(v + src);
}

// x [NKV, T, HD]: thread i copies chunk (i % cpr) of token ((i / cpr) % T), kv head (i / cpr / T), from x
// into its page (fill) or from its page into x (gather; a token whose page is out of range reads zeros)
template <bool GATHER>
__global__ __launch_bounds__(256) void fill_kernel(const uint16_t *k, const uint16_t *v, uint16_t *kc, uint16_t *vc,
                                                   uint16_t *ko, uint16_t *vo, const int *page_table, int T,
                                                   int start, int NKV, int HD, int block, int table_len,
                                                   int num_blocks) {
    const int cpr = HD / 8;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    const long total = (long)NKV * T * cpr;
    if (i >= total) return;
    const int ch = (int)(i % cpr);
    const long r = i / cpr;
    const int tok = (int)(r % T);
    const int hk = (int)(r / T);
    const int p = start + tok;
    const int bi = p / block;
    const int page = bi < table_len ? page_table[bi] : -1;
    const bool ok = page >= 0 && page < num_blocks;
    const size_t pg = (((size_t)page * NKV + hk) * block + p % block) * HD + ch * 8;
    const size_t x = (size_t)r * HD + ch * 8;
    if (GATHER) {
        const uint4 z = make_uint4(0, 0, 0, 0);
        if (ko) *reinterpret_cast<uint4 *>(ko + x) = ok ? *reinterpret_cast<const uint4 *>(kc + pg) : z;
        if (vo) *reinterpret_cast<uint4 *>(vo + x) = ok ? *reinterpret_cast<const uint4 *>(vc + pg) : z;
    } else if (ok) {
        if (k) *reinterpret_cast<uint4 *>(kc + pg) = *reinterpret_cast<const uint4 *>(k + x);
        if (v) *reinterpret_cast<uint4 *>(vc + pg) = *reinterpret_cast<const uint4 *>(v + x);
    }
}

}  // namespace

extern "C" int qs_paged_kv_append(const uint16_t *k, const uint16_t *v, uint16_t *k_cache, uint16_t *v_cache,
                                  const int *block_table, const int *positions, int B, int T, int NKV, int HD,
                                  int block, int max_blocks, int num_blocks, int *status, void *stream) {
    QS_REQUIRE(k && v && k_cache && v_cache && block_table && positions, "qs_paged_kv_append: null pointer");
    QS_REQUIRE(B > 0 && T > 0 && NKV > 0 && block > 0 && max_blocks > 0 && num_blocks > 0,
               "qs_paged_kv_append: sizes must be positive");
    QS_REQUIRE(HD > 0 && HD % 8 == 0, "qs_paged_kv_append: HD must be a multiple of 8 (got %d)", HD);
    const long total = (long)B * T * NKV * (HD / 8);
    if (total == 0) return QS_OK;
    append_kernel<<<(unsigned)((total + 255) / 256), 256, 0, QS_STREAM(stream)>>>(
        k, v, k_cache, v_cache, block_table, positions, B, T, NKV, HD, block, max_blocks, num_blocks, status);
    return qs::launch_status("qs_paged_kv_append");
}

extern "C" int qs_paged_kv_fill(const uint16_t *k, const uint16_t *v, uint16_t *k_cache, uint16_t *v_cache,
                                const int *page_table, int T, int start, int NKV, int HD, int block, int table_len,
                                int num_blocks, void *stream) {
    QS_REQUIRE(page_table, "qs_paged_kv_fill: null page table");
    QS_REQUIRE((k == nullptr) == (k_cache == nullptr) && (v == nullptr) == (v_cache == nullptr) && (k || v),
               "qs_paged_kv_fill: give k with k_cache and/or v with v_cache");
    QS_REQUIRE(T >= 0 && start >= 0 && NKV > 0 && block > 0 && table_len > 0 && num_blocks > 0,
               "qs_paged_kv_fill: bad sizes");
    QS_REQUIRE(HD > 0 && HD % 8 == 0, "qs_paged_kv_fill: HD must be a multiple of 8 (got %d)", HD);
    QS_REQUIRE((long)(start + T + block - 1) / block <= table_len,
               "qs_paged_kv_fill: %d tokens from %d need more than the %d table entries", T, start, table_len);
    const long total = (long)NKV * T * (HD / 8);
    if (total == 0) return QS_OK;
    fill_kernel<false><<<(unsigned)((total + 255) / 256), 256, 0, QS_STREAM(stream)>>>(
        k, v, k_cache, v_cache, nullptr, nullptr, page_table, T, start, NKV, HD, block, table_len, num_blocks);
    return qs::launch_status("qs_paged_kv_fill");
}

extern "C" int qs_paged_kv_gather(const uint16_t *k_cache, const uint16_t *v_cache, const int *page_table,
                                  uint16_t *k, uint16_t *v, int T, int start, int NKV, int HD, int block,
                                  int table_len, int num_blocks, void *stream) {
    QS_REQUIRE(page_table, "qs_paged_kv_gather: null page table");
    QS_REQUIRE((k == nullptr) == (k_cache == nullptr) && (v == nullptr) == (v_cache == nullptr) && (k || v),
               "qs_paged_kv_gather: give k with k_cache and/or v with v_cache");
    QS_REQUIRE(T >= 0 && start >= 0 && NKV > 0 && block > 0 && table_len > 0 && num_blocks > 0,
               "qs_paged_kv_gather: bad sizes");
    QS_REQUIRE(HD > 0 && HD % 8 == 0, "qs_paged_kv_gather: HD must be a multiple of 8 (got %d)", HD);
    QS_REQUIRE((long)(start + T + block - 1) / block <= table_len,
               "qs_paged_kv_gather: %d tokens from %d need more than the %d table entries", T, start, table_len);
    const long total = (long)NKV * T * (HD / 8);
    if (total == 0) return QS_OK;
    fill_kernel<true><<<(unsigned)((total + 255) / 256), 256, 0, QS_STREAM(stream)>>>(
        nullptr, nullptr, const_cast<uint16_t *>(k_cache), const_cast<uint16_t *>(v_cache), k, v, page_table, T,
        start, NKV, HD, block, table_len, num_blocks);
    return qs::launch_status("qs_paged_kv_gather");
}

// The step's position advance (ResidentModel.step moves every user's position by the rows it decodes,
// model.py:1314-1351, :1499-1508): base_out[b] <- lens[b] (the cached rows before the step, nullable) and
// lens[b] <- lens[b] + T for every user with lens[b] >= 0 (a negative length marks an idle slot and is left
// as it is). A length that would pass max_len (the block table's capacity, model.py's max_pos and
// generator_vllm.py:94's max_model_len assert) is still advanced, so every attention launch of the step
// treats the user as invalid, and QS_STATUS_LENGTH is set in status.
namespace {
__global__ void advance_kernel(int *lens, int *base_out, int B, int T, int max_len, int *status) {
    const int b = blockIdx.x * 64 + threadIdx.x;
    if (b >= B) return;
    const int n = lens[b];
    if (base_out) base_out[b] = n;
    if (n < 0) return;
    if (n + T > max_len && status) atomicOr(status, QS_STATUS_LENGTH);
    lens[b] = n + T;
}
}  // namespace

extern "C" int qs_advance_lengths(int *lens, int *base_out, int B, int T, int max_len, int *status, void *stream) {
    QS_REQUIRE(lens, "qs_advance_lengths: null lens");
    QS_REQUIRE(B > 0 && T >= 1 && max_len > 0, "qs_advance_lengths: bad sizes (B %d, T %d, max_len %d)", B, T, max_len);
    QS_REQUIRE(base_out != lens, "qs_advance_lengths: base_out must not alias lens");
    advance_kernel<<<(B + 63) / 64, 64, 0, QS_STREAM(stream)>>>(lens, base_out, B, T, max_len, status);
    return qs::launch_status("qs_advance_lengths");
}
