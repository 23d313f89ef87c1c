/*
 * qwen_state.h — C ABI of the MI355X (gfx950) decode-time state path of the hybrid Gated-DeltaNet /
 * full-attention Qwen3.6-27B engine (libqwen_state.so).
 *
 * Conventions shared by every entry point:
 *   - all data pointers are DEVICE memory owned by the caller; bf16 tensors are passed as uint16_t bit
 *     patterns, fp32 as float, indices as int32;
 *   - every call takes the HIP stream (hipStream_t, passed as void*) it enqueues on, returns 0 on success,
 *     QS_EINVAL for an argument the library rejects (the message is in qs_last_error()), QS_EHIP for a HIP
 *     launch error; no call allocates device memory, synchronises the host or records a memset, so every
 *     call can be captured into a HIP graph;
 *   - state tensors are updated in place where the reference updates them in place
 *     (kernels/gdn_head_writer.cpp:109-114, kernels/attn_worker_writer.cpp:128-139);
 *   - workspaces are caller-owned device buffers of the size the matching *_workspace_bytes() returns,
 *     ZEROED ONCE before first use; the kernels leave them zeroed again (self-resetting counters), so one
 *     workspace serves every later call on the same stream. Calls that run concurrently must not share a
 *     workspace.
 *
 * Reference interfaces replaced are cited as path:line into sott0n/tt-qwen-resident.
 *
 * Layouts:
 *   conv state   [B, C, K-1] bf16, oldest input first; taps [C, K] bf16 (tap 0 multiplies the oldest)
 *   GDN state    [B, NV, DK, DV] fp32, S[k][v] row-major; value head h uses key head h / (NV / NK)
 *   q|k|v        conv channels q (NK*DK) | k (NK*DK) | v (NV*DV)
 *   KV pool      [num_blocks, NKV, block, HD] bf16; position p of user b lives in page
 *                block_table[b * max_blocks + p / block], row p % block
 */
#ifndef QWEN_STATE_H
#define QWEN_STATE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QS_OK 0
#define QS_EINVAL (-1)
#define QS_EHIP (-2)

/* Bits of the optional device status word (int32, caller-owned, zeroed by the caller; kernels OR bits into
 * it and never clear it). Entry points that read lengths, positions, block-table entries or accept lengths
 * from device memory take a nullable `int *status`: with it, an invalid value is reported there (the host
 * reads the word after the step, as the reference's asserts stop a bad step, generator_vllm.py:94); with or
 * without it the kernel handles the value in the documented, bounded way and exits normally. */
#define QS_STATUS_LENGTH 1 /* a length or position past the block table (max_blocks * block rows) */
#define QS_STATUS_PAGE 2   /* a block-table entry needed for a valid position outside [0, num_blocks) */
#define QS_STATUS_ACCEPT 4 /* an accept length outside [1, T] */

/* ABI version (bumped when a signature changes) and the last error message of the calling thread. */
int qs_abi_version(void);
const char *qs_last_error(void);

/* ---------------------------------------------------------------------------------------- a1: conv1d
 * Causal depthwise conv1d update + SiLU for one token per user, state shifted in place.
 * Replaces the conv pass of the streamer (kernels/streamer_compute.cpp:275-370, ring order
 * kernels/streamer_common.hpp:158-166) whose torch statement is model.py:255-259.
 *   x [B, C] bf16, conv_state [B, C, K-1] bf16 (in/out), taps [C, K] bf16 -> y [B, C] bf16.  K == 4. */
int qs_conv1d_update(const uint16_t *x, uint16_t *conv_state, const uint16_t *taps, uint16_t *y, int B, int C,
                     int K, void *stream);

/* ---------------------------------------------------------------------------------------- a3: gates
 * g = neg_a * softplus(a + dt_bias) (threshold 20), beta = sigmoid(b) per (user, value head).
 * Replaces the gate stage of kernels/gdn_head_compute.cpp:198-243 (torch model.py:268-269).
 *   a, b [B, NV] bf16; dt_bias, neg_a [NV] fp32 -> g, beta [B, NV] fp32. */
int qs_gdn_gates(const uint16_t *a, const uint16_t *b, const float *dt_bias, const float *neg_a, float *g,
                 float *beta, int B, int NV, void *stream);

/* ---------------------------------------------------------------------------------------- a2+a4: delta rule
 * One gated delta rule decode step from post-conv q, k, v: L2-norm of q (times scale) and k, then
 * delta = beta (v - (e^g k)^T S), S <- e^g S + k delta^T (in place), o = q^T S.
 * Replaces the GDN head cores (kernels/gdn_head_compute.cpp:180-350, reader :105-212, writer :39-122;
 * torch model.py:262-273).
 *   q, k [B, NK, DK] bf16; v [B, NV, DV] bf16; g, beta [B, NV] fp32; state [B, NV, DK, DV] fp32 (in/out)
 *   -> o [B, NV, DV] bf16.  DK == DV == 128, NV % NK == 0. */
int qs_gdn_decode_step(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *g, const float *beta,
                       float *state, uint16_t *o, int B, int NK, int NV, int DK, int DV, float scale, float eps,
                       void *stream);

/* Workspace of qs_gdn_decode_fused: two self-resetting counters (q and k channels) per (user, key head). */
size_t qs_gdn_workspace_bytes(int B, int NK);

/* Conv1d update + L2-norm + delta rule of one decode step in one launch (a1+a2+a4): the GDN mixer state
 * path of torch_step model.py:255-273 behind the projection. x [B, C] is the projection's q|k|v slice
 * (C = 2 NK DK + NV DV); conv_state is shifted in place; y_out (nullable) receives the conv output.
 * z, norm_w (both nullable; f1, the mixer's epilogue, model.py:274-275, kernels/gdn_head_compute.cpp:320-346):
 * with them o receives bf16(o rsqrt(mean(o^2) + eps) norm_w silu(z)) per value head, normalised from the
 * fp32 o as the reference does, instead of bf16(o); z is the projection's z slice, row b at z + b ldz
 * (NV DV values; ldz >= NV DV, a multiple of 4, z 8-byte aligned), norm_w [DV] fp32 (16-byte aligned).
 * eps is the L2-norm's and the RMSNorm's (both 1e-6 in the reference, model.py:264-267, common.py:15).
 * lens (nullable, [B] device int32, the step's sequence lengths): a user with lens[b] < 0 is an idle slot
 * whose state, conv history and output are left untouched. */
int qs_gdn_decode_fused(const uint16_t *x, uint16_t *conv_state, const uint16_t *taps, const float *g,
                        const float *beta, float *state, uint16_t *o, uint16_t *y_out, const uint16_t *z, int ldz,
                        const float *norm_w, void *workspace, const int *lens, int B, int NK, int NV, int DK, int DV,
                        int K, float scale, float eps, void *stream);

/* qs_gdn_decode_fused for callers that cannot allocate (code under HIP graph capture, serving loops that
 * forbid hipMalloc): the same kernels, with the conv counters in a static device array of the library
 * (64 KB per device, held until the process ends) instead of a workspace. No counterpart in the reference.
 * B * NK <= 8192 (QS_EINVAL beyond). No call allocates or frees device memory; the first call on a device
 * looks the array up and clears it with a fill kernel on the given stream. Every call on one device shares
 * the array, so calls that overlap on a device (concurrent streams) race. */
int qs_gdn_decode_fused_noalloc(const uint16_t *x, uint16_t *conv_state, const uint16_t *taps, const float *g,
                                const float *beta, float *state, uint16_t *o, uint16_t *y_out, const int *lens,
                                int B, int NK, int NV, int DK, int DV, int K, float scale, float eps, void *stream);

/* Diagnostics of qs_gdn_decode_fused_noalloc (no counterpart in the reference; for tests and for callers that
 * want to check the library's counters are at rest between calls): copies the first n (1 <= n <= 16384)
 * ints of the current device's static counter array into dst (device memory) on the stream. Allocates
 * nothing. */
int qs_gdn_noalloc_scratch_read(int *dst, int n, void *stream);

/* Gated RMSNorm epilogue of the GDN mixer (the path's edge, torch model.py:274-275): for each row of DV
 * values, out = bf16(o * rsqrt(mean(o^2) + eps) * norm_w * silu(z)). o, z, out [rows, DV] bf16 (rows = B * NV,
 * or B * T * NV after a verify step; z is the projection's z slice), norm_w [DV] fp32. Replaces steps 7-8
 * of the GDN head cores (kernels/gdn_head_compute.cpp:320-346). */
int qs_gdn_gated_norm(const uint16_t *o, const uint16_t *z, const float *norm_w, uint16_t *out, int rows, int DV,
                      float eps, void *stream);

/* ---------------------------------------------------------------------------------------- a7: verify
 * T tokens per user (1 <= T <= 8) through conv + delta rule in sequence, keeping every intermediate:
 *   x [B, T, C] bf16; conv_state_in [B, C, K-1]; g, beta [B, T, NV]; state_in [B, NV, DK, DV]
 *   -> conv_states_out [T, B, C, K-1], states_out [T, B, NV, DK, DV], o [B, T, NV, DV], y_out (nullable)
 *   [B, T, C]. Inputs are not modified.
 * lens (nullable, [B] device int32, the step's lengths): a user with lens[b] < 0 is an idle slot, for which
 * nothing is computed or written.
 * Replaces the verify rows of the GDN head cores (kernels/gdn_head_reader.cpp:149-187,
 * gdn_head_writer.cpp:60-66, :109) and the conv pair-slot ring (kernels/streamer_common.hpp:38-44). */
int qs_gdn_verify_step(const uint16_t *x, const uint16_t *conv_state_in, uint16_t *conv_states_out,
                       const uint16_t *taps, const float *g, const float *beta, const float *state_in,
                       float *states_out, uint16_t *o, uint16_t *y_out, const int *lens, int B, int T, int NK,
                       int NV, int DK, int DV, int K, float scale, float eps, void *stream);

/* The verify step reading each user's input from a slot of the previous verify step's snapshots, so a
 * rollback costs no copy (the reference's slot select: kernels/gdn_head_reader.cpp:17-20, :149-187, the
 * conv pair slots kernels/streamer_common.hpp:38-44): user b's state and conv history are slot in_slot[b]
 * of states_in [n_slots, B, NV, DK, DV] and conv_states_in [n_slots, B, C, K-1]; in_slot [B] int32 is
 * device memory (a slot outside [0, n_slots) reads slot 0). Outputs as qs_gdn_verify_step; they must not
 * alias the inputs (callers alternate two snapshot sets). An idle slot (lens non-null, lens[b] < 0) verifies
 * no token: its input state and conv history are copied unchanged into the same slot of the outputs (when
 * that slot is below T), which the next step reads, since the acceptance leaves an idle slot's slot as it is. */
int qs_gdn_verify_step_slots(const uint16_t *x, const uint16_t *conv_states_in, uint16_t *conv_states_out,
                             const uint16_t *taps, const float *g, const float *beta, const float *states_in,
                             float *states_out, const int *in_slot, int n_slots, uint16_t *o, uint16_t *y_out,
                             const int *lens, int B, int T, int NK, int NV, int DK, int DV, int K, float scale,
                             float eps, void *stream);

/* Acceptance without copies: slot[b] <- accept_len[b] - 1 (the snapshot the next verify step reads) and,
 * when seq_lens is non-null, seq_lens[b] <- base_lens[b] + accept_len[b] (the KV truncation), for
 * accept_len[b] in [1, T]; a user with another accept length is left untouched and reported
 * (QS_STATUS_ACCEPT). An idle slot (base_lens non-null, base_lens[b] < 0) keeps its slot and length.
 * Replaces the hub's slot/ring advance (kernels/mlp_hub.cpp:48-58; model.py:1314-1318). */
int qs_verify_accept(const int *accept_len, int *slot, int *seq_lens, const int *base_lens, int B, int T,
                     int *status, void *stream);

/* Rollback after verify: state[b] <- states_out[accept_len[b]-1, b], conv_state[b] <- conv_states_out[...]
 * (bit-exact copies), and, when seq_lens is non-null, seq_lens[b] <- base_lens[b] + accept_len[b] (the KV
 * truncation; no KV bytes move). accept_len is device memory, 1 <= accept_len[b] <= T; an idle slot
 * (base_lens non-null, base_lens[b] < 0) is left untouched.
 * Replaces the slot/ring advance of the hub (kernels/mlp_hub.cpp:48-58; model.py:1314-1318). */
int qs_gdn_rollback(const float *states_out, float *state, const uint16_t *conv_states_out, uint16_t *conv_state,
                    const int *accept_len, int *seq_lens, const int *base_lens, int B, int T, int NV, int DK,
                    int DV, int C, int K, void *stream);

/* The same rollback for L GDN layers in one launch (the hub switches every layer's slot at once,
 * kernels/mlp_hub.cpp:48-58): layer l's tensors start l * <its layer stride> elements past the given
 * pointers (states_out [L][T, B, NV, DK, DV], state [L][B, NV, DK, DV], conv_states_out [L][T, B, C, K-1],
 * conv_state [L][B, C, K-1]); seq_lens, when non-null, is set once. */
int qs_gdn_rollback_layers(const float *states_out, size_t states_out_layer_stride, float *state,
                           size_t state_layer_stride, const uint16_t *conv_states_out,
                           size_t conv_states_out_layer_stride, uint16_t *conv_state, size_t conv_state_layer_stride,
                           const int *accept_len, int *seq_lens, const int *base_lens, int L, int B, int T, int NV,
                           int DK, int DV, int C, int K, void *stream);

/* ---------------------------------------------------------------------------------------- a5: paged append
 * Write T new K and V rows per user at positions positions[b] + t into the paged pools (bit-exact).
 *   k, v [B, T, NKV, HD] bf16; pools [num_blocks, NKV, block, HD]; block_table [B, max_blocks]; positions [B].
 * A negative position marks an idle slot (nothing written); a row past the table (QS_STATUS_LENGTH) or on
 * an entry outside the pool (QS_STATUS_PAGE) is skipped and reported.
 * Replaces the tail-core append (kernels/attn_compute_common.hpp:281-341, kernels/attn_worker_writer.cpp
 * :128-143; torch model.py:245-246) with the vLLM block-table contract (block 64, tt-model.yaml:41). */
int qs_paged_kv_append(const uint16_t *k, const uint16_t *v, uint16_t *k_cache, uint16_t *v_cache,
                       const int *block_table, const int *positions, int B, int T, int NKV, int HD, int block,
                       int max_blocks, int num_blocks, int *status, void *stream);

/* The step's position advance, the first launch of a decode or verify step (ResidentModel.step moves the
 * position by the decoded rows, model.py:1314-1351, :1499-1508): base_out[b] <- lens[b] (nullable; the
 * verify step's acceptance adds the accept length to it) and lens[b] <- lens[b] + T, so lens goes from the
 * rows cached before the step to the rows valid after it, which is the seq_lens the step's attention
 * launches take. A negative length (idle slot) is left as it is. A length that passes max_len (the block
 * table's rows: model.py's max_pos, the max_model_len assert of generator_vllm.py:94) is advanced anyway and
 * reported (QS_STATUS_LENGTH); the attention launches then skip that user. */
int qs_advance_lengths(int *lens, int *base_out, int B, int T, int max_len, int *status, void *stream);

/* ---------------------------------------------------------------------------------------- a9: paged fill
 * paged_fill_cache for one sequence: token i of k, v [NKV, T, HD] goes to page page_table[(start+i)/block],
 * row (start+i) % block. Either of k/k_cache or v/v_cache may be null.
 * Replaces ttnn.experimental.paged_fill_cache (prefill/pp_prefill.py:826-827). */
int qs_paged_kv_fill(const uint16_t *k, const uint16_t *v, uint16_t *k_cache, uint16_t *v_cache,
                     const int *page_table, int T, int start, int NKV, int HD, int block, int table_len,
                     int num_blocks, void *stream);

/* The inverse of qs_paged_kv_fill: positions start .. start+T-1 of one sequence, read from its pages into
 * contiguous k, v [NKV, T, HD] (either pair may be null). A position whose table entry is outside
 * [0, num_blocks) reads zeros. With qs_paged_kv_fill it converts between the paged pools and the
 * per-sequence row layout in both directions, bit-exact.
 * Replaces the KV part of the prefill-to-decode export (prefill/pp_prefill.py:1241-1249, the paged-to-rows
 * page copies of prefill/kernels/handoff.cpp:4-8). */
int qs_paged_kv_gather(const uint16_t *k_cache, const uint16_t *v_cache, const int *page_table, uint16_t *k,
                       uint16_t *v, int T, int start, int NKV, int HD, int block, int table_len, int num_blocks,
                       void *stream);

/* ---------------------------------------------------------------------------------------- a6: attention
 * Paged GQA decode attention with split-K over block-table pages and an ordered merge.
 *   q [B, T, NQ, HD] bf16; seq_lens [B] = positions valid after this step's T tokens; query t of user b
 *   attends positions 0 .. seq_lens[b] - T + t (causal among the T new rows); o [B, T, NQ, HD] bf16.
 *   When k_new/v_new [B, T, NKV, HD] are non-null the T new rows are also appended (a5 fused): the
 *   workgroup owning a new row's page writes it first and waits for the store, then reads it back with the
 *   page, so no call sees a half-written row.
 *   pages_per_split (1..64): pages one workgroup walks (the split-K grain); the workspace holds the partials.
 *   A user with seq_lens[b] < T is an idle slot: nothing is appended or attended and its output rows are
 *   zero. A user with seq_lens[b] > max_blocks * block is treated the same and reported (QS_STATUS_LENGTH);
 *   a page entry outside [0, num_blocks) is not attended and is reported (QS_STATUS_PAGE).
 * Replaces the attention leader / chunk workers / tail core (kernels/attn_worker_compute.cpp:77-270,
 * kernels/attn_leader_compute.cpp:42-105, kernels/attn_leader_writer.cpp:86-106, split schedule
 * kernels/attn_common.hpp:139-154; torch model.py:239-246). HD == 256, block == 64, NQ / NKV <= 8. */
size_t qs_paged_attention_workspace_bytes(int B, int T, int NQ, int NKV, int HD, int max_blocks,
                                          int pages_per_split);
int qs_paged_gqa_decode(const uint16_t *q, const uint16_t *k_new, const uint16_t *v_new, uint16_t *k_cache,
                        uint16_t *v_cache, const int *block_table, const int *seq_lens, uint16_t *o,
                        void *workspace, int B, int T, int NQ, int NKV, int HD, int block, int max_blocks,
                        int num_blocks, int pages_per_split, float scale, int *status, void *stream);

/* The attention mixer of one decode / verify step around a5 + a6 (the path's edges, torch model.py:237-246):
 *   qn = rope(rmsnorm(q) * wq), kn = bf16(rope(rmsnorm(k_new) * wk)) appended with v_new, and
 *   o = bf16(softmax(qn K^T) V * sigmoid(gate)), causal among the T new rows as qs_paged_gqa_decode.
 * rmsnorm(x) = x * rsqrt(mean(x^2) + eps) over the head dim; wq, wk [HD] fp32, 16-byte aligned, with the
 * softmax scale folded into wq as the reference folds 1/sqrt(HD) (model.py:237); rope rotates the first rot
 * dims of each head with halves paired as model.py:135-140, rope_cos / rope_sin [B, T, rot / 2] fp32 holding
 * each token's table (model.py:128-132); rot 0 skips it. q, gate [B, T, NQ, HD] bf16 (raw projection
 * slices), k_new, v_new [B, T, NKV, HD] bf16. Replaces the q/k norm + rope of the attention cores
 * (kernels/attn_compute_common.hpp:153-279) and the gate of kernels/attn_leader_compute.cpp:22-79. */
int qs_attn_mixer_decode(const uint16_t *q, const uint16_t *k_new, const uint16_t *v_new, const uint16_t *gate,
                         const float *wq, const float *wk, const float *rope_cos, const float *rope_sin, int rot,
                         uint16_t *k_cache, uint16_t *v_cache, const int *block_table, const int *seq_lens,
                         uint16_t *o, void *workspace, int B, int T, int NQ, int NKV, int HD, int block,
                         int max_blocks, int num_blocks, int pages_per_split, float eps, int *status, void *stream);

/* ---------------------------------------------------------------------------------------- a8: prefill
 * Chunked gated delta rule over one sequence (WY/UT form, bf16 MFMA, fp32 state carry), L2-norm of q
 * (times scale) and k inside:
 *   q, k [T, NK, DK] bf16; v [T, NV, DV] bf16; g, beta [T, NV] fp32; initial_state [NV, DK, DV] fp32
 *   -> o [T, NV, DV] bf16 (token-major), final_state [NV, DK, DV] fp32 (may alias initial_state).
 * chunk: 32 (the reference prefill's chunk_size, prefill/pp_prefill.py:56, :801) or 64. The chunked form
 * equals the token-by-token recurrence for every chunk size, so both run the kernels' 64-token chunks;
 * any other value is rejected.
 * Replaces ttnn.transformer.chunk_gated_delta_rule as called at prefill/pp_prefill.py:791-807. */
size_t qs_gdn_chunk_prefill_workspace_bytes(int T, int NK, int NV, int DK, int DV, int chunk);
int qs_gdn_chunk_prefill(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *g,
                         const float *beta, const float *initial_state, uint16_t *o, float *final_state,
                         void *workspace, int T, int NK, int NV, int DK, int DV, int chunk, float scale,
                         float eps, void *stream);

/* ---------------------------------------------------------------------------------------- f2: prefill conv
 * Causal depthwise conv1d + SiLU over the T prompt tokens of one sequence, carry in and out: the window of
 * channel c is [carry (3, oldest first; zeros when conv_state_in is null), x[0..T-1]], y is written to
 * the q | k | v planes the channels belong to, and conv_state_out receives the last 3 window inputs (bits
 * unchanged), i.e. the decode conv state of the sequence. Same tap-sum order as qs_conv1d_update, so y
 * equals T successive decode conv steps bit for bit. T = 0 copies the carry (x, q, k, v may then be null).
 *   x [T, ldx] bf16 (conv channels in columns [0, 2 CQ + CV)); conv_state_in, conv_state_out [C, K-1]
 *   (may be the same buffer); taps [C, K] -> q, k [T, CQ], v [T, CV] bf16. K == 4; every buffer 16-byte
 *   aligned; CQ, CV, ldx multiples of 8.
 * Replaces the prefill conv with its carry update (prefill/pp_prefill.py:384-445, prefill/kernels/
 * conv_compute.cpp:1-12) and the conv-history handoff to the decode (prefill/pp_prefill.py:1128-1175,
 * prefill/kernels/hist_scatter.cpp:1-12). */
int qs_conv1d_prefill(const uint16_t *x, int ldx, const uint16_t *conv_state_in, const uint16_t *taps, uint16_t *q,
                      uint16_t *k, uint16_t *v, uint16_t *conv_state_out, int T, int CQ, int CV, int K,
                      void *stream);

/* ------------------------------------------------------------------- f4: weight-streaming projections + MLP
 * Weights in OCP microscaling formats, 32 values along K per E8M0 scale: MXFP4 (fmt 4, E2M1 values; the
 * reference streams gate | up in 4-bit block floating point), MXINT8 (fmt 9, two's-complement int8 values
 * times 2^-6: a sign and 7 magnitude bits under the shared scale, the precision of the reference's 8-bit
 * block floating point bfloat8_b for down and the 8-bit projections, model.py:53-58) and MXFP8 (fmt 8, E4M3
 * values, 3 mantissa bits). A weight W [K, N] (y = h W) is quantized and laid out once, on the device, by
 * qs_mx_quantize into qs_mx_packed_bytes(K, N, fmt) bytes of MFMA fragment order (per 16-column tile and
 * K group of 128 (fmt 4) or 64 (fmt 8, 9) values: 1024 value bytes, lane 16 g + r holding column r's values
 * KG q + 32 s + 8 g .. + 7 of every 32-value step s, then column r's step scales). Scale of a block:
 * 2^(floor(log2 amax) - emax), emax 2 (E2M1), 8 (E4M3) or 0 (INT8), exponent clamped to [-126, 127]; values
 * round to the nearest code, ties to even, saturating at 6 / 448 / +-127. N % 16 == 0; K % 128 (fmt 4) or
 * % 64 (fmt 8, 9) == 0.
 * Replaces the reference's host-side weight quantization and bank layout (common.py:115-116 `quantize`;
 * tests/bench_resident_mlp.py:51-80 `interleaved_bank_layout`). */
size_t qs_mx_packed_bytes(int K, int N, int fmt);
int qs_mx_quantize(const float *w, uint8_t *packed, int K, int N, int fmt, void *stream);

/* y [B, N] fp32 = h [B, K] bf16 times the packed W, for 1 <= B <= 16 activation rows: the M = 1..16
 * projections of the reference's streamers (kernels/streamer_compute.cpp:371-449: rmsnorm'd rows times
 * streamed weight tiles). K is split over workgroups when the rows of one split would not fit in 24 KB of
 * LDS or the grid would be small; the splits' partials meet in a caller workspace of
 * qs_mx_gemv_workspace_bytes (0 when none is needed; zeroed once, like every workspace) and the last split
 * of each 16-column tile sums them in split order, inside the launch. */
size_t qs_mx_gemv_workspace_bytes(int B, int K, int N, int fmt);
int qs_mx_gemv(const uint16_t *h, const uint8_t *w, float *y, void *workspace, int B, int K, int N, int fmt,
               void *stream);

/* The MLP half of a decoder layer for 1 <= B <= 16 rows: h = bf16(x rsqrt(mean(x^2) + eps) gamma) per row,
 * z = bf16(silu(h G) (h U)), x_out = x + z D; gate, up packed MXFP4 [H, I], down packed [I, H] in down_fmt
 * (9: MXINT8, the reference's 8-bit precision; 8: MXFP8);
 * x, x_out [B, H] fp32 (may alias), gamma [H] fp32 or null when the norm weight is already folded into the
 * rows of gate and up (the reference's weights.py:107-112 does so); H % 128 == 0, I % 64 == 0. Two launches for one row
 * with H <= 5120 (the gate | up workgroups normalise the row themselves), three otherwise. The workspace
 * (qs_mlp_decode_workspace_bytes, zeroed once) holds arrival counters, h, z and the K-split partials.
 * Replaces the streamers' MLP phase and its residual (kernels/streamer_compute.cpp:452-464,
 * mlp_hub.cpp:309-364 all-reduce on one device; torch pattern tests/bench_resident_mlp.py:98-105). */
size_t qs_mlp_decode_workspace_bytes(int B, int H, int I);
int qs_mlp_decode(const float *x, const float *gamma, const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                  int down_fmt, float *x_out, void *workspace, int B, int H, int I, float eps, void *stream);

/* ------------------------------------------------------------------- measurement probes (no reference part)
 * The bare access patterns the kernels are measured against (bench.py reports them beside each kernel):
 * qs_probe_read streams `bytes` (a multiple of 16384) with nontemporal loads, a wave per 16 KB chunk;
 * qs_probe_copy reads src and writes dst (which may be src) once each, the stores written through the L2 as
 * the GDN state's are; qs_probe_gather reads the K and V tiles of
 * pages 0 .. npages - 1 of every user's block-table row for every KV head with the paged attention's load
 * schedule (pps pages per workgroup, no compute). The loaded data only feeds a checksum that decides a
 * store into sink (device memory of qs_probe_sink_words(bytes) / qs_probe_gather_sink_words words). */
size_t qs_probe_sink_words(size_t bytes);
int qs_probe_read(const void *src, size_t bytes, uint32_t *sink, void *stream);
int qs_probe_copy(const void *src, void *dst, size_t bytes, void *stream);
size_t qs_probe_gather_sink_words(int B, int NKV, int max_blocks, int pps);
int qs_probe_gather(const uint16_t *k_cache, const uint16_t *v_cache, const int *block_table, int B, int NKV,
                    int max_blocks, int npages, int num_blocks, int pps, uint32_t *sink, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* QWEN_STATE_H */
