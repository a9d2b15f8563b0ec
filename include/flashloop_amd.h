/*
 * flashloop_amd -- C ABI of the MI355X (gfx950) quantized cross-loop KV decode path.
 *
 * Every entry point is a plain C function over device pointers and sizes.  It is
 * asynchronous on the HIP stream passed as `stream` (a hipStream_t, NULL = the null
 * stream), allocates nothing (outputs and workspaces belong to the caller), throws
 * nothing, and returns FL_OK (0) or a negative FL_E* code; fl_last_error() then holds
 * a message for the calling thread.  Argument checks that need no device access
 * happen before any launch, so an error return means nothing was enqueued.
 *
 * The reference boundary these replace is the pybind11 module `flashloop_kivi_gemv`
 * (flashloop/csrc/kivi_outer_gemv_binding.cpp:5-34, declared in
 * flashloop/csrc/kivi_outer_gemv_cuda.h:6-120) plus the Triton packing kernels it
 * relies on (flashloop/kivi_backend.py:162-256) and the torch glue around
 * selection and token-sparse updates (flashloop/engine.py:84-109, 276-333,
 * flashloop/prefill.py:158-237).  Each declaration below cites the function it
 * replaces.
 *
 * Fixed geometry (flashloop/config.py:18-65, 92-134): head_dim 128, 4-bit codes,
 * group 64, multi-head attention (query heads == KV heads), at most 4 loops.
 */
#ifndef FLASHLOOP_AMD_H
#define FLASHLOOP_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FL_OK 0
#define FL_E_INVALID -1 /* bad argument: null pointer, shape, range */
#define FL_E_LAUNCH -2  /* a HIP launch or runtime call failed */
#define FL_E_CAPACITY -3 /* a size exceeds what the kernel or a buffer supports */

#define FL_HEAD_DIM 128
#define FL_GROUP 64
#define FL_MAX_LOOPS 4

/*
 * One layer's packed cross-loop KV cache for a batch of sequences, in HBM.
 *
 * Rows are addressed per (batch, head) pair `bh = b * heads + h`.  Stream s holds
 * loop s+1: s = 0 is the int4 anchor, s >= 1 the int4 residual against the previous
 * loop's reconstruction.  Streams 0 and 1 are dense over the packed prefix; streams 2
 * and 3 store only the rows active in loops 3 and 4, at compact rows given by the
 * rank maps.  Code rows are token-major: byte j of a 64-byte row holds channel 2j in
 * its low nibble and channel 2j+1 in its high nibble (flashloop/packing.py:1-6, 49-54).
 * The K and V rows of one token share one 128-byte line (FL_CODE_STRIDE): key_codes[s]
 * points at byte 0 of row 0 and value_codes[s] at byte 64, consecutive rows are 128
 * bytes apart, so a selected token costs one aligned line per stream.
 *
 *   key_codes[s]   u8  [B*H, row_capacity[s], 64]  row stride FL_CODE_STRIDE
 *   key_meta[s]    f32 [B*H, token_capacity/64, 128, 2]  (scale, min) per channel per
 *                      logical 64-token group (groups of streams 2/3 are logical too)
 *   value_codes[s] u8  [B*H, row_capacity[s], 64]  row stride FL_CODE_STRIDE
 *   value_meta[s]  f32 [B*H, row_capacity[s], 2, 2]      (scale, min) per 64-channel half
 *   value_meta_token f32 [B*H, token_capacity, 2, 4, 2]  the same V (scale, min) again,
 *                      per logical token: [half][stream] in one 64-byte record, so that a
 *                      reader of selected tokens fetches one line for every stream's
 *                      V metadata (entries of streams 2/3 at inactive tokens are unused)
 *   key_meta_half[s] f16 [B*H, token_capacity/64, 128, 2]  key_meta[s] rounded to fp16
 *                      (nearest even, overflow to +-inf, as torch's .to(torch.float16))
 *   value_meta_half[s] f16 [B*H, row_capacity[s], 2, 2]  value_meta[s] rounded likewise
 *                      The readers stream these fp16 copies (half the metadata bytes;
 *                      the reference's CUDA engine keeps all metadata in fp16,
 *                      flashloop/packing.py:46); the fp32 values stay the stored,
 *                      bit-exact codec state.
 *   rank[0], rank[1] i32 [B, token_capacity]  compact row of stream 2 / 3, or -1
 *   tail_key[r], tail_value[r] bf16 [B*H, tail_capacity, 128]  loop r's BF16 tail
 *   packed_tokens, tail_tokens  i32 [B] (device)  per-sequence prefix / tail lengths
 *
 * Metadata is float32 so that the stored scale/min are bit-identical to the reference
 * codec (flashloop_torch/kv_quantization.py:395-414) and the residual chain stays exact.
 */
#define FL_CODE_STRIDE 128 /* bytes between consecutive code rows of a stream */

typedef struct fl_cache_view {
  int32_t batch;
  int32_t heads;
  int32_t token_capacity;  /* multiple of 64 */
  int32_t tail_capacity;
  int32_t row_capacity[4]; /* row_capacity[0] == row_capacity[1] == token_capacity; all >= 1 */
  uint8_t* key_codes[4];
  float* key_meta[4];
  uint8_t* value_codes[4];
  float* value_meta[4];
  int32_t* rank[2];
  uint16_t* tail_key[4];
  uint16_t* tail_value[4];
  const int32_t* packed_tokens;
  const int32_t* tail_tokens;
  int32_t max_packed_tokens; /* host-side upper bound of packed_tokens (grid sizing) */
  int32_t max_tail_tokens;   /* host-side upper bound of tail_tokens */
  float* value_meta_token;   /* per-token V metadata records (written by fl_pack_kv_groups) */
  uint16_t* key_meta_half[4]; /* fp16 copies of key_meta (written by fl_pack_kv_groups) */
  uint16_t* value_meta_half[4]; /* fp16 copies of value_meta (written by fl_pack_kv_groups) */
} fl_cache_view;

/* Message for the last failing call on this thread ("" if none). */
const char* fl_last_error(void);
/* ABI version of this library (bumped on any signature change). */
int32_t fl_abi_version(void);

/*
 * J1 -- quantize and pack 64-token temporal groups through the residual chain.
 *
 * Replaces the Triton packers `_triton_pack_kivi` / `pack_kivi_k_per_channel` /
 * `pack_kivi_v_per_token` (flashloop/kivi_backend.py:162-256, 404-475) as driven by
 * `CrossLoopKVLayerBuilder.from_loop1/add_loop2/finalize` (flashloop/cache.py:342-625)
 * and `_roll_one_group` (flashloop/cache.py:1778-1838), with the arithmetic of
 * `encode_temporal_group` (flashloop_torch/kv_quantization.py:531-650).
 *
 * For each batch b with dst_group0[b] >= 0 and each j < n_groups, the group of 64
 * source rows starting at `src_row_offset + 64*j` of every (b,h) is encoded into
 * logical group `dst_group0[b] + j` of `view` for loops 0..loops-1:
 *   R_0 = fq(L_0);  R_r = R_{r-1} + fq(L_r - R_{r-1}) over the rows active in loop r.
 * Sources: bf16 rows of 128 channels, (b,h) block stride `src_bh_stride` rows.
 * masks[0], masks[1]: u8 [B, mask_stride] activity of loops 3/4 by source row, or NULL
 * for all rows; an active row must have rank >= 0 in the matching rank map.
 * recon_keys/recon_values (optional, per loop, same layout as the sources) receive
 * R_r as bf16.
 */
int32_t fl_pack_kv_groups(const fl_cache_view* view, int32_t loops,
                          const uint16_t* const* src_keys, const uint16_t* const* src_values,
                          int64_t src_bh_stride, int32_t src_row_offset,
                          const uint8_t* const* masks, int64_t mask_stride,
                          const int32_t* dst_group0, int32_t n_groups,
                          uint16_t* const* recon_keys, uint16_t* const* recon_values,
                          void* stream);

/*
 * J2 -- fused dense decode reader: dequantize, rebuild loop `loop`, q.K^T, online
 * softmax, P.V, split over tokens and merged.
 *
 * Replaces `dense_source_attention_cuda` (flashloop/csrc/kivi_outer_gemv_cuda.h:98-120,
 * kernels at flashloop/csrc/kivi_outer_gemv_cuda.cu:722-1013, 1914-2076) as called by
 * `CrossLoopKVLayer.dense_source_attention` (flashloop/cache.py:1644-1756).  Keys:
 * packed prefix (streams 0..loop, streams 2/3 through the rank maps), then loop
 * `loop`'s tail, then the current token.  q, k_cur, v_cur: bf16 [B*H, 128].
 * out: f32 [B*H, 128].  logits (optional): f32, row bh at `logits + bh*logits_stride`,
 * holding scaling*q.k for the packed_tokens[b] + tail_tokens[b] + 1 keys (never written
 * past logits_stride, should the device lengths exceed the view's host maxima).
 * `loop` in 0..3 (the reference kernel supports 0..1; 2..3 serve
 * enable_sparse_decode=False, flashloop/engine.py:422).
 * workspace: fl_decode_attn_dense_workspace() bytes (16-byte aligned, any content) for the
 * per-split partials; calls that share a workspace must be ordered on one stream.
 */
size_t fl_decode_attn_dense_workspace(const fl_cache_view* view);
int32_t fl_decode_attn_dense(const fl_cache_view* view, int32_t loop,
                             const uint16_t* q, const uint16_t* k_cur, const uint16_t* v_cur,
                             float scaling, float* out, float* logits, int64_t logits_stride,
                             void* workspace, size_t workspace_bytes, void* stream);

/*
 * Allocation-free form of fl_decode_attn_dense.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory or pass a workspace (code under HIP
 * graph capture that must not call hipMalloc, tight serving loops, harnesses that
 * forbid allocation).  Same arguments and results as fl_decode_attn_dense (bit for bit:
 * the same kernels and grid), without the workspace: the per-split partials go to a
 * static device array of fl_decode_attn_dense_noalloc_max_bytes() bytes (8 MiB), one
 * per GPU, held until the process ends.  A cache whose partials exceed it (about 7000
 * (batch, head) rows on a 256-CU GPU) is rejected with FL_E_CAPACITY.  It allocates
 * nothing.  Every call on one GPU shares that GPU's array: calls that may overlap on
 * one GPU (two streams, or two threads) race and must be ordered by the caller.
 */
size_t fl_decode_attn_dense_noalloc_max_bytes(void);
int32_t fl_decode_attn_dense_noalloc(const fl_cache_view* view, int32_t loop,
                                     const uint16_t* q, const uint16_t* k_cur, const uint16_t* v_cur,
                                     float scaling, float* out, float* logits, int64_t logits_stride,
                                     void* stream);

/* Loops 1 and 2 of a decode step (streams 0 and 1; loop 2 with logits) in one reader
 * launch plus one merge launch.  Same results as fl_decode_attn_dense(loop 0) followed by
 * fl_decode_attn_dense(loop 1, logits): logits bit-identical, outputs within float
 * rounding of the partial sums (the split points differ).  No counterpart in the
 * reference, whose decode runs every layer of loop 1 before loop 2
 * (flashloop/engine.py:393-394), so only a caller holding both loops' queries at once
 * can use it; one launch pays the persistent grid's end-of-launch imbalance once.
 * logits1 is required.
 * workspace: fl_decode_attn_dense_pair_workspace() bytes (16-byte aligned, any content).
 */
size_t fl_decode_attn_dense_pair_workspace(const fl_cache_view* view);
int32_t fl_decode_attn_dense_pair(const fl_cache_view* view,
                                  const uint16_t* q0, const uint16_t* k_cur0, const uint16_t* v_cur0, float* out0,
                                  const uint16_t* q1, const uint16_t* k_cur1, const uint16_t* v_cur1, float* out1,
                                  float scaling, float* logits1, int64_t logits_stride,
                                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * Measurement hook (no counterpart in the reference; for benchmarks): record a pair of
 * HIP events on the reader kernel's own dispatch (not the merge; hipExtLaunchKernel, so
 * the events carry the kernel's start and end and no marker packet runs beside it) for
 * the next `launches` calls of fl_decode_attn_dense with this `loop` index (-1: any).
 * `launches` = 0 stops recording and frees the events.  Calls made while the stream is
 * being captured into a graph are not recorded.  fl_profile_dense_reader_read waits
 * for the recorded events and returns the summed elapsed time and the number of
 * recorded launches, then clears them.
 */
int32_t fl_profile_dense_reader(int32_t loop, int32_t launches);
int32_t fl_profile_dense_reader_read(float* total_ms, int32_t* launches);

/*
 * J3 -- decode top-k key selection for sparse late-loop decode.
 *
 * Replaces the torch sequence softmax -> topk -> sort -> gather -> `_pad_decode_indices`
 * -> mass -> normalise of `FlashLoopEngine.decode` (flashloop/engine.py:438-498,
 * 84-109) and `select_decode_keys` (flashloop/selection.py:72-88).  Row r holds
 * n_keys[r / heads_per_count] scores at `scores + r*scores_stride` (the dense reader's
 * logits).  It selects k = min(n, max(1, ceil(n*fraction))) keys ranked by their fp32
 * softmax weight, as the reference ranks `softmax(logits, dtype=float32)`, ties (equal
 * fp32 weights, e.g. weights that underflow to 0) to the lower index, and writes them
 * ascending:
 *   indices i32 [rows, capacity] (0-padded), valid u8 [rows, capacity],
 *   mass f32 [rows] = sum of the selected softmax weights,
 *   weights f32 [rows, capacity] = softmax weight / mass (0 where invalid).
 * The weight of score x is RN(e * RN(1/Z)) with e = exp(RN(x - max)) from IEEE fma/mul
 * (within 2 ulp of exp) and Z the sum of e in a fixed order, so it is reproducible
 * bit for bit off the GPU.
 * `capacity` must be >= k for every row (the engine uses (k/64+1)*64).
 * counts (optional) i32 [rows] receives k.
 * nonfinite (optional) i32 [rows] receives the row's number of NaN / +-inf scores;
 * `flashloop/selection.py:78-79` rejects non-finite weights, so a caller that validates
 * checks it.  A row holding a NaN or +inf (or only -inf) has no finite softmax: its
 * keys are ranked by score (-0.0 equal to +0.0, -inf as -FLT_MAX, lower index first)
 * and its mass and weights are NaN, as torch's are.
 */
int32_t fl_decode_topk(const float* scores, int64_t scores_stride, int32_t rows,
                       const int32_t* n_keys, int32_t rows_per_count, double fraction,
                       int32_t capacity, int32_t* indices, uint8_t* valid, float* mass,
                       float* weights, int32_t* counts, int32_t* nonfinite, void* stream);

/*
 * J2 + J3 -- the loop-2 dense read and its key selection in two launches instead of
 * three: fl_decode_attn_dense(view, loop, ..., logits required) followed by
 * fl_decode_topk on the logits rows with n = packed_tokens[b] + tail_tokens[b] + 1 keys
 * for the rows of batch b -- the `dense_source_attention(loop=1, return_logits=True)` +
 * selection sequence of `FlashLoopEngine.decode` (flashloop/engine.py:422-453, 84-109;
 * flashloop/cache.py:1644-1756).  The reader launch is followed by one launch whose
 * first B*H workgroups select the keys of one row each while the others merge the
 * reader's rows (the top-k's one-workgroup-per-row grid leaves them free); results are
 * bit-identical to the two calls.  Rows must fit the register-resident top-k:
 * logits_stride <= 35840 and ceil(logits_stride * fraction) <= 8192, otherwise
 * FL_E_INVALID (use the two calls).  Workspace: fl_decode_attn_dense_workspace() bytes,
 * as for fl_decode_attn_dense.  No counterpart in the reference as one call.
 */
int32_t fl_decode_attn_dense_select(const fl_cache_view* view, int32_t loop,
                                    const uint16_t* q, const uint16_t* k_cur, const uint16_t* v_cur,
                                    float scaling, float* out, float* logits, int64_t logits_stride,
                                    double fraction, int32_t capacity, int32_t* indices, uint8_t* valid,
                                    float* mass, float* weights, int32_t* counts, int32_t* nonfinite,
                                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * J2 (sparse) -- weighted sum of selected V rows of loop `loop`.
 *
 * Replaces `pv_cross_loop_cuda` (flashloop/csrc/kivi_outer_gemv_cuda.h:54-67, kernel
 * flashloop/csrc/kivi_outer_gemv_cuda.cu:296-394) as used by
 * `FlashLoopEngine._selected_value_aggregate` (flashloop/engine.py:346-371):
 *   out[bh] = sum_j valid*weights[bh,j] * V_loop[indices[bh,j]],
 * where index packed_tokens[b]+tail_tokens[b] is the current token (v_cur).
 * indices/valid/weights: [B*H, capacity].  out f32 [B*H, 128].
 * counts (nullable) i32 [B*H]: row r's valid slots all lie below counts[r] (clamped to
 * [0, capacity]; slots at or past it are not read), as fl_decode_topk writes them.  The
 * readers then partition only the slots below each row's count, so a ragged batch's
 * padding costs nothing; null = every row holds `capacity` slots.  The reference passes
 * no counts (its kernels also visit every padding slot); results are identical with or
 * without them whenever the contract holds.
 * workspace: fl_decode_selected_workspace() bytes, with the same contract as
 * fl_decode_attn_dense.  The sparse readers (this call and the two below) address V
 * codes through the K line (the view's value_codes[s] must be key_codes[s] + 64, as
 * laid out above; FL_E_INVALID otherwise), and they take token_capacity and every
 * row_capacity[s] up to 2^24 (32-bit line offsets within a (b,h) row; FL_E_INVALID above).
 */
size_t fl_decode_selected_workspace(const fl_cache_view* view, int32_t capacity);
int32_t fl_decode_selected_pv(const fl_cache_view* view, int32_t loop, const int32_t* indices,
                              const uint8_t* valid, const float* weights, int32_t capacity,
                              const int32_t* counts, const uint16_t* v_cur, float* out,
                              void* workspace, size_t workspace_bytes, void* stream);

/*
 * J2 (sparse) -- cached-mass late-loop attention correction for loops 3/4.
 *
 * Replaces `sparse_attention_delta_cuda` (flashloop/csrc/kivi_outer_gemv_cuda.h:69-96,
 * kernels flashloop/csrc/kivi_outer_gemv_cuda.cu:1015-1331) as called by
 * `CrossLoopKVLayer.cached_mass_sparse_attention_delta` (flashloop/cache.py:1517-1617):
 *   delta = mass * (softmax_S(scaling*q.K_loop[S]) . V_loop[S] - source_output)
 * over the valid selected indices S (the current token handled as in
 * fl_decode_selected_pv, with k_cur/v_cur; counts as there).  source_output f32
 * [B*H,128], mass f32 [B*H], out f32 [B*H,128].
 */
int32_t fl_decode_attn_sparse_delta(const fl_cache_view* view, int32_t loop,
                                    const uint16_t* q, const uint16_t* k_cur,
                                    const uint16_t* v_cur, const int32_t* indices,
                                    const uint8_t* valid, int32_t capacity, const int32_t* counts,
                                    const float* source_output, const float* mass,
                                    float scaling, float* out,
                                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * J2 (sparse, fused) -- fl_decode_attn_sparse_delta that also forms its source_output.
 *
 * Same result as fl_decode_selected_pv(loop=1, source_weights, source_v_cur) followed by
 * fl_decode_attn_sparse_delta(loop, ...), in one pass over the selected rows: the
 * loop-`loop` reader already loads V streams 0 and 1 of every selected row, which is
 * all the loop-2 aggregate needs (flashloop/engine.py:346-371 computes it at loop 2
 * and consumes it at loops 3 and 4, engine.py:511-528).  source_output f32 [B*H,128]
 * receives the aggregate for reuse by the loop-4 call.  loop must be 2 or 3.
 */
int32_t fl_decode_attn_sparse_delta_fused(const fl_cache_view* view, int32_t loop,
                                          const uint16_t* q, const uint16_t* k_cur,
                                          const uint16_t* v_cur, const int32_t* indices,
                                          const uint8_t* valid, const float* source_weights,
                                          const uint16_t* source_v_cur, int32_t capacity,
                                          const int32_t* counts, const float* mass, float scaling, float* source_output,
                                          float* out, void* workspace, size_t workspace_bytes,
                                          void* stream);

/*
 * J4 -- token-sparse update row movement.
 *
 * fl_gather_rows replaces the `index_select` of active rows (flashloop/prefill.py:158,
 * flashloop/engine.py:284-316); fl_scatter_rows replaces `index_copy_`
 * (flashloop/prefill.py:193-194, 237).  A tensor is seen as [outer, rows, row_bytes]
 * with the given strides (bytes):
 *   gather: dst[o, i] = src[o, index[i]]   for i < n_index
 *   scatter: dst[o, index[i]] = src[o, i]  for i < n_index  (indices distinct)
 * row_bytes and all strides must be multiples of 4; indices are bounds-checked on the
 * device (an out-of-range index skips its row and sets *error_flag to 1 if given).
 */
int32_t fl_gather_rows(const void* src, int64_t src_outer_stride, int64_t src_row_stride,
                       int64_t src_rows, void* dst, int64_t dst_outer_stride,
                       int64_t dst_row_stride, int64_t outer, int64_t row_bytes,
                       const int32_t* index, int64_t n_index, int32_t* error_flag,
                       void* stream);
int32_t fl_scatter_rows(const void* src, int64_t src_outer_stride, int64_t src_row_stride,
                        void* dst, int64_t dst_outer_stride, int64_t dst_row_stride,
                        int64_t dst_rows, int64_t outer, int64_t row_bytes,
                        const int32_t* index, int64_t n_index, int32_t* error_flag,
                        void* stream);

/*
 * J4 -- loop-boundary token score and selection.
 *
 * fl_hidden_delta_score replaces `_hidden_delta_score` (flashloop/engine.py:78-81):
 *   score[r] = ||cur[r] - prev[r]|| / max(||cur[r]||, 1e-12) over bf16 rows of `dim`.
 * fl_select_tokens replaces `select_prefill_tokens` (flashloop/selection.py:26-69):
 * per batch row of `tokens` scores, budget = max(1, ceil(tokens*fraction)); among the
 * eligible tokens (eligible u8 [B, tokens] or NULL) minus the forced last token, the
 * top (count - forced) by score (ties: lower index) are selected, and the last token
 * is always selected when force_last != 0.  mask u8 [B, tokens] out; positions
 * (optional) i32 [B, tokens] ascending selected positions; counts (optional) i32 [B].
 * Returns FL_E_INVALID if the forced last token is ineligible (checked on device:
 * *error_flag set to 1 and the row left empty).
 */
int32_t fl_hidden_delta_score(const uint16_t* cur, const uint16_t* prev, int64_t rows,
                              int32_t dim, float* score, void* stream);
int32_t fl_select_tokens(const float* scores, int32_t batch, int32_t tokens, double fraction,
                         const uint8_t* eligible, int32_t force_last, uint8_t* mask,
                         int32_t* positions, int32_t* counts, int32_t* error_flag,
                         void* stream);

/*
 * Decode-step model ops -- the per-layer work around the readers in one decode step
 * (flashloop/engine.py:396-537: q/k/v projections + RoPE, o_proj, the sandwich norms and
 * residual adds, the SwiGLU MLP, lm_head), fused into few launches.
 *
 * fl_gemv_bf16: y[m, n] = sum_k x[m, k] * W[n, k] for m < M (1..8), W bf16 row-major
 * [N, K] (nn.Linear weights, 16-byte aligned), K % 8 == 0, N % 4 == 0, fp32 accumulation,
 * output rounded to bf16 as the Linear's.  x is bf16, or f32 (x_is_f32) rounded to bf16
 * on load (`out.to(bf16)` before o_proj).  epilogue:
 *   0 plain:  outputs[0] bf16 [M, N]
 *   1 f32:    outputs[0] f32 [M, N] = the bf16 value widened (lm_head(...).float())
 *   2 add:    outputs[0] bf16 = bf16(y) + addend (bf16 [M, N], row stride addend_stride)
 *   3 swiglu: weights = {gate, up}; outputs[0] bf16 = bf16(silu(gate·x)) * (up·x)
 *   4 rope:   weights = {q, k, v} (each [N, K]); outputs = {q, k, v} bf16 [M, N]; q and k
 *             get rotate-half RoPE with the bf16 tables rope_cos/rope_sin [M, head_dim]
 *             (apply_rope, flashloop/engine.py:64-75), each binary op rounded to bf16.
 * fl_norm_chain: per row m of [M, d] bf16 tensors (row stride `stride`):
 *   h = x ? r + RMSNorm_a(x) : r;  if w_f: h = RMSNorm_f(h);  h_out = h;  z_out = RMSNorm_b(h)
 * with RMSNorm_w(v) = bf16(w * v * rsqrt(mean(v^2) + eps)) computed in fp32 (the model's
 * RMSNorm module); every optional pointer may be NULL.  d % 8 == 0, d <= 8192, all
 * tensors 16-byte aligned.
 */
int32_t fl_gemv_bf16(const void* x, int32_t x_is_f32, int64_t x_stride, int32_t m, int32_t k,
                     const uint16_t* const* weights, int32_t n, int32_t epilogue,
                     void* const* outputs, int64_t out_stride, const uint16_t* addend,
                     int64_t addend_stride, const uint16_t* rope_cos, const uint16_t* rope_sin,
                     int32_t head_dim, void* stream);
/*
 * fl_append_tail: the decode append of one layer (CrossLoopKVLayer.append_decode_token,
 * flashloop/cache.py:1758-1776, device half): for every sequence b, the step's rows
 * keys[r] / values[r] (bf16 [B*H, 128], r = loop 0..3) are written to tail_key[r] /
 * tail_value[r] at row tail_tokens[b], tail_active[j][b, tail_tokens[b]] = 1 (u8
 * [B, tail_capacity], j = loop 3/4), then tail_tokens[b] += 1 (tail_tokens: the view's
 * length array, passed writable) -- all on the device, so
 * a captured step replays it.  A sequence whose tail is full is left unchanged (the
 * caller rolls a group out first).
 */
int32_t fl_append_tail(const fl_cache_view* view, const uint16_t* const* keys,
                       const uint16_t* const* values, uint8_t* const* tail_active,
                       int32_t* tail_tokens, void* stream);
int32_t fl_norm_chain(int32_t m, int32_t d, float eps, const uint16_t* x, const uint16_t* r,
                      const uint16_t* w_a, const uint16_t* w_f, const uint16_t* w_b,
                      uint16_t* h_out, uint16_t* z_out, int64_t stride, void* stream);
/*
 * fl_gemv_bf16_chain: fl_norm_chain followed by fl_gemv_bf16 in one launch (no reference
 * counterpart: the engine's RMSNorm -> Linear module pairs, flashloop/engine.py:396-537,
 * whose norm otherwise costs a launch of its own).  The GEMV's input rows are z of the
 * chain (h when w_b is NULL), computed by every workgroup with the same arithmetic as
 * fl_norm_chain (bit-identical results); h_out (optional) receives h.  The chain reads r
 * and x (optional) with row stride `stride`; d = k <= 4096.  The GEMV arguments are
 * those of fl_gemv_bf16 (x is the chain output, bf16).
 */
int32_t fl_gemv_bf16_chain(int32_t m, int32_t k, float eps, const uint16_t* x, const uint16_t* r,
                           const uint16_t* w_a, const uint16_t* w_f, const uint16_t* w_b, uint16_t* h_out,
                           int64_t stride, const uint16_t* const* weights, int32_t n, int32_t epilogue,
                           void* const* outputs, int64_t out_stride, const uint16_t* addend,
                           int64_t addend_stride, const uint16_t* rope_cos, const uint16_t* rope_sin,
                           int32_t head_dim, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHLOOP_AMD_H */
