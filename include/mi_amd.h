/*
 * mi_amd.h -- C ABI of the MI355X (gfx950) ragged paged-attention library.
 *
 * Every entry point is `extern "C"`, takes raw device pointers, element
 * strides and sizes, and a HIP stream passed as `void*` (a hipStream_t; NULL
 * is the legacy default stream).  Calls are asynchronous on that stream: no
 * entry point synchronises the device, reads device memory on the host or
 * allocates memory.  Entry points return MI_OK (0) or a negative MI_ERR_*
 * code; mi_last_error() then returns a message for the calling thread.
 *
 * KV-pool layout ("NHD", one pool per layer):
 *   pool[num_pages][2][page_size][num_kv_heads][head_dim] bf16, contiguous,
 *   K at index 0 and V at index 1 of the second axis
 *   (reference: scheduler.py:168-202, PagedKVCache.kv_data).
 *
 * Page table in CSR form, int32 device arrays
 *   (reference: scheduler.py:267-302, build_csr_metadata):
 *   kv_indptr[batch+1], kv_indices[kv_indptr[batch]], kv_last_page_len[batch];
 *   request b owns pages kv_indices[kv_indptr[b] .. kv_indptr[b+1]) and holds
 *   kv_len_b = (npages_b - 1) * page_size + kv_last_page_len[b] tokens
 *   (0 when npages_b == 0).
 */
#ifndef MI_AMD_H_
#define MI_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mi_stream_t; /* a hipStream_t */

#define MI_OK 0
#define MI_ERR_INVALID (-1)     /* bad argument: shape, size, alignment, range  */
#define MI_ERR_UNSUPPORTED (-2) /* head_dim / group size / page size not built  */
#define MI_ERR_WORKSPACE (-3)   /* caller-supplied workspace too small          */
#define MI_ERR_LAUNCH (-4)      /* HIP runtime reported an error on launch      */

/* Message for the last failing call on this thread ("" if none). */
const char* mi_last_error(void);

/* Library ABI version (major * 10000 + minor * 100 + patch). */
int mi_version(void);

/* ------------------------------------------------------------------------ *
 * Paged KV append.
 * Replaces flashinfer.page.append_paged_kv_cache as called at
 * model.py:207-216 (positional: append_key, append_value, batch_indices,
 * positions, paged_kv_cache, kv_indices, kv_indptr, kv_last_page_len).
 *
 * For token i: b = batch_indices[i], p = positions[i]; K row i (all heads) is
 * written to pool[kv_indices[kv_indptr[b] + p / page_size]][0][p % page_size]
 * and the V row to [..][1][..].  A token whose page slot lies outside request
 * b's page list (kv_indptr[b] + p/page_size >= kv_indptr[b+1]), or whose page
 * id is outside [0, num_pages), is not written.
 * key/value: [num_tokens][num_kv_heads][head_dim] bf16 with the given element
 * strides (head_dim contiguous; rows 16-byte aligned).
 * ------------------------------------------------------------------------ */
int mi_paged_kv_append(const void* append_key, int64_t key_stride_token, int64_t key_stride_head,
                       const void* append_value, int64_t value_stride_token,
                       int64_t value_stride_head, const int32_t* batch_indices,
                       const int32_t* positions, int64_t num_tokens, void* paged_kv_cache,
                       int64_t num_pages, const int32_t* kv_indices, const int32_t* kv_indptr,
                       const int32_t* kv_last_page_len, int32_t batch_size, int32_t num_kv_heads,
                       int32_t head_dim, int32_t page_size, mi_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Fused rotate-half RoPE + paged KV append.
 * Replaces, per layer, apply_rotary_emb on q and k (model.py:92-107, called
 * at model.py:169-170) followed by the append of model.py:203-216.
 *
 * qkv: [num_tokens] rows of bf16, row stride qkv_stride_token elements; each
 * row holds num_qo_heads q heads, then num_kv_heads k heads, then
 * num_kv_heads v heads, head_dim contiguous each.  Token i is rotated with
 * row rope_positions[i] (clamped to [0, table_rows)) of cos_table / sin_table
 * ([table_rows][head_dim] bf16, the rotate-half layout of model.py:79-89):
 * out = bf16(bf16(x * cos) + bf16(rotate_half(x) * sin)), bit-identical to
 * the reference's bf16 torch ops.  Rotated q goes to q_out (element strides;
 * it may alias qkv's q columns); rotated k and the v row are appended with
 * the placement rule of mi_paged_kv_append.  head_dim: multiple of 16.
 * ------------------------------------------------------------------------ */
int mi_rope_append(const void* qkv, int64_t qkv_stride_token, const int32_t* rope_positions,
                   const void* cos_table, const void* sin_table, int64_t table_rows, void* q_out,
                   int64_t q_out_stride_token, int64_t q_out_stride_head,
                   const int32_t* batch_indices, const int32_t* positions, int64_t num_tokens,
                   void* paged_kv_cache, int64_t num_pages, const int32_t* kv_indices,
                   const int32_t* kv_indptr, const int32_t* kv_last_page_len, int32_t batch_size,
                   int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                   mi_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Split-K paged decode attention.
 * Replaces flashinfer.decode.BatchDecodeWithPagedKVCacheWrapper:
 *   plan  -- scheduler.py:402-413, 905-916, 927-938
 *   run   -- model.py:235 (mode == "decode")
 *
 * mi_decode_plan runs a one-workgroup GPU kernel that reads kv_indptr,
 * kv_last_page_len and the first page ids of each split from kv_indices, and
 * writes the split-K work list into `workspace`; it does not touch the host.
 * mi_decode_run reads the work list and kv_indices (which must not change
 * between plan and run), so one plan serves every layer of a step and a
 * graph-captured run replays correctly after any later plan with the same
 * (batch_size, heads, head_dim) shape.
 *
 * q / out: [batch][num_qo_heads][head_dim] bf16 (element strides given).
 * Q head h reads KV head h / (num_qo_heads / num_kv_heads): any integer group
 * size 1..8 runs natively (no head padding).  sm_scale <= 0 selects
 * 1/sqrt(head_dim).  head_dim in {64, 128, 256}; page_size == 16.
 * max_units <= 0 lets plan and run size the work list from workspace_bytes
 * (both must then see the same workspace_bytes); mi_decode_workspace_size
 * with max_units <= 0 returns a size suited to 8 units per compute unit.
 * ------------------------------------------------------------------------ */
size_t mi_decode_workspace_size(int32_t batch_size, int32_t num_qo_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t max_units);

int mi_decode_plan(void* workspace, size_t workspace_bytes, const int32_t* kv_indptr,
                   const int32_t* kv_indices, const int32_t* kv_last_page_len, int32_t batch_size,
                   int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                   int32_t max_units, mi_stream_t stream);

int mi_decode_run(void* workspace, size_t workspace_bytes, const void* q, int64_t q_stride_batch,
                  int64_t q_stride_head, const void* paged_kv_cache, int64_t num_pages,
                  const int32_t* kv_indices, void* out, int64_t out_stride_batch,
                  int64_t out_stride_head, int32_t batch_size, int32_t num_qo_heads,
                  int32_t num_kv_heads, int32_t head_dim, int32_t page_size, float sm_scale,
                  int32_t max_units, mi_stream_t stream);

/* Decode attention with the step's RoPE and K/V append in the same launch:
 * the three per-layer calls of the reference's decode step -- apply_rotary_emb
 * on q and k (model.py:92-107, called at 169-170), append_paged_kv_cache
 * (model.py:203-216) and the decode wrapper's run (model.py:235) -- for a
 * batch that appends exactly one token per request at its last position
 * (kv_len - 1, the decode step: scheduler.py:862-879), after mi_decode_plan
 * of the CSR that already counts that token.  qkv: [batch] rows of bf16, row
 * stride qkv_stride_token elements, each row num_qo_heads q heads, then
 * num_kv_heads k heads, then num_kv_heads v heads (head_dim contiguous each).
 * Request b's q heads and its k heads are rotated with row kv_len_b - 1 --
 * the decode position, which the reference's RoPE takes from position_ids
 * (model.py:399-400) -- clamped to [0, table_rows), of cos_table / sin_table,
 * with the bf16 arithmetic of mi_rope_append; rotated k and v are written to
 * the slot (last_page_len[b] - 1) of the request's last page, and the
 * attention output goes to out as mi_decode_run writes it.  Pool contents and
 * output are bit-identical to mi_rope_append (with batch_indices = b,
 * positions = rope positions = kv_len - 1) followed by mi_decode_run on the
 * rotated q; q is not written back.  Same shapes, workspace and plan rules as
 * mi_decode_run. */
int mi_decode_rope_append_run(void* workspace, size_t workspace_bytes, const void* qkv,
                              int64_t qkv_stride_token, const void* cos_table, const void* sin_table,
                              int64_t table_rows,
                              void* paged_kv_cache, int64_t num_pages, const int32_t* kv_indices,
                              void* out, int64_t out_stride_batch, int64_t out_stride_head,
                              int32_t batch_size, int32_t num_qo_heads, int32_t num_kv_heads,
                              int32_t head_dim, int32_t page_size, float sm_scale, int32_t max_units,
                              mi_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Decode attention with no caller workspace.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under graph capture that may not call hipMalloc, allocation-
 * free serving loops).  It runs the plan and the run of mi_decode_plan /
 * mi_decode_run (same kernels, same results) with the work list in a static
 * device array of mi_decode_static_capacity() bytes (16 MiB; each GPU the
 * library runs on holds one until the process ends) instead of a workspace.
 * Arguments mean what they mean for mi_decode_plan + mi_decode_run.  A batch
 * whose work list does not fit the array (batch x num_kv_heads beyond a few
 * thousand units at head_dim 128) returns MI_ERR_WORKSPACE.  It allocates
 * nothing and never frees.  All calls on one device share that device's
 * array: calls that overlap on one device (several streams or threads)
 * race, and must be ordered by the caller.  The first call on a device looks
 * up the array's device address (not under graph capture).
 * ------------------------------------------------------------------------ */
size_t mi_decode_static_capacity(void);

int mi_decode_static(const void* q, int64_t q_stride_batch, int64_t q_stride_head,
                     const void* paged_kv_cache, int64_t num_pages, const int32_t* kv_indptr,
                     const int32_t* kv_indices, const int32_t* kv_last_page_len, void* out,
                     int64_t out_stride_batch, int64_t out_stride_head, int32_t batch_size,
                     int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                     float sm_scale, mi_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Ragged (varlen) paged prefill attention on bf16 MFMA.
 * Replaces flashinfer.prefill.BatchPrefillWithPagedKVCacheWrapper:
 *   plan  -- scheduler.py:704-716 (qo_indptr, paged_kv_indptr,
 *            paged_kv_indices, paged_kv_last_page_len, causal=True)
 *   run   -- model.py:235 (mode == "prefill")
 *
 * q / out: [total_q][num_qo_heads][head_dim] bf16, rows of request b are
 * qo_indptr[b] .. qo_indptr[b+1].  Any non-negative element strides (token,
 * head) that keep rows 16-byte aligned, including head-major views whose head
 * stride exceeds the token stride; the positions one workgroup tile covers
 * must span at most 2^30 elements (else MI_ERR_INVALID).  With causal != 0, query row i of request b
 * attends to KV tokens j <= i + (kv_len_b - qo_len_b) (bottom-right aligned).
 * total_q must be >= qo_indptr[batch_size]; it sizes the launch on the host.
 * plan() takes the head counts and head_dim (as FlashInfer's plan does): a
 * workgroup serves all num_qo_heads / num_kv_heads (1..8) Q heads of one KV
 * head, and the query positions per workgroup depend on both.
 * head_dim in {64, 128, 256}; page_size == 16.
 * ------------------------------------------------------------------------ */
size_t mi_prefill_workspace_size(int32_t batch_size, int64_t total_q);

int mi_prefill_plan(void* workspace, size_t workspace_bytes, const int32_t* qo_indptr,
                    const int32_t* kv_indptr, const int32_t* kv_last_page_len, int32_t batch_size,
                    int64_t total_q, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                    int32_t page_size, mi_stream_t stream);

int mi_prefill_run(void* workspace, size_t workspace_bytes, const void* q, int64_t q_stride_token,
                   int64_t q_stride_head, const void* paged_kv_cache, int64_t num_pages,
                   const int32_t* kv_indices, void* out, int64_t out_stride_token,
                   int64_t out_stride_head, int32_t batch_size, int64_t total_q,
                   int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                   int32_t page_size, int32_t causal, float sm_scale, mi_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Fused batched sampler.
 * Replaces sample_batch (scheduler.py:319-343) and sample (310-316).
 *
 * logits: [batch][vocab] bf16 rows (row stride in elements).
 * temperature[b] (float, device) is rounded to bf16 as the reference does
 * (its temperature tensor has the logits dtype).  Rows with temperature <= 0
 * take argmax(logits) (lowest index among equal maxima; NaN ranks highest).
 * Other rows draw from softmax(bf16(logit / temperature)) in fp32, restricted
 * to the top-p nucleus when top_p != NULL and top_p[b] < 1 (the smallest set
 * of highest-probability tokens whose mass reaches top_p; tokens tied with the
 * smallest kept probability are kept).  Draws use Philox4x32-10 keyed by
 * `seed`, with the 64-bit counter *rng_offset (device) advanced once per call
 * on the stream, so graph replays draw fresh numbers.
 * out_tokens: [batch] int64 device.
 * workspace: device buffer of at least mi_sample_workspace_size(batch_size,
 * vocab_size) bytes, zero-filled before its first use (the counters in it
 * are back at zero after every call); one call at a time per workspace.
 * Each row is split over ceil(vocab / 4096) workgroups in two launches.
 * ------------------------------------------------------------------------ */
size_t mi_sample_workspace_size(int32_t batch_size, int32_t vocab_size);

int mi_sample(const void* logits, int64_t logits_row_stride, int32_t batch_size, int32_t vocab_size,
              const float* temperature, const float* top_p, uint64_t seed, uint64_t* rng_offset,
              int64_t* out_tokens, void* workspace, size_t workspace_bytes, mi_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Device page table: FIFO free-page ring + per-slot page lists, and the CSR
 * metadata build for a decode step.
 * Replaces PagedKVCache.allocate_pages / release_pages
 * (scheduler.py:208-221), the admission / growth / retire allocator call
 * order (scheduler.py:624-637, 843-847, 984-1003), build_csr_metadata
 * (scheduler.py:267-302) and the decode metadata + graph padding
 * (scheduler.py:862-901).
 *
 * State lives in one caller-owned int32 device buffer of
 * mi_page_table_state_size() bytes.  Pages 0 .. num_pages-2 start on the free
 * ring in ascending order; page num_pages-1 is the scratch page.
 *
 * mi_page_table_step applies, in this order (the reference's deque order):
 *   1. release: the pages of each slot in release_slots[0..n_release), in
 *      order, are appended to the ring tail and the slot emptied;
 *   2. admit: slot admit_slots[k] receives admit_npages[k] pages popped from
 *      the ring head, k ascending;
 *   3. grow: for each decode row i in order, slot decode_slots[i] receives
 *      pages until it holds ceil((decode_pos[i] + 1) / page_size);
 *   4. CSR: for rows i < n_decode, indptr/indices/last_page_len for
 *      seq_len = decode_pos[i] + 1, batch_indices[i] = i,
 *      positions[i] = decode_pos[i]; rows n_decode .. padded_batch-1 are
 *      graph padding and own exactly the scratch page with last_page_len 1
 *      and position 0, so their appends land in the scratch page.
 * `ops` is a device int32 array laid out as
 *   [n_release][n_admit][n_decode][padded_batch]
 *   release_slots[n_release] admit_slots[n_admit] admit_npages[n_admit]
 *   decode_slots[n_decode] decode_pos[n_decode]
 * Outputs (device int32): indptr[padded_batch+1], indices[capacity],
 * last_page_len[padded_batch], batch_indices[padded_batch],
 * positions[padded_batch].  Released page ids are written, in release order,
 * to released_pages (device int32, may be NULL) for mi_pages_zero.  A pop from
 * an empty ring, a slot overflow or an indices overflow sets the sticky error
 * word read by mi_page_table_error_word (device int32 at the returned offset);
 * the host mirrors free counts and never lets that happen.
 * ------------------------------------------------------------------------ */
size_t mi_page_table_state_size(int32_t num_pages, int32_t max_slots, int32_t max_pages_per_slot);

int mi_page_table_init(void* state, int32_t num_pages, int32_t max_slots,
                       int32_t max_pages_per_slot, mi_stream_t stream);

int mi_page_table_step(void* state, int32_t num_pages, int32_t max_slots,
                       int32_t max_pages_per_slot, const int32_t* ops, int32_t ops_len,
                       int32_t page_size, int32_t* indptr, int32_t* indices,
                       int64_t indices_capacity, int32_t* last_page_len, int32_t* batch_indices,
                       int32_t* positions, int32_t* released_pages, mi_stream_t stream);

/* mi_page_table_step followed, in the same single-workgroup launch, by
 * mi_decode_plan of the batch_size (= padded_batch, <= 1024) rows it laid
 * out, into decode_workspace for num_qo_heads / num_kv_heads / head_dim: the
 * per-step metadata build (scheduler.py:862-901) and the decode wrapper's
 * plan() (scheduler.py:905-916) in one launch, with the plan taking the rows'
 * page counts from on-chip memory.  The decode workspace afterwards holds
 * exactly what mi_decode_plan would have written for the same CSR, so
 * mi_decode_run (with the same indices buffer) follows it as it follows
 * mi_decode_plan.  If the step's ops are malformed, its CSR overflows
 * indices_capacity or padded_batch != batch_size, the plan is empty and its
 * header error word is 2.  The plan's header error (1: items did not fit the
 * workspace, 2: no complete CSR to plan) is also ORed, shifted left by 8,
 * into the state's sticky error word, so a run of steps is checked with one
 * read of that word. */
int mi_page_table_step_decode_plan(void* state, int32_t num_pages, int32_t max_slots,
                                   int32_t max_pages_per_slot, const int32_t* ops, int32_t ops_len,
                                   int32_t page_size, int32_t* indptr, int32_t* indices,
                                   int64_t indices_capacity, int32_t* last_page_len,
                                   int32_t* batch_indices, int32_t* positions, int32_t* released_pages,
                                   int32_t batch_size, void* decode_workspace, size_t decode_workspace_bytes,
                                   int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                   mi_stream_t stream);

/* Byte offset of the sticky error word inside the state buffer.  Bits: 1 a
 * release the slot lists disagree with, 2 an admission from an empty ring,
 * 4 decode growth from an empty ring, 8 a CSR over indices_capacity, 16
 * malformed ops; 256 / 512 the fused decode plan's errors 1 / 2. */
size_t mi_page_table_error_offset(int32_t num_pages, int32_t max_slots,
                                  int32_t max_pages_per_slot);

/* Zero `n_pages` pages (ids in page_ids, device int32) in each of `num_layers`
 * pools laid out back to back with `layer_stride_bytes` between pools; each
 * page is `page_bytes` long.  Reference: release_pages zeroes each page of
 * each layer (scheduler.py:216-221). */
int mi_pages_zero(void* pools, int64_t layer_stride_bytes, int32_t num_layers,
                  int64_t num_pages, int64_t page_bytes, const int32_t* page_ids, int32_t n_pages,
                  mi_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Dense-layer fusions around the attention path.
 *
 * mi_add_rms_norm replaces the residual add of DecoderLayer.forward
 * (model.py:335-343) and the RMSNorm that follows it (model.py:115-122,
 * F.rms_norm): for each of `rows` rows of `hidden` bf16 values,
 *   x' = bf16(x + delta)           (delta may be null: x' = x)
 *   h  = bf16(x' * rsqrt(mean(x'^2) + eps) * weight)   (fp32, one rounding)
 * x' is written to x_out when x_out is not null (x_out may alias x); h is
 * written when h_out is not null.  hidden: multiple of 8, <= 16384; rows and
 * weight 16-byte aligned (element strides multiples of 8).
 *
 * mi_silu_mul replaces silu(gate(x)) * up(x) of the MLP (model.py:301-311)
 * over the fused gate/up projection [rows][2 * intermediate]:
 *   out = bf16(bf16(g / (1 + exp(-g))) * u),  g = row[j], u = row[intermediate + j].
 * ------------------------------------------------------------------------ */
int mi_add_rms_norm(const void* x, int64_t x_stride, const void* delta, int64_t delta_stride,
                    const void* weight, void* x_out, int64_t x_out_stride, void* h_out,
                    int64_t h_stride, int64_t rows, int32_t hidden, float eps, mi_stream_t stream);

int mi_silu_mul(const void* gate_up, int64_t gate_up_stride, void* out, int64_t out_stride,
                int64_t rows, int32_t intermediate, mi_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MI_AMD_H_ */
