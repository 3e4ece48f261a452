/*
 * akv_amd -- C ABI of the MI355X (gfx950) Drop + Reposition hot path.
 *
 * Plain C: raw pointers, sizes and a HIP stream handle (void*, NULL = the
 * default stream).  No entry point allocates device memory, frees it,
 * synchronises the stream or reads device memory back to the host: every
 * compute entry point only validates its host-visible arguments and enqueues
 * kernels on `stream`.  Device buffers must stay alive until the stream has
 * finished with them (the caller's lifetime contract).
 *
 * Return value: 0 on success, AKV_EINVAL for an invalid argument, AKV_EHIP
 * when the HIP runtime rejected a launch, AKV_ERUNTIME for an internal
 * consistency failure the reference reports as RuntimeError.  akv_last_error() returns the
 * message of the last failure on the calling thread.
 *
 * Paths in the citations are relative to the reference repository root.
 */
#ifndef AKV_AMD_H
#define AKV_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AKV_OK 0
#define AKV_EINVAL (-22)
#define AKV_EHIP (-5)
#define AKV_ERUNTIME (-71)

/* Storage dtypes of KV buffers and RoPE tables. */
#define AKV_F32 0
#define AKV_F16 1
#define AKV_BF16 2

/* Integer dtypes of index vectors. */
#define AKV_I32 0
#define AKV_I64 1

/*
 * Bits of the status word akv_compact_rows writes (int32, device memory).
 * Once the call's launches have run: 0 = the outputs are complete and
 * usable; AKV_STATUS_SIZES = fresh_count or an output capacity does not
 * match the batch (lists truncated or partly unwritten); AKV_STATUS_INCOMPLETE
 * = an output was not written (set while the one-launch kernel runs, never
 * left set once its finishing launch has run); AKV_STATUS_REBUILT = the
 * one-launch kernel's tiles could not all meet at its barrier and the
 * finishing launch rebuilt their outputs (informational: the outputs are
 * complete).  Consumers that take a `status` pointer (the gated Reposition,
 * akv_decode_indices, akv_decode_attention*, akv_copy_kv_rows) read the word
 * on the device and, when (*status & AKV_STATUS_UNUSABLE) != 0, write
 * nothing and read no K/V row or table entry through the lists, so the
 * compaction's outputs can be handed on with no host read or sync.
 */
#define AKV_STATUS_SIZES 1
#define AKV_STATUS_INCOMPLETE 2
#define AKV_STATUS_REBUILT 4
#define AKV_STATUS_UNUSABLE (AKV_STATUS_SIZES | AKV_STATUS_INCOMPLETE)

/* Message of the last failed call on this thread ("" if none). */
const char* akv_last_error(void);

/* Library version string. */
const char* akv_version(void);

/*
 * Fused all-layer Reposition: for every token t and layer l of the group,
 * re-rotate the rotary part of K from position pairs[t][0] to pairs[t][1]
 * (fp32, inverse rotation then forward rotation, IEEE division, no FMA
 * contraction, round-to-nearest-even store), copy the non-rotary K tail and
 * all of V, from slot src[t] to slot dst[t].  k_ptrs/v_ptrs are DEVICE
 * arrays of n_layers base addresses of [slots, heads, head_dim] buffers
 * that share the given element strides.
 *
 * Replaces reposition_kv_layers / _reposition_layers_kernel,
 * akv/system/sglang/kernels/ops/attention/context_reposition.py:126-236
 * (kernel :28-123).
 */
int akv_reposition_kv_layers(const uint64_t* k_ptrs, const uint64_t* v_ptrs,
                             int32_t n_layers, int32_t kv_dtype,
                             int32_t n_heads, int32_t head_dim,
                             int32_t rotary_dim, int64_t k_stride_slot,
                             int64_t k_stride_head, int64_t v_stride_slot,
                             int64_t v_stride_head, const int32_t* src,
                             const int32_t* dst, const int32_t* pairs,
                             int64_t pair_stride, int64_t n_tokens,
                             const void* cos_sin, int32_t cos_sin_dtype,
                             int64_t rope_stride, int32_t is_neox,
                             int32_t skip_unmapped, void* stream);

/*
 * akv_reposition_kv_layers gated by the status word of the akv_compact_rows
 * call that wrote src / dst / pairs: when status is not NULL and
 * (*status & AKV_STATUS_UNUSABLE) != 0 on the device, no list entry is
 * dereferenced and nothing is written.  The word is read by every
 * workgroup, so the lists go from the compaction to the Reposition on one
 * stream with no host read.  status NULL = akv_reposition_kv_layers.
 * Same kernels and arguments as akv_reposition_kv_layers, whose signature
 * the reference's callers keep.  The gate is what the reference's "no
 * GPU-to-CPU reads and no synchronization" contract needs once the lists
 * are built on the device
 * (akv/system/sglang/kernels/ops/attention/context_reposition.py:148-151).
 */
int akv_reposition_kv_layers_gated(const uint64_t* k_ptrs, const uint64_t* v_ptrs,
                                   int32_t n_layers, int32_t kv_dtype,
                                   int32_t n_heads, int32_t head_dim,
                                   int32_t rotary_dim, int64_t k_stride_slot,
                                   int64_t k_stride_head, int64_t v_stride_slot,
                                   int64_t v_stride_head, const int32_t* src,
                                   const int32_t* dst, const int32_t* pairs,
                                   int64_t pair_stride, int64_t n_tokens,
                                   const void* cos_sin, int32_t cos_sin_dtype,
                                   int64_t rope_stride, int32_t is_neox,
                                   int32_t skip_unmapped, const int32_t* status,
                                   void* stream);

/*
 * Device bytes of the workspace akv_compact_rows needs for a batch of
 * n_requests holding total_tokens raw tokens in all (16-byte aligned).  The
 * workspace must be zero-filled once before its first use (a workspace that
 * was not is not detected); every call leaves it ready for the next,
 * whatever that call's batch size.  Calls that share a workspace must not
 * overlap (issue them on one stream).
 */
int64_t akv_compact_workspace_bytes(int32_t n_requests, int64_t total_tokens);

/*
 * Passes akv_compact_rows makes over the tokens on the current device for a
 * batch of n_requests holding total_tokens raw tokens whose largest list
 * (fresh slots, retired / kept / kv_indices capacity) holds largest_list
 * entries: 1 (one kernel over every tile, the tiles meeting at an in-kernel
 * barrier, then a one-workgroup finishing launch) or 2 (a count launch,
 * then a scatter launch); 0 for an empty batch, AKV_EINVAL for negative
 * sizes.  Either way the call makes two launches.  When tile_tokens is not
 * NULL it receives the tokens per tile of that path (0 for an empty batch).
 * No device work.  No counterpart in the reference: it tells a caller which
 * path to expect.
 */
int akv_compact_launches(int32_t n_requests, int64_t total_tokens,
                         int64_t largest_list, int64_t* tile_tokens);

/*
 * Batched page-table compaction of a single-owner final forward.  For
 * request b, raw tokens [req_offsets[b], req_offsets[b+1]) of the flat
 * keep / birth_positions / final_positions vectors (req_offsets[B] ==
 * total_tokens); its raw row is
 * row_pointers[req_rows[b]] when row_pointers != NULL, else
 * table + req_rows[b] * row_stride.  The birth slots are read from the flat
 * birth_slots vector (same indexing as keep) when it is not NULL, else from
 * the raw row itself (which then holds them on entry).  A kept token is
 * "moved" when its final position differs from its birth position; moved
 * tokens take fresh_slots in request-major raw order.
 * Outputs (flat, request-major, raw order):
 *   raw row (in place)  keep ? (moved ? fresh : birth) : -1
 *   retired             birth slots of dropped or moved tokens
 *   copy_src/copy_dst/copy_pairs   the Reposition inputs (pairs [M,2])
 *   raw_indices/active_positions   decode layout of kept tokens
 *   kv_indices (opt.)   compacted rows, then generated[b] raw-row entries
 *                       after the prompt, laid out by kv_indptr
 *   kv_indptr  (opt.)   [B+1] exclusive scan of kept + generated
 *   last_page_len (opt.) [B] ((kept + generated - 1) % page_size) + 1, 0 if empty
 *   counts     (opt.)   [B,3] kept, moved, retired
 *   status     (opt.)   device int32, AKV_STATUS_* bits: 0 when the
 *                       outputs are complete; AKV_STATUS_SIZES when
 *                       fresh_count or a capacity does not match the batch;
 *                       AKV_STATUS_REBUILT when the one-pass path's
 *                       finishing launch rebuilt the outputs of tiles that
 *                       stopped waiting at its barrier.  Never read on the
 *                       host here: pass it to the consumers' status
 *                       argument, which then skip their work on the device
 *                       when the outputs are unusable.
 * retired, the copy lists and raw_indices / active_positions may be NULL
 * when retired_capacity, fresh_count and kept_capacity are 0.
 * One pass when the batch has at most 512 requests, fewer than 2^29
 * tokens (and list capacities) and some tile size lets every tile be
 * resident at once: tiles publish tagged counts, groups of 64 tiles are
 * released in order, each by its last arrival after summing the earlier
 * groups' totals, and a one-workgroup finishing launch rebuilds the
 * outputs of any tile whose bounded wait ran out (so the outputs never
 * depend on every tile actually being resident); otherwise two passes:
 * per-tile counts, then per-tile prefixes and every output.
 * Replaces the CPU numpy/H2D path of OccurrenceState.advance +
 * terminal_slots + ReqToTokenPool.write + ContextDecodeLayout.from_layout,
 * akv/system/sglang/srt/context_system/occurrence.py:47-66,632-767 and
 * akv/system/sglang.patch:3161-3164,4230-4235; request_active_slots,
 * akv/system/sglang/srt/disaggregation/context_transfer.py:110-128.
 */
int akv_compact_rows(int32_t n_requests, const int64_t* req_offsets,
                     int64_t total_tokens, int32_t* table, int64_t row_stride,
                     const int64_t* row_pointers, const int64_t* req_rows,
                     const uint8_t* keep, const int32_t* birth_positions,
                     const int32_t* final_positions, const int32_t* birth_slots,
                     const int32_t* fresh_slots,
                     int64_t fresh_count, int32_t* retired,
                     int64_t retired_capacity, int32_t* copy_src,
                     int32_t* copy_dst, int32_t* copy_pairs,
                     int32_t* raw_indices, int32_t* active_positions,
                     int64_t kept_capacity, const int32_t* generated,
                     int32_t* kv_indices, int64_t kv_capacity,
                     int32_t* kv_indptr, int32_t* last_page_len,
                     int32_t page_size, int32_t* counts, void* workspace,
                     int64_t workspace_bytes, int32_t* status, void* stream);

/*
 * Page-granular compaction with copy-on-write, page_size P >= 1, for
 * requests whose final positions are 0 .. kept-1 (a closing Reposition).
 * Per request b (raw tokens req_offsets[b] .. req_offsets[b+1]):
 *   p0 = first dropped raw token / P (ceil(n / P) when nothing is dropped);
 *   logical pages < p0 keep their physical pages; every kept token of rank
 *   r >= p0 * P moves to fresh_pages[fresh_b + r / P - p0] * P + r % P with
 *   copy (old slot, new slot, (birth pos, r)); dropped tokens get -1;
 *   released_pages lists old pages of logical index >= p0 (raw order);
 *   page_table lists the new pages of the request, ceil(kept / P) of them.
 * bases int64 [6, B+1], host-computed from the layout:
 *   row 0: p0 * P per request; rows 1..5: exclusive offsets of kept
 *   tokens, copies, fresh pages, page-table entries and released pages.
 * One launch, one thread per raw token; every write is bounded by bases.
 * Every list pointer must be non-null, also for a list whose total in bases
 * is 0 (a batch with nothing copied or released): nothing is written
 * through it then, so any valid device word will do.
 * No counterpart in the reference, whose Reposition rejects page_size != 1
 * (akv/system/sglang/kernels/ops/attention/context_reposition.py:153-154);
 * its P = 1 case equals akv_compact_rows' row/copy outputs
 * (occurrence.py:632-767).
 */
int akv_compact_pages(int32_t n_requests, const int64_t* req_offsets,
                      int64_t max_tokens, int32_t page_size, int32_t* table,
                      int64_t row_stride, const int64_t* row_pointers,
                      const int64_t* req_rows, const uint8_t* keep,
                      const int32_t* birth_positions,
                      const int32_t* final_positions,
                      const int32_t* birth_slots, const int64_t* bases,
                      const int32_t* fresh_pages, int32_t* copy_src,
                      int32_t* copy_dst, int32_t* copy_pairs,
                      int32_t* released_pages, int32_t* page_table,
                      int32_t* raw_indices, int32_t* active_positions,
                      void* stream);

/*
 * Decode read indices over raw request rows through the registry rows
 * int64 [rows, 6] = (raw_ids_ptr, positions_ptr, prompt_len, active,
 * next_pos, row_ptr):
 *   out[indptr[b] + i] = T(row[raw]), raw = raw_ids[start+i] if start+i <
 *   active else prompt + start + i - active (raw = start + i when raw_ids_ptr
 *   is 0); T(x) = mapping[x] * multiplier when mapping != NULL.
 * rows/lengths/indptr/output/starts/mapping take AKV_I32 or AKV_I64.
 * status (opt.): the akv_compact_rows status word when the registry's raw
 * ids or the rows come from that call; nothing is read through them or
 * written when (*status & AKV_STATUS_UNUSABLE) != 0.
 * Replaces context_decode_indices,
 * akv/system/sglang/kernels/ops/attention/context_page_table.py:34-76.
 */
int akv_decode_indices(const int64_t* registry, const int32_t* table,
                       int64_t row_stride, const void* rows, int32_t rows_dtype,
                       const void* lengths, int32_t lengths_dtype,
                       const void* indptr, int32_t indptr_dtype, void* output,
                       int32_t output_dtype, const void* starts,
                       int32_t starts_dtype, const void* mapping,
                       int32_t mapping_dtype, int64_t multiplier,
                       int32_t n_requests, const int32_t* status, void* stream);

/*
 * Sliding-window visible key counts (inclusive q_pos - k_pos <= window),
 * by binary search over the compacted positions of each registry row;
 * min(length, window) for ordinary rows.  When starts != NULL it also
 * writes starts[b] = lengths[b] - output[b] (same dtype as lengths).
 * Replaces context_window_lengths,
 * akv/system/sglang/kernels/ops/attention/context_page_table.py:7-31
 * (and the starts of context_backend.py:792,807).
 */
int akv_window_lengths(const int64_t* registry, const void* rows,
                       int32_t rows_dtype, const void* lengths,
                       int32_t lengths_dtype, void* output,
                       int32_t output_dtype, void* starts, int64_t window,
                       int32_t n_requests, void* stream);

/*
 * indptr[0] = 0, indptr[b+1] = sum(lengths[0..b]); when last_page_len !=
 * NULL also last_page_len[b] = ((lengths[b] - 1) % page_size) + 1 (0 for
 * an empty request).  indptr_scale != 1 instead writes the page-table form
 * indptr[b] = b * indptr_scale (lengths unused).
 * Replaces kv_indptr[1:] = cumsum(seq_lens), akv/system/sglang.patch:2266-2268,
 * and the fill_table indptr, context_backend.py:793.
 */
int akv_build_indptr(const void* lengths, int32_t lengths_dtype,
                     int32_t n_requests, void* indptr, int32_t indptr_dtype,
                     int32_t* last_page_len, int32_t page_size,
                     int64_t indptr_scale, void* stream);

/*
 * Side-row scatter: ((int32_t*)pointers[rows[i]])[columns[i]] = values[i].
 * Replaces write_row_slots, akv/system/sglang/kernels/ops/memory/context_rows.py:7-15.
 */
int akv_write_row_slots(const int64_t* pointers, const void* rows,
                        int32_t rows_dtype, const void* columns,
                        int32_t columns_dtype, const void* values,
                        int32_t values_dtype, int64_t n, void* stream);

/*
 * Extend write of request rows.  For request b (table row r =
 * req_rows[b]; its row is row_pointers[r] when row_pointers != NULL, else
 * table + r * row_stride):
 *   row[0, pre_lens[b])             = prefix_b[0, pre_lens[b]),
 *   row[pre_lens[b], seq_lens[b])   = out_cache_loc[s_b, s_b + seq - pre),
 * prefix_b the device array at address prefix_ptrs[b] (prefix_dtype), s_b
 * the sum of extend_lens[0, b).  Values are stored as int32.
 * Replaces write_req_to_token_pool_triton with RowPointers,
 * akv/system/sglang.patch:238-278 (called from write_cache_indices,
 * sglang.patch:4066-4090).
 */
int akv_write_extend_rows(int32_t* table, int64_t row_stride,
                          const int64_t* row_pointers, const void* req_rows,
                          int32_t rows_dtype, const int64_t* prefix_ptrs,
                          int32_t prefix_dtype, const void* pre_lens,
                          const void* seq_lens, const void* extend_lens,
                          int32_t lens_dtype, const void* out_cache_loc,
                          int32_t loc_dtype, int32_t n_requests, void* stream);

/*
 * Device bytes of the split-K scratch of akv_decode_attention.
 */
int64_t akv_decode_attention_workspace_bytes(int32_t n_requests,
                                             int32_t kv_heads, int32_t head_dim,
                                             int64_t max_len);

/*
 * One GQA decode step over compacted page-one indices with per-head sink
 * logits: for request b and q head h (KV head h / (q_heads / kv_heads)),
 *   out[b, h] = sum_j e^{s_j} v_j / (sum_j e^{s_j} + e^{sinks[h]}),
 *   s_j = scale * q[b, h] . k_j, j over kv_indices[kv_indptr[b] ..
 *   kv_indptr[b+1]) (no sink term when sinks == NULL).  bf16 q / K / V,
 * head_dim 64 or 128, at most 16 q heads per KV head; max_len bounds every
 * request's key count (it sizes the split).  out is bf16 or f32.
 * status (opt.): the akv_compact_rows status word when kv_indptr /
 * kv_indices come from that call; no key index is read and nothing is
 * written when (*status & AKV_STATUS_UNUSABLE) != 0.
 * The consumer of the compacted metadata (the reference's sink
 * normalisation o * sigmoid(lse - sink),
 * akv/system/sglang/srt/layers/attention/context_backend.py:254-272, over the
 * decode indices of context_page_table.py:34-76).
 */
int akv_decode_attention(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                         const void* k_buffer, const void* v_buffer,
                         int64_t k_stride_slot, int64_t k_stride_head,
                         int64_t v_stride_slot, int64_t v_stride_head,
                         int32_t n_requests, int32_t q_heads, int32_t kv_heads,
                         int32_t head_dim, const int32_t* kv_indptr,
                         const int32_t* kv_indices, const float* sinks,
                         float scale, void* out, int32_t out_dtype,
                         int64_t out_stride_b, int64_t out_stride_h,
                         int64_t max_len, void* workspace,
                         int64_t workspace_bytes, const int32_t* status,
                         void* stream);

/*
 * akv_decode_attention without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  The split-K
 * partials live in a static device array of
 * akv_decode_attention_noalloc_max_bytes() bytes per GPU (32 MiB), held
 * until the process ends; a call whose partials need more
 * (akv_decode_attention_workspace_bytes) fails with AKV_EINVAL.  Allocates
 * nothing.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (two streams, two host threads) race.
 */
int64_t akv_decode_attention_noalloc_max_bytes(void);
int akv_decode_attention_noalloc(const void* q, int64_t q_stride_b,
                                 int64_t q_stride_h, const void* k_buffer,
                                 const void* v_buffer, int64_t k_stride_slot,
                                 int64_t k_stride_head, int64_t v_stride_slot,
                                 int64_t v_stride_head, int32_t n_requests,
                                 int32_t q_heads, int32_t kv_heads,
                                 int32_t head_dim, const int32_t* kv_indptr,
                                 const int32_t* kv_indices, const float* sinks,
                                 float scale, void* out, int32_t out_dtype,
                                 int64_t out_stride_b, int64_t out_stride_h,
                                 int64_t max_len, const int32_t* status,
                                 void* stream);

/*
 * Prefill context attention over occurrence metadata (MFMA, bf16 in, fp32
 * accumulate).  Segment s: queries q[qo_indptr[s] .. qo_indptr[s+1]) with
 * their own keys k_ext/v_ext (causal by index) after the prefix keys
 * kv_indices[kv_indptr[s] .. kv_indptr[s+1]) of the pool (all visible);
 * with sliding_window >= 0 a key is visible only if q_pos <= k_pos + window,
 * positions from q_positions / kv_positions (both or neither; without them
 * q_pos = prefix_len + i, k_pos = j).  Positions ascend within a segment.
 * sinks (opt.) f32 [q_heads] add e^sink to the softmax denominator.
 * logit_cap > 0 caps every scaled score s to logit_cap * tanh(s / logit_cap)
 * before the softmax (0 = no cap).
 * q [Nq, q_heads, D], k_ext/v_ext [Nq, kv_heads, D], pool [slots, kv_heads, D]
 * bf16 with unit dim stride; out bf16 or f32 like q; D a multiple of 8 up
 * to 128; q_heads a multiple of kv_heads with at most 128 q heads per KV
 * head, q_heads < 32768; scale > 0.  indptrs / indices / positions: AKV_I32
 * or AKV_I64.  max_query_len: host bound on every segment's query count.
 * Replaces the Triton extend attention launched by
 * ContextAttentionMetadata.forward with context positions,
 * akv/system/sglang/srt/layers/attention/context_backend.py:180-251 and
 * akv/system/sglang.patch:106-237 (extend_attention_fwd).
 */
int akv_context_attention(const void* q, int64_t q_stride_t,
                          int64_t q_stride_h, const void* k_ext,
                          const void* v_ext, int64_t k_ext_stride_t,
                          int64_t k_ext_stride_h, int64_t v_ext_stride_t,
                          int64_t v_ext_stride_h, const void* k_buffer,
                          const void* v_buffer, int64_t k_stride_slot,
                          int64_t k_stride_head, int64_t v_stride_slot,
                          int64_t v_stride_head, int32_t n_segments,
                          int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                          const void* qo_indptr, const void* kv_indptr,
                          int32_t indptr_dtype, const void* kv_indices,
                          int32_t indices_dtype, const void* q_positions,
                          const void* kv_positions, int32_t positions_dtype,
                          int32_t sliding_window, const float* sinks,
                          float scale, float logit_cap, void* out,
                          int32_t out_dtype, int64_t out_stride_t,
                          int64_t out_stride_h, int64_t max_query_len,
                          void* stream);

/*
 * Host (CPU) occurrence window of one forward: the (raw token, position)
 * versions its attention reads and the order in which they are first
 * needed.  Inputs are the compiled layout's int32 vectors (birth positions
 * and stages [n], transition offsets [stage_count+1] and raw / old / new
 * [offsets[stage_count]]), visible_until [n] (a token is readable by
 * queries before it) and terminal_positions [n].
 * akv_window_count writes counts[4] = {occurrences, segments, keys,
 * first_final}: occurrences [n, first_final) are versions read by a
 * segment, [first_final, occurrences) the terminal versions materialised
 * after the last stage.  akv_window_compile fills, for those counts:
 * occurrence_raw_tokens / occurrence_positions [occurrences] (ids 0..n-1
 * are the births), terminal_occurrences [n], segment_query_starts / ends
 * [segments], segment_key_offsets [segments+1], segment_key_occurrences
 * [keys].  Same results and messages as compile_occurrence_window,
 * akv/system/sglang/srt/context_system/occurrence.py:112-265.
 */
int akv_window_count(int64_t n, const int32_t* birth_positions,
                     const int32_t* birth_stages,
                     const int32_t* transition_offsets, int64_t stage_count,
                     const int32_t* transition_raw_tokens,
                     const int32_t* transition_old_positions,
                     const int32_t* transition_new_positions,
                     const int32_t* visible_until,
                     const int32_t* terminal_positions, int64_t query_start,
                     int64_t query_end, int64_t* counts);

int akv_window_compile(int64_t n, const int32_t* birth_positions,
                       const int32_t* birth_stages,
                       const int32_t* transition_offsets, int64_t stage_count,
                       const int32_t* transition_raw_tokens,
                       const int32_t* transition_old_positions,
                       const int32_t* transition_new_positions,
                       const int32_t* visible_until,
                       const int32_t* terminal_positions, int64_t query_start,
                       int64_t query_end, const int64_t* counts,
                       int32_t* occurrence_raw_tokens,
                       int32_t* occurrence_positions,
                       int32_t* terminal_occurrences,
                       int32_t* segment_query_starts,
                       int32_t* segment_query_ends,
                       int32_t* segment_key_offsets,
                       int32_t* segment_key_occurrences);

/*
 * The same window in one replay: fills the output arrays up to
 * capacities[3] = {occurrences, segments, keys} (terminal_occurrences [n],
 * segment_key_offsets [segments capacity + 1]) and writes the exact
 * counts[4] as akv_window_count does.  When a count exceeds its capacity
 * the arrays are incomplete and the caller compiles again with those
 * counts.  Occurrences never exceed n + offsets[stage_count] (a token gets
 * a new version only after a transition moved it) and segments never
 * exceed query_end - query_start.  Replaces the count + fill pair for
 * compile_occurrence_window,
 * akv/system/sglang/srt/context_system/occurrence.py:112-265.
 */
int akv_window_compile_bounded(int64_t n, const int32_t* birth_positions,
                               const int32_t* birth_stages,
                               const int32_t* transition_offsets,
                               int64_t stage_count,
                               const int32_t* transition_raw_tokens,
                               const int32_t* transition_old_positions,
                               const int32_t* transition_new_positions,
                               const int32_t* visible_until,
                               const int32_t* terminal_positions,
                               int64_t query_start, int64_t query_end,
                               const int64_t* capacities, int64_t* counts,
                               int32_t* occurrence_raw_tokens,
                               int32_t* occurrence_positions,
                               int32_t* terminal_occurrences,
                               int32_t* segment_query_starts,
                               int32_t* segment_query_ends,
                               int32_t* segment_key_offsets,
                               int32_t* segment_key_occurrences);

/*
 * Device bytes of the scratch buffer akv_bind_occurrences needs.
 */
int64_t akv_bind_workspace_bytes(int32_t n_requests, int64_t max_occurrences);

/*
 * Slot binding of a fresh request's whole-prompt forward (query_start = 0,
 * query_end = n, every slot request-owned) from its occurrence window
 * (akv_window_compile): for request b, occurrences bases[0][b] ..
 * bases[0][b+1] (request-local raw index and position; ids < n are the
 * births), raw tokens bases[1][b] .. bases[1][b+1] (terminal occurrence,
 * keep, birth slot).  A version is required when it is a birth, read by a
 * segment (id < first_final = bases[5][b]) or the terminal version of a
 * kept token; it reuses the birth slot when its position is the birth
 * position, else it takes the next fresh slot (occurrence order) and a copy
 * (birth slot -> fresh slot, (birth position, position)).
 * Outputs: occurrence_slots (-1 for versions nothing needs), copy lists at
 * bases[2][b] .., retired at bases[3][b] .. (birth slots that are not
 * terminal, raw order; then, from bases[4][b], fresh slots that are not
 * terminal, allocation order), and the request row (table row req_rows[b]
 * or row_pointers[req_rows[b]]): kept ? terminal slot : -1.
 * bases int64 [6, B+1] are host-computed; every write is bounded by them.
 * Replaces plan_occurrence_materialization + OccurrenceState.advance +
 * terminal_slots for that forward,
 * akv/system/sglang/srt/context_system/occurrence.py:341-466,632-767.
 */
int akv_bind_occurrences(int32_t n_requests, const int64_t* bases,
                         int64_t max_occurrences,
                         const int32_t* occurrence_raw_tokens,
                         const int32_t* occurrence_positions,
                         const int32_t* terminal_occurrences,
                         const uint8_t* keep, const int32_t* birth_slots,
                         const int32_t* fresh_slots, int32_t* occurrence_slots,
                         int32_t* copy_src, int32_t* copy_dst,
                         int32_t* copy_pairs, int32_t* retired, int32_t* table,
                         int64_t row_stride, const int64_t* row_pointers,
                         const int64_t* req_rows, void* workspace,
                         int64_t workspace_bytes, void* stream);

/*
 * All-layer K and V row copy between two slot spaces: for token t and
 * layer l, the row_bytes-long K row (and V row) at slot src_slots[t] of
 * src_k_ptrs[l] (src_v_ptrs[l]) goes to slot dst_slots[t] of dst_k_ptrs[l]
 * (dst_v_ptrs[l]); a NULL slot vector means slot t (a packed buffer).
 * Pointer tables are DEVICE arrays of n_layers base addresses; strides are
 * bytes between slots; rows, strides and bases are 16-byte aligned.
 * Destinations may be peer-GPU addresses.  status (opt.): the
 * akv_compact_rows status word when a slot vector comes from that call; no
 * row is read or written when (*status & AKV_STATUS_UNUSABLE) != 0.
 * Replaces the compacted final-version transfer's gather/scatter of
 * request_active_slots and the D-side destination fill,
 * akv/system/sglang/srt/disaggregation/context_transfer.py:110-128,201-259
 * (the transport itself is external).
 */
int akv_copy_kv_rows(const uint64_t* src_k_ptrs, const uint64_t* src_v_ptrs,
                     const uint64_t* dst_k_ptrs, const uint64_t* dst_v_ptrs,
                     int32_t n_layers, int64_t row_bytes,
                     int64_t src_k_stride, int64_t src_v_stride,
                     int64_t dst_k_stride, int64_t dst_v_stride,
                     const int32_t* src_slots, const int32_t* dst_slots,
                     int64_t n_tokens, const int32_t* status, void* stream);

/*
 * Host event compiler (CPU, no device work).  Replays Drop and Reposition
 * events over the raw token stream.  Two calls, like the reference's count
 * and fill passes: akv_plan_count returns the number of transitions through
 * *transition_count (status 0), or status 1 with *bad_boundary set when a
 * Reposition has no active token.  akv_plan_compile fills caller-provided
 * host arrays; status 2 with *bad_token when a token id is outside
 * [0, INT32_MAX].  Invalid event metadata returns AKV_EINVAL with the
 * reference's message in akv_last_error().
 * Replaces count_radix_reposition_transitions and
 * compile_radix_reposition_layout,
 * akv/system/sglang/kernels/ops/attention/context_plan.py:80-532.
 */
int akv_plan_count(int64_t token_count, const int32_t* drop_insert_offsets,
                   int64_t drop_count, const int32_t* drop_range_offsets,
                   const int32_t* drop_ranges, int64_t drop_ranges_len,
                   const int32_t* reposition_raw_boundaries,
                   const int32_t* reposition_insert_offsets,
                   int64_t reposition_count, int32_t* transition_counts,
                   int64_t* status);

int akv_plan_compile(const void* token_ids, int32_t token_ids_dtype,
                     int64_t token_count, const int32_t* drop_insert_offsets,
                     int64_t drop_count, const int32_t* drop_range_offsets,
                     const int32_t* drop_ranges, int64_t drop_ranges_len,
                     const int32_t* reposition_raw_boundaries,
                     const int32_t* reposition_insert_offsets,
                     int64_t reposition_count, int32_t* records,
                     uint8_t* virtual_mask, int64_t* key_to_token,
                     int64_t record_capacity, int64_t* token_to_key,
                     int32_t* positions, uint8_t* keep_mask,
                     int32_t* materialized_stage, int32_t* birth_positions,
                     int32_t* birth_stages, int32_t* transition_offsets,
                     int32_t* transition_raw_tokens,
                     int32_t* transition_old_positions,
                     int32_t* transition_new_positions,
                     int64_t transition_capacity,
                     int32_t* effective_reposition_stages,
                     int64_t* drop_event_to_key, uint8_t* effective_repositions,
                     uint8_t* ignored_repositions, int64_t* status);

/*
 * Host (CPU arrays) ownership plan of one prefill forward over the queries
 * [query_start, query_end) of a raw prompt of n tokens: which occurrences
 * of the window need a page (segment keys, this forward's births, published
 * terminal versions), which reuse an owner row (source_rows[o] = r for the
 * canonical version of raw r, n + r for its terminal version, -1 unbound),
 * and the allocated ones in occurrence order with their copy source rows
 * and (old, new) position pairs.  selected_terminal[query_end]: published
 * terminal occurrence per raw token or -1.  Outputs sized by the occurrence
 * count (allocated, copy rows, 2x pairs) and n (cached flags);
 * *allocated_count receives the allocation count.  Replaces
 * plan_occurrence_materialization,
 * akv/system/sglang/srt/context_system/occurrence.py:341-466 (same
 * decisions and ValueError messages).
 */
int akv_plan_ownership(int64_t n, int64_t query_start, int64_t query_end,
                       int64_t exact_prefix_len, int64_t occurrence_count,
                       const int32_t* occurrence_raw_tokens,
                       const int32_t* occurrence_positions,
                       const int32_t* terminal_occurrences, int64_t key_count,
                       const int32_t* key_occurrences,
                       const int32_t* canonical_positions,
                       const uint8_t* canonical_present,
                       const uint8_t* canonical_owned,
                       const uint8_t* terminal_present,
                       const uint8_t* terminal_keep, int64_t* source_rows,
                       int64_t* allocated, int64_t* copy_source_rows,
                       int32_t* copy_position_pairs, int64_t* selected_terminal,
                       uint8_t* read_cached, uint8_t* repositioned_cached,
                       int64_t* allocated_count);

/*
 * Host (CPU arrays) binding of a planned forward: owner rows address the
 * request's slot sequence old[0:old_count] ++ query[0:query_count] ++
 * extra[0:extra_count].  Writes the owner row of every occurrence (0 when
 * unbound), the copy source / destination rows, the successor's owner rows
 * (ascending) with their ownership and SWA flags, its canonical / terminal
 * rows and canonical positions over [0, end), the retired private rows
 * (ascending) and, when track_swa, the fresh copy destinations whose source
 * has no SWA peer.  counts[3] = {successor rows, retired rows, unused-SWA
 * rows}; row outputs have capacity old_count + query_count + extra_count.
 * Replaces the index work of OccurrenceState.advance,
 * akv/system/sglang/srt/context_system/occurrence.py:632-755.
 */
int akv_advance_ownership(
    int64_t n, int64_t start, int64_t end, int64_t old_count,
    int64_t query_count, int64_t extra_count, const uint8_t* owned,
    const int64_t* canonical_rows, const int64_t* terminal_rows,
    const int32_t* canonical_positions, int32_t track_swa,
    const uint8_t* swa_resident, int64_t occurrence_count,
    const int32_t* occurrence_positions, const int32_t* terminal_occurrences,
    const int64_t* source_rows, const int64_t* allocated,
    const int64_t* copy_source_rows, const int64_t* selected_terminal,
    const int32_t* visible_until, int64_t* occurrence_rows,
    int64_t* copy_source_index, int64_t* copy_destination_index,
    int64_t* successor_rows, int64_t* retired_rows, int64_t* unused_swa_rows,
    uint8_t* next_owned, int64_t* next_canonical, int64_t* next_terminal,
    int32_t* next_positions, uint8_t* next_swa, uint8_t* retired_swa,
    int64_t* counts);

/*
 * Batched owner-row -> slot gather (DEVICE arrays).  sources[6 * b ..]:
 * device address and length of up to three slot pieces of request b
 * (AKV_I32 or AKV_I64 slots, all of slot_dtype); segment s covers elements
 * [segment_offsets[s], segment_offsets[s + 1]) and belongs to request
 * segment_requests[s].  Element i = slot of rows[i] in its request's
 * concatenated pieces (n_requests of them), -1 for row -1 or a row / request
 * out of range; elements [0, wide_count) go to
 * out_wide (slot_dtype), the rest to out_narrow (int32).  One launch for a
 * whole batch; replaces the per-request torch.cat and indexing of
 * akv/system/sglang/srt/context_system/occurrence.py:733-767,795-798,856-864
 * and the batch concatenation of akv/system/sglang.patch:3174-3180.
 */
int akv_gather_slots(int32_t slot_dtype, const int64_t* sources,
                     int64_t n_requests, int64_t n_segments,
                     const int64_t* segment_offsets,
                     const int64_t* segment_requests, const int64_t* rows,
                     int64_t total, int64_t wide_count, void* out_wide,
                     int32_t* out_narrow, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AKV_AMD_H */
