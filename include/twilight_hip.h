/*
 * twilight_hip.h - C ABI of the MI355X (gfx950) sparse-decode KV path.
 *
 * One shared library, libtwilight_hip.so, built by hipcc for gfx950 and loaded
 * with ctypes exactly as the reference loads its natives (raw pointers,
 * int64 sizes, an opaque stream, an int status).  No torch types cross this
 * boundary.  Every entry point:
 *   - returns TW_OK (0) or a nonzero TW_E* status; the Python layer maps
 *     TW_EINVAL / TW_ERANGE to ValueError and the rest to RuntimeError;
 *   - enqueues work on `stream` (a hipStream_t, NULL = legacy default stream)
 *     and never synchronizes it, unless the comment says otherwise;
 *   - takes caller-allocated outputs.  Entry points that need scratch take a
 *     `workspace` pointer whose size is given by the matching *_workspace_size
 *     query; its arrival counters (a fixed 64 KiB region at its start, one
 *     counter per KV group, at most 16384 groups) must be zero before the
 *     first call -- a zeroed buffer -- and the library leaves them zero after
 *     every call and never puts other data there, so a workspace is reusable
 *     by any later call whatever its sizes, but two calls sharing one
 *     workspace must not overlap in time.
 *
 * dtype codes: TW_DTYPE_F16, TW_DTYPE_BF16, TW_DTYPE_F32 (key/value/metadata
 * storage); queries for scoring are always fp32, as in the reference.
 *
 * Reference paths below are relative to source/headinfer/headinfer/ unless
 * they start with scripts/.
 */
#ifndef TWILIGHT_HIP_H
#define TWILIGHT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum tw_status {
  TW_OK = 0,
  TW_EINVAL = 1,      /* bad shape, dtype, pointer or flag */
  TW_ERANGE = 2,      /* an index is outside its source (gather natives) */
  TW_ENOMEM = 3,      /* workspace too small */
  TW_EHIP = 4,        /* HIP runtime error; see tw_last_hip_error() */
  TW_EUNSUPPORTED = 5 /* valid request this library does not implement */
};

enum tw_dtype { TW_DTYPE_F16 = 0, TW_DTYPE_BF16 = 1, TW_DTYPE_F32 = 2 };

/* Human-readable status text; never NULL. */
const char* tw_status_string(int status);
/* The hipError_t recorded by the most recent TW_EHIP return (0 if none). */
int tw_last_hip_error(void);
/* Library version, (major << 16) | minor. */
int tw_version(void);

/* ------------------------------------------------------------------------
 * Prompt metadata, one launch for n_entries KV heads.
 * Replaces QuestTopKOffloadedCache._build_metadata
 * (quest_offload_cache.py:276-289: per-page amin/amax over rows
 * [sink + p*bs, sink + (p+1)*bs), complete pages only) and the Twilight
 * override (twilight_offload_cache.py:925-936) calling affine_int4_pack
 * (twilight_offload_cache.py:25-37).
 *   keys      [n_entries][key_entry_stride] elements, row t of entry e at
 *             keys + e*key_entry_stride + t*D; rows 0..T-1 are read.
 *   page_min/page_max (nullable together) [n_entries][page_entry_stride]
 *             elements, page p at + p*D; pages = T > sink ? (T-sink)/bs : 0.
 *   packed/scale/minimum (nullable together): packed u8 [..][T][D/2] with
 *             quant_entry_stride rows per entry (row t at + t*D/2), scale and
 *             minimum [..][quant_entry_stride] in the key dtype.
 * min/max use the IEEE total order (-0 < +0); a NaN anywhere in the reduced
 * set yields the dtype's canonical NaN.  INT4 codes: low nibble = channel 2j,
 * a NaN code is stored as 0.  D must be even and <= 1024.
 * ---------------------------------------------------------------------- */
int tw_build_page_metadata(const void* keys, int64_t key_entry_stride, int n_entries, int T, int D,
                           int dtype, int sink, int block_size, void* page_min, void* page_max,
                           int64_t page_entry_stride, void* packed, void* scale, void* minimum,
                           int64_t quant_entry_stride, void* stream);

/* Decode-time metadata update, one launch for n_entries KV heads, after row
 * `position` of each entry was written (stream order after the append).
 * Writes the INT4 code, scale and minimum of row `position` and, when the
 * row completes page p = (position - sink) / bs (i.e. position >= sink and
 * (position - sink + 1) % bs == 0), page p's min/max over rows
 * [sink + p*bs, sink + (p+1)*bs).  Layouts as in tw_build_page_metadata;
 * the keys may live in HBM or in mapped pinned host memory.  The outputs
 * equal those of tw_build_page_metadata over position + 1 rows bit for bit.
 * The reference builds page metadata and INT4 keys at prefill only
 * (quest_offload_cache.py:528-537, twilight_offload_cache.py:925-936) and
 * caps the candidate pages at the prompt's (quest_offload_cache.py:342-345);
 * this entry point lets the selection cover pages completed during decode. */
int tw_update_page_metadata(const void* keys, int64_t key_entry_stride, int n_entries, int position, int D,
                            int dtype, int sink, int block_size, void* page_min, void* page_max,
                            int64_t page_entry_stride, void* packed, void* scale, void* minimum,
                            int64_t quant_entry_stride, void* stream);

/* Ragged tw_update_page_metadata: entry e's new row is positions[e] (int32,
 * device).  Rows beyond max_position and pages at or beyond max_pages are
 * skipped (the buffers' capacity), as are negative positions.  Otherwise the
 * same outputs as tw_update_page_metadata entry by entry. */
int tw_update_page_metadata_ragged(const void* keys, int64_t key_entry_stride, int n_entries, const int32_t* positions,
                                   int max_position, int D, int dtype, int sink, int block_size, void* page_min,
                                   void* page_max, int max_pages, int64_t page_entry_stride, void* packed,
                                   void* scale, void* minimum, int64_t quant_entry_stride, void* stream);

/* affine_int4_dequantize (twilight_offload_cache.py:40-47):
 * out[n][d] = f32(code)*f32(scale[n]) + f32(minimum[n]) (mul, then add). */
int tw_int4_dequantize(const void* packed, const void* scale, const void* minimum, int dtype,
                       int64_t N, int D, float* out, void* stream);

/* ------------------------------------------------------------------------
 * fused_quest_score (twilight_fused_quest.py:35-46 / _score :12-32).
 *   q [G][R][D] fp32; page_min/page_max: group g page p at
 *   + g*page_group_stride + p*D; out [G][R][P] fp32.
 * score = sum_d f32(q_d > 0 ? max_d : min_d) * q_d in the reference order:
 * 32 accumulators (d mod 32) filled chunk by chunk, then an adjacent-pair
 * tree; no fused multiply-add.  Bit-exact for D = 128; the same order
 * generalises to any D <= 256.
 * ---------------------------------------------------------------------- */
int tw_quest_score(const float* q, const void* page_min, const void* page_max, int dtype, int G,
                   int R, int P, int D, int64_t page_group_stride, float* out, void* stream);

/* ------------------------------------------------------------------------
 * torch.topk(scores, k, sorted=False).indices.sort()
 * (quest_offload_cache.py:373-374, twilight_offload_cache.py:1153).
 * scores [rows][P] fp32 (row stride score_row_stride) -> out [rows][k] int64
 * ascending page ids.  Ties go to the lowest index, NaN ranks highest, -0
 * equals +0.  1 <= k <= P.
 * Rows of P > 8192 scores first keep the top min(k, n) of every 8192-score
 * segment (an extra launch) and select among those: they need a workspace of
 * tw_topk_sorted_workspace_size(rows, P) bytes (0, and workspace may be
 * NULL, when P <= 8192) and (P / 8192) * k + min(k, P % 8192) <= 8192,
 * else TW_EUNSUPPORTED.
 * ---------------------------------------------------------------------- */
size_t tw_topk_sorted_workspace_size(int rows, int P);
int tw_topk_sorted(const float* scores, int rows, int P, int64_t score_row_stride, int k,
                   int64_t* out, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Quest selection for one decoder layer: score, top-k and the GQA union
 * plan, two launches (score kernel, then one selection block per query
 * head; the last block of each KV group builds the group's plan).  Covers
 * prepare_layer_selection (quest_offload_cache.py:299-401) followed by
 * _selected_positions (:403-511) for the G entries of a layer, and the
 * Twilight stage-1 B0 selection (twilight_offload_cache.py:1128-1166).
 *   q [G][R][D] fp32; metadata as in tw_quest_score; P pages scored.  Above
 *   8192 pages a segment pass (one more launch, as tw_topk_sorted) keeps each
 *   8192-page segment's top k first, so (P / 8192) * k + min(k, P % 8192)
 *   <= 8192 and, with a plan, the union's page bitmap (P / 4 + 8 * min(P, R*k)
 *   bytes) within the 160 KB of LDS, else TW_EUNSUPPORTED.
 *   scores (nullable) [G][R][P] fp32 copy of the scores.
 *   sel_pages (nullable) [G][R][k] int32 ascending page ids per head
 *   (torch.topk(sorted=False) then sort, quest_offload_cache.py:373-374;
 *   ties to the lowest page, NaN highest, -0 == +0).
 *   Union plan (nullable): plan_pages[g*plan_stride + u], u < plan_counts[g],
 *   the ascending pages selected by any of the R heads of group g, and
 *   plan_masks the bitmask of heads that selected each.  plan_stride >=
 *   min(P, R*k).
 *   Row plan (nullable): for group g, rows[g*rows_stride + i] lists token
 *   positions [0,sink_end) ++ (sink + p*bs + [0,bs)) for every union page p
 *   ascending ++ [recent_start, length), then, if append_position >= 0,
 *   append_position itself.  row_masks gets the heads that see each row
 *   (pages: heads that selected them; all other rows: all heads),
 *   row_counts[g] the number of rows.
 *   Window: sink_end = min(sink, length); recent_start = max(sink_end,
 *   length - max(0, recent - 1))  (quest_offload_cache.py:330-332).
 * R <= 8 when a plan is requested.  workspace: tw_quest_select_workspace_size
 * bytes, zero before the first call (the library leaves its counters zero).
 * ---------------------------------------------------------------------- */
size_t tw_quest_select_workspace_size(int G, int R, int P);
int tw_quest_select(const float* q, const void* page_min, const void* page_max, int dtype, int G,
                    int R, int P, int D, int64_t page_group_stride, int k, float* scores,
                    int32_t* sel_pages, int32_t* plan_pages, uint8_t* plan_masks, int32_t* plan_counts,
                    int64_t plan_stride, int32_t* rows, uint8_t* row_masks, int32_t* row_counts,
                    int64_t rows_stride, int sink, int recent, int block_size, int length,
                    int append_position, void* workspace, size_t workspace_bytes, void* stream);

/* tw_quest_select with no workspace argument, for callers that cannot
 * allocate device memory: code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc.  No counterpart in the reference.  The
 * workspace is a static device array of tw_quest_select_static_capacity()
 * bytes (16 MiB) that each GPU holds until the process ends; a call whose
 * tw_quest_select_workspace_size(G, R, P) exceeds it returns TW_ENOMEM.  The
 * first call on a device takes the array's address and enqueues a zero fill
 * (a kernel, capture-safe) ahead of its own kernels; nothing is allocated.
 * Every call on one GPU shares the array: calls that overlap in time on one
 * GPU race (issue them on one stream).  Outputs and validation are those of
 * tw_quest_select. */
size_t tw_quest_select_static_capacity(void);
int tw_quest_select_static(const float* q, const void* page_min, const void* page_max, int dtype, int G, int R,
                           int P, int D, int64_t page_group_stride, int k, float* scores, int32_t* sel_pages,
                           int32_t* plan_pages, uint8_t* plan_masks, int32_t* plan_counts, int64_t plan_stride,
                           int32_t* rows, uint8_t* row_masks, int32_t* row_counts, int64_t rows_stride, int sink,
                           int recent, int block_size, int length, int append_position, void* stream);

/* Ragged groups: tw_quest_select's score, top-k and union plan for G groups
 * of different lengths in one launch pair (e.g. the KV heads of several
 * requests at one layer).  lengths [G] (int32, device) gives each group's
 * tokens L_g; group g scores its candidate pages P_g = min(P_max,
 * (recent_start_g - sink_end_g) / block_size) with the window of
 * tw_quest_select, keeps k_g = min(k, P_g) pages per head (sel_pages slots
 * k_g .. k-1 get -1) and writes the union plan of those.  Nothing depends on
 * a host-side length, so a captured graph replays it as lengths advance.
 * Same orders, ties and workspace (tw_quest_select_workspace_size(G, R,
 * P_max)) as tw_quest_select; no row plan.  The reference is batch-1
 * (slab_cache.py:5, quest_offload_cache.py:520-521); this batches its
 * prepare_layer_selection (quest_offload_cache.py:299-401) over requests. */
int tw_quest_select_ragged(const float* q, const void* page_min, const void* page_max, int dtype, int G, int R,
                           int P_max, int D, int64_t page_group_stride, const int32_t* lengths, int k,
                           int32_t* sel_pages, int32_t* plan_pages, uint8_t* plan_masks, int32_t* plan_counts,
                           int64_t plan_stride, int sink, int recent, int block_size, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Quest selection as per-head page bitmaps, for the fused decode path.  The
 * score and top-k of tw_quest_select (same orders and ties; lengths
 * (nullable, device [G] int32) selects per group as tw_quest_select_ragged
 * does), but instead of a union plan -- built by one block per group after
 * its heads' top-k -- every head's selection is written as a bitmap: bit p
 * of sel_bits[(g*R + r)*bits_stride + p/32] (32-bit words) is set when head
 * r of group g selected page p.  2*ceil(P/64) words per row are written;
 * bits_stride is even and sel_bits 8-byte aligned, so a row reads as 64-bit
 * words.  tw_decode_attention_pages_bits ranks the union from these rows.
 * Replaces prepare_layer_selection's page ids and the GQA union of the
 * decode branches (quest_offload_cache.py:299-401, mp.py:239-279): the set
 * of pages is the same, only the form differs.  P <= 8192 (longer rows:
 * tw_quest_select), k in [1, P].  scores, sel_pages (nullable) as in
 * tw_quest_select (ragged: each group's own pages and k_g slots, the rest
 * -1).  Workspace: tw_quest_select_workspace_size(G, R, P). */
int tw_quest_select_bits(const float* q, const void* page_min, const void* page_max, int dtype, int G, int R,
                         int P, int D, int64_t page_group_stride, const int32_t* lengths, int k, float* scores,
                         int32_t* sel_pages, uint32_t* sel_bits, int64_t bits_stride, int sink, int recent,
                         int block_size, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Twilight stage 2, INT4 QK estimate over the B0 candidates of every head.
 * Replaces fused_affine_int4_qk (twilight_fused_qk.py:12-55) with the
 * 1/sqrt(D) scaling of prepare_layer_selection (twilight_offload_cache.py:
 * 1197-1261).  The candidates of head r of group g are the b0_pages pages it
 * chose in stage 1, ascending, each expanded to block_size positions
 * sink + page*block_size + [0, block_size): candidate n = slot*block_size + i
 * of the head's slot-th page.  They are read from the stage-1 union plan
 * (plan_pages / plan_masks / plan_counts of tw_quest_select, k = b0_pages)
 * so every INT4 row is loaded once for all R heads.
 *   q [G][R][D] fp32 (16-byte aligned); packed[(g*quant_entry_stride + t)*
 *   D/2 + d/2] (low nibble = even channel), scale/minimum [G][
 *   quant_entry_stride] in dtype (tw_build_page_metadata's quantized keys);
 *   quant_rows valid rows per entry (candidates beyond it are skipped).
 *   logits [G][R][b0_pages*block_size] fp32, the estimate of qk_scale * (q .
 *   k~) with k~_d = code_d*scale + min, defined exactly: Q_d = rint(q_d *
 *   2^(22-E)) with E the frexp exponent of max |q|, S = sum_d code_d * Q_d
 *   (exact integer), logit = qk_scale * ((scale * ldexp(S, E-22)) + (min *
 *   ldexp(sum_d Q_d, E-22))) in fp32 (a non-finite q gives NaN).  D = 4 ..
 *   256, a power of two; R <= 8.
 *   slot_u / page_rows (both or neither): for tw_twilight_select_pages,
 *   slot_u [G][R][b0_pages] int32 gets the union index of each head's B0
 *   slot and page_rows[g*plan_stride + u] is cleared for every union page.
 * ---------------------------------------------------------------------- */
int tw_twilight_qk(const float* q, int G, int R, int D, const uint8_t* packed, const void* scale,
                   const void* minimum, int dtype, int64_t quant_entry_stride, int64_t quant_rows,
                   const int32_t* plan_pages,
                   const uint8_t* plan_masks, const int32_t* plan_counts, int64_t plan_stride, int b0_pages,
                   int sink, int block_size, float qk_scale, float* logits, int32_t* slot_u, uint32_t* page_rows,
                   void* stream);

/* INT4 QK at explicit positions: the fused_affine_int4_qk call surface
 * (twilight_fused_qk.py:34-55).  q [G][R][D] fp32; positions [G][R][N] int64
 * rows of entry g's INT4 keys (layout as in tw_twilight_qk; rows outside
 * [0, quant_rows) give no output).  materialize = 0: out [G][R][N] =
 * qk_scale * (q . k~) in tw_twilight_qk's order (qk_scale 1 reproduces the
 * raw dot); materialize != 0: out [G][R][N][D] = k~.
 * D = 4 .. 256, a power of two. */
int tw_int4_qk_positions(const float* q, int G, int R, int D, const uint8_t* packed, const void* scale,
                         const void* minimum, int dtype, int64_t quant_entry_stride, int64_t quant_rows,
                         const int64_t* positions, int N, float qk_scale, int materialize, float* out,
                         void* stream);

/* ------------------------------------------------------------------------
 * Twilight stage 2, top-p budgets, token selection and the GQA union.
 * Replaces the top-p of ExactTopPGraph (twilight_exact_top_p_graph.py:19-32;
 * inline twilight_offload_cache.py:1274-1310), matched_budget_counts
 * (twilight_offload_cache.py:50-86, per group, every head's capacity N) and
 * the GPU GQA union (twilight_offload_cache.py:1517-1614).
 *   logits [G][R][N] from tw_twilight_qk, N = b0_pages*block_size <=
 *   tw_twilight_max_candidates() (16384);
 *   sel_pages [G][R][b0_pages] the stage-1 pages (ascending) that map
 *   candidate n of head r to position sink + sel_pages[n/bs]*bs + n%bs.
 *   desired (nullable) [G][R]: the exact top-p count -- masses E_n =
 *   floor(exp(l_n - max l) * 2^40) with a fixed fp32 exp polynomial, Z = sum
 *   E_n, and the smallest c whose c largest logits (ties to the lower n)
 *   carry at least ceil(round(top_p*2^24) * Z / 2^24).
 *   budget_mode 0 (dynamic): each head keeps its desired candidates.
 *   budget_mode 1 (matched): allocated = matched_budget_counts(desired,
 *   target_total) per group, and each head keeps its top-allocated
 *   candidates (ties to the lower n).  R <= target_total <= R*N.
 *   budget_mode 2 (given): allocated [G][R] is an input (counts clamped to
 *   [1, N]); each head keeps its top-allocated candidates, desired is not
 *   computed.  For callers that allocate one budget across more heads than
 *   one call takes (R > 8 split into sub-groups).
 *   allocated (nullable) [G][R] the kept counts.
 *   head_bits (nullable) [G][R][ceil(N/32)]: bit n of head r's row is set
 *   when the head keeps candidate n (its own selection before the union).
 *   rows[g*rows_stride + i] gets group g's ascending union of [0, sink_end),
 *   the kept positions of its R heads and [recent_start, length), then
 *   append_position if >= 0; row_counts[g] the count.  rows_stride >=
 *   length + 1.  workspace: tw_twilight_select_workspace_size bytes, zero
 *   before the first call (the library leaves its counters zero).
 * ---------------------------------------------------------------------- */
size_t tw_twilight_select_workspace_size(int G, int R, int N);
/* Largest candidate count per head (N = b0_pages * block_size) the Twilight
 * selection entry points take (16384: a 512-thread block, 32 candidates per
 * thread); beyond it they return TW_EUNSUPPORTED.  The reference has no such
 * limit (twilight_offload_cache.py:183-381 checks only that the budget is
 * positive); TwilightOffloadCache refuses, at construction, a budget the
 * longest cache would take past it. */
int tw_twilight_max_candidates(void);
int tw_twilight_select(const float* logits, int G, int R, int N, const int32_t* sel_pages, int b0_pages,
                       float top_p, int budget_mode, int target_total, int32_t* desired, int32_t* allocated,
                       uint32_t* head_bits, int32_t* rows, int32_t* row_counts, int64_t rows_stride, int sink,
                       int recent, int block_size, int length, int append_position, void* workspace,
                       size_t workspace_bytes, void* stream);
/* tw_twilight_select (dynamic budgets, no decode row in the union) over
 * groups of different lengths: group g has lengths[g] tokens (int32,
 * device; <= max_length, rows_stride > max_length), ragged_pages =
 * min(whole pages between sink and recent, page_capacity) candidate pages,
 * and min(that, b0_pages) B0 pages per head in sel_pages (the slots beyond
 * are -1, as tw_quest_select_ragged leaves them), so min(..) * block_size
 * valid candidates in its logits rows (N apart).  A group with no candidate
 * page keeps its sink and recent windows only (desired 0).  Batches the
 * reference's per-request top-p and GQA union (twilight_offload_cache.py
 * :1265-1311,1517-1614) for the graph-captured decode step. */
int tw_twilight_select_ragged(const float* logits, int G, int R, int N, const int32_t* sel_pages, int b0_pages,
                              float top_p, int32_t* desired, int32_t* allocated, uint32_t* head_bits,
                              int32_t* rows, int32_t* row_counts, int64_t rows_stride, int sink, int recent,
                              int block_size, const int32_t* lengths, int max_length, int page_capacity,
                              void* workspace, size_t workspace_bytes, void* stream);

/* Twilight top-p with dynamic budgets, the kept rows published per union
 * page instead of as a row list (the union attention then walks the B0
 * union pages with these row masks, tw_decode_attention_page_rows).  Same
 * selection as tw_twilight_select(_ragged): every kept candidate n = slot *
 * block_size + i of head r sets bit i of page_rows[g*page_rows_stride +
 * slot_u[g][r][slot]] (slot_u and the cleared page_rows from tw_twilight_qk
 * with the same plan stride).  desired [G][R] as tw_twilight_select.
 * lengths (nullable): ragged groups as tw_twilight_select_ragged, each
 * clamped to `length` (its max_length; page_capacity bounds their candidate
 * pages); else every group has `length` tokens.  block_size <= 32, and it
 * divides or is divided by the candidates each thread holds (2 to 32, a power
 * of two: true for power-of-two page sizes); workspace as tw_twilight_select.
 * No counterpart in the reference, which builds the union row list
 * (twilight_offload_cache.py:1517-1614); the row set is the same. */
int tw_twilight_select_pages(const float* logits, int G, int R, int N, const int32_t* sel_pages, int b0_pages,
                             float top_p, const int32_t* slot_u, uint32_t* page_rows, int64_t page_rows_stride,
                             int32_t* desired, int sink, int recent, int block_size, int length,
                             const int32_t* lengths, int page_capacity, void* workspace, size_t workspace_bytes,
                             void* stream);

/* Words (32-bit) of one KV group's Twilight union record over P scored
 * pages (the output of tw_twilight_select_fused, the input of
 * tw_decode_attention_union): a page bitmap of 2*ceil(P/64) words (bit p of
 * word p/32: some head keeps a row of page p), then, from the next multiple
 * of 4 words, each page's kept rows as a 16-bit mask, two pages per word
 * (page p in bits 16*(p&1) .. of word p/2), padded to 16 bytes. */
int tw_twilight_union_record_words(int P);

/* Workspace bytes of tw_twilight_select_fused. */
size_t tw_twilight_select_fused_workspace_size(int G, int R, int P, int b0_pages);

/* The whole Twilight selection of a layer in two launches, dynamic budgets:
 * a score + INT4 QK launch (one block per KV group and 64-page tile: the
 * Quest score of the tile's pages for the R heads, bit for bit as
 * tw_quest_select, and the INT4 QK estimate of every row of those pages for
 * the R heads, the logits of tw_twilight_qk bit for bit), then one block
 * per (group, head) that picks the head's B0 pages (the top b0_pages
 * scores, ties to the lowest page), gathers their rows' logits, keeps the
 * top-p rows (the desired count and set of tw_twilight_select in dynamic
 * mode) and ORs them into the group's union record (union_rec +
 * g*rec_stride, tw_twilight_union_record_words(P) <= rec_stride, a multiple
 * of 4; 16-byte aligned), which the first launch clears.  No union plan or
 * row list is built.
 *   q [G][R][128] fp32; page_min/page_max as tw_quest_select (P pages,
 *   16-bit); packed / qscale / qmin the INT4 keys of tw_build_page_metadata
 *   (quant_entry_stride rows apart, quant_rows >= sink + 16*P valid rows,
 *   packed 16-byte aligned); qk_scale the logit scale (1/sqrt(D) in the reference);
 *   lengths (nullable, device [G] int32): group g has min(lengths[g],
 *   length) tokens, so its own candidate pages P_g <= P and min(b0_pages,
 *   P_g) B0 pages; else every group has `length` tokens and P candidate
 *   pages.  Outputs: desired [G][R] (the top-p counts, 0 for a group with no
 *   candidate); sel_pages [G][R][b0_pages] (nullable; ascending, -1 past a
 *   ragged group's pages); logits [G][R][b0_pages*16] (nullable).
 * D = 128, block_size 16, R <= 8, P <= 8192, b0_pages*16 <= 8192.
 * Workspace: tw_twilight_select_fused_workspace_size(G, R, P, b0_pages)
 * bytes (scores, per-tile key ranges, the rows' logits; no state carries
 * over between calls).  Replaces
 * prepare_layer_selection's stages 1-2 and the GPU GQA union of the
 * dynamic-budget path (twilight_offload_cache.py:996-1614); the union is
 * the reference's token set, held as page row masks. */
int tw_twilight_select_fused(const float* q, const void* page_min, const void* page_max, int dtype, int G, int R,
                             int P, int D, int64_t page_group_stride, const uint8_t* packed, const void* qscale,
                             const void* qmin, int64_t quant_entry_stride, int64_t quant_rows, int b0_pages,
                             float top_p, float qk_scale, int sink, int recent, int block_size,
                             const int32_t* lengths, int length, int32_t* sel_pages, float* logits, int32_t* desired,
                             uint32_t* union_rec, int64_t rec_stride, void* workspace, size_t workspace_bytes,
                             void* stream);

/* tw_twilight_select_fused with its launches chosen, for timing one of them
 * in isolation: phase 1 runs the score + INT4 QK launch only (its
 * workspace outputs and the cleared records; desired and the other outputs
 * are left as they were), phase 3 the whole selection.  No counterpart in
 * the reference: the measurement's per-kernel split of
 * prepare_layer_selection (twilight_offload_cache.py:996-1614). */
int tw_twilight_select_fused_phase(const float* q, const void* page_min, const void* page_max, int dtype, int G,
                                   int R, int P, int D, int64_t page_group_stride, const uint8_t* packed,
                                   const void* qscale, const void* qmin, int64_t quant_entry_stride,
                                   int64_t quant_rows, int b0_pages, float top_p, float qk_scale, int sink,
                                   int recent, int block_size, const int32_t* lengths, int length,
                                   int32_t* sel_pages, float* logits, int32_t* desired, uint32_t* union_rec,
                                   int64_t rec_stride, void* workspace, size_t workspace_bytes, int phase,
                                   void* stream);

/* tw_twilight_select_fused with matched budgets, in three launches: the
 * score + INT4 QK launch, the per-head B0 + top-p launch (desired counts, no
 * record), then one block per (group, head) that forms the group's
 * allocation (matched_budget_counts of the desired counts towards
 * target_total, twilight_offload_cache.py:50-86, the same as
 * tw_twilight_select in matched mode), keeps the head's top-allocated
 * candidates by logit (ties to the lower candidate) and ORs their rows into
 * the union record.  lengths null: every group has `length` tokens and
 * target_total rows (R <= target_total <= R*b0_pages*16); lengths (device,
 * [G] int32): group g has min(lengths[g], length) tokens, its own candidate
 * and B0 pages (as tw_twilight_select_fused), and target fixed_g*16*R with
 * fixed_g = min(candidates_g, max(1, ceil(matched_fraction * eligible_g /
 * 16))) (twilight_offload_cache.py:1019-1083; at most every candidate),
 * 0 < matched_fraction <= 1.  sel_pages is required (the last launch reads
 * it).  Outputs as tw_twilight_select_fused plus allocated [G][R]
 * (nullable).  Workspace: tw_twilight_select_fused_workspace_size.
 * Replaces prepare_layer_selection's stages 1-2, the matched reallocation
 * and the GPU GQA union of the matched path (twilight_offload_cache.py:
 * 996-1614). */
int tw_twilight_select_fused_matched(const float* q, const void* page_min, const void* page_max, int dtype, int G,
                                     int R, int P, int D, int64_t page_group_stride, const uint8_t* packed,
                                     const void* qscale, const void* qmin, int64_t quant_entry_stride,
                                     int64_t quant_rows, int b0_pages, float top_p, float qk_scale, int sink,
                                     int recent, int block_size, const int32_t* lengths, int length,
                                     int target_total, double matched_fraction, int32_t* sel_pages, float* logits,
                                     int32_t* desired, int32_t* allocated, uint32_t* union_rec, int64_t rec_stride,
                                     void* workspace, size_t workspace_bytes, void* stream);
/* tw_twilight_select_fused_matched for a KV group of more than 8 query heads,
 * run as sub-groups of at most 8 (R here) that share one allocation over all
 * heads_all <= 64 heads of the group, in two parts per sub-group.  Part 1:
 * the score + INT4 QK launch and the head launch, the sub-group's top-p counts
 * into desired [G][R] (and its B0 pages, logits and key ranges into sel_pages
 * and the workspace; union_rec cleared).  Part 2, once the caller has placed
 * every sub-group's counts in desired_all [G][heads_all] (this sub-group's at
 * columns head0 .. head0 + R - 1): the allocation over all heads_all heads
 * (matched_budget_counts towards target_total, or with lengths fixed_g * 16 *
 * heads_all; twilight_offload_cache.py:50-86, 1019-1083) and this
 * sub-group's top-allocated rows ORed into union_rec, with the same
 * workspace, sel_pages and union_rec as its part 1.  The group's union is
 * the OR of its sub-groups' records.  Other arguments as
 * tw_twilight_select_fused_matched.  Replaces the matched path of
 * prepare_layer_selection for wide GQA groups (twilight_offload_cache.py:
 * 996-1614), which has no head limit. */
int tw_twilight_select_fused_matched_part(const float* q, const void* page_min, const void* page_max, int dtype,
                                          int G, int R, int P, int D, int64_t page_group_stride,
                                          const uint8_t* packed, const void* qscale, const void* qmin,
                                          int64_t quant_entry_stride, int64_t quant_rows, int b0_pages, float top_p,
                                          float qk_scale, int sink, int recent, int block_size,
                                          const int32_t* lengths, int length, int target_total,
                                          double matched_fraction, int32_t* sel_pages, float* logits,
                                          int32_t* desired, int32_t* allocated, uint32_t* union_rec,
                                          int64_t rec_stride, int part, const int32_t* desired_all, int heads_all,
                                          int head0, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Sparse GQA decode attention, split-K over selected rows, one query
 * token per group.  Replaces _flash_attention_varlen_forward
 * (mp.py:21-52) on the decode paths that call it (GQA group branch
 * mp.py:239-279, layer-flat branch :283-321, per-head reference :424-452).
 *
 * Group g (G = B * Hk sequences x KV heads) attends with its R query heads
 *   q[g][r][0..D)                       (dtype, contiguous [G][R][D])
 * over its rows.  Two row modes:
 *   rows != NULL (indexed): row i of group g is position rows[g*rows_stride+i]
 *     of entry g, i.e. k_base + (g*entry_stride_rows + pos) * D, for
 *     i < row_counts[g]; optional row_masks drop heads per row.
 *   rows == NULL (varlen): cu_seqlens_k[B+1] (int32, device) delimits
 *     sequence b = g / Hk; row i of group g is
 *     k_base + (cu_seqlens_k[b] + i) * (Hk*D) + (g % Hk) * D.
 *     window_left >= 0 keeps only the last window_left+1 keys
 *     (flash-attn window_size=(w,w) at q_len 1).
 * cur_k/cur_v (nullable, [G][D]): one extra key/value appended after the
 * rows of each group (the decode token).
 * softmax_scale multiplies q.k; out [G][R][D] in dtype.  k_base/v_base may
 * point at HBM or at mapped pinned host memory.  max_rows bounds every
 * group's row count and sizes the grid.
 * ---------------------------------------------------------------------- */
size_t tw_decode_attention_workspace_size(int G, int R, int D, int max_rows);
/* The same attention over a union plan from tw_quest_select: group g's rows
 * are [0, sink_end) ++ the plan's pages expanded to block_size rows each
 * (heads per plan_masks, nullable = all) ++ [recent_start, length) ++ the
 * decode token, read by position from the group's entry
 * (k_base + (g*entry_stride_rows + pos)*D).  The decode token is the cache
 * row append_position (if >= 0) or, when cur_k/cur_v ([G][D]) are given,
 * cur_k/cur_v -- which the call then also writes to row append_position of
 * every entry (the per-step append, quest_offload_cache.py:633-638, fused
 * into the attention launch).  max_rows bounds every group's row count
 * (sink_end + max_pages*block_size + recent rows + 1) and sizes the grid and
 * the workspace (tw_decode_attention_workspace_size). */
int tw_decode_attention_pages(const void* q, const void* k_base, const void* v_base, int dtype, int G, int R,
                              int D, const int32_t* plan_pages, const uint8_t* plan_masks,
                              const int32_t* plan_counts, int64_t plan_stride, int max_rows,
                              int64_t entry_stride_rows, int sink, int recent, int block_size, int length,
                              int append_position, const void* cur_k, const void* cur_v, float softmax_scale,
                              void* out, void* workspace, size_t workspace_bytes, void* stream);
/* tw_decode_attention_pages in two phases: phase 1 launches only the split-K
 * kernel (groups that span one chunk get their final output; the others
 * leave (m, l, o) partials in the workspace), phase 2 only the merge of those
 * partials into out, phase 3 both (= tw_decode_attention_pages).  Phase 2
 * takes the arguments and the workspace of the phase-1 call it completes.
 * For callers that combine or time the two halves separately (e.g. partials
 * combined across devices before the merge). */
int tw_decode_attention_pages_phase(const void* q, const void* k_base, const void* v_base, int dtype, int G,
                                    int R, int D, const int32_t* plan_pages, const uint8_t* plan_masks,
                                    const int32_t* plan_counts, int64_t plan_stride, int max_rows,
                                    int64_t entry_stride_rows, int sink, int recent, int block_size, int length,
                                    int append_position, const void* cur_k, const void* cur_v, float softmax_scale,
                                    void* out, void* workspace, size_t workspace_bytes, int phase, void* stream);
/* Ragged tw_decode_attention_pages: group g attends with the window of its
 * own length lengths[g] (int32, device) -- [0, sink_end) ++ its union pages
 * ++ [recent_start, L_g) ++ the decode token, which is cur_k/cur_v[g] (also
 * written to row L_g of the entry when append != 0) or, without cur_k, the
 * cache row L_g (append != 0) or none (append == 0).  16-bit K/V, D = 128,
 * block_size = 16 (the page-tile kernel).  max_rows >= sink + recent bounds
 * every group's rows with its union pages (plan pages beyond it are not
 * attended); lengths[g] must be below entry_stride_rows (larger values are
 * clamped).  Workspace as tw_decode_attention_workspace_size(G, R, D,
 * max_rows).  Batches the reference's batch-1 GQA decode attention
 * (mp.py:239-279) over requests.  page_min/page_max (nullable, append != 0):
 * the decode-time metadata update of tw_update_page_metadata_ragged fused
 * in -- when the appended row L_g completes page p ((L_g - sink + 1) % 16 ==
 * 0, p < meta_pages), page_min/page_max[g * page_entry_stride + p * D ..]
 * (16-bit, 4-byte aligned) get that page's min/max. */
int tw_decode_attention_pages_ragged(const void* q, const void* k_base, const void* v_base, int dtype, int G, int R,
                                     int D, const int32_t* plan_pages, const uint8_t* plan_masks,
                                     const int32_t* plan_counts, int64_t plan_stride, int max_rows,
                                     int64_t entry_stride_rows, int sink, int recent, int block_size,
                                     const int32_t* lengths, int append, const void* cur_k, const void* cur_v,
                                     float softmax_scale, void* page_min, void* page_max,
                                     int64_t page_entry_stride, int meta_pages, void* out, void* workspace,
                                     size_t workspace_bytes, void* stream);

/* The page-tile attention of tw_decode_attention_pages(_ragged) with the
 * union taken from selection bitmaps (tw_quest_select_bits) instead of a
 * union plan: group g's union pages are the pages p < P whose bit is set in
 * any of its R rows sel_bits[(g*R + r)*bits_stride ..], in ascending order,
 * each attended by the heads whose bit is set (the plan's head masks).  The
 * same tiles in the same order as the plan path, so the output is the same.
 * lengths (nullable, device) or length, append, cur_k/cur_v and the fused
 * page metadata update (page_min/page_max) as tw_decode_attention_page_rows;
 * phase as tw_decode_attention_pages_phase.  P <= 8192 (128 words a row),
 * bits_stride even, sel_bits 8-byte aligned; D = 128, 16-row pages, 16-bit
 * K/V, R <= 8; max_rows bounds every group's rows (sink_end + union pages *
 * 16 + recent rows + 1); workspace as tw_decode_attention for max_rows. */
int tw_decode_attention_pages_bits(const void* q, const void* k_base, const void* v_base, int dtype, int G, int R,
                                   int D, const uint32_t* sel_bits, int64_t bits_stride, int P, int max_rows,
                                   int64_t entry_stride_rows, int sink, int recent, int block_size,
                                   const int32_t* lengths, int length, int append, const void* cur_k,
                                   const void* cur_v, float softmax_scale, void* page_min, void* page_max,
                                   int64_t page_entry_stride, int meta_pages, void* out, void* workspace,
                                   size_t workspace_bytes, int phase, void* stream);

/* The Twilight union attention from a union record (tw_twilight_select_
 * fused): the page-tile attention over the sink rows, the kept rows of every
 * union page (the pages whose bitmap bit is set, ascending; every head
 * attends every kept row, the rows no head keeps are neither read nor
 * attended), the recent rows and the decode token.  The block stages the
 * group's row masks in LDS in the same round trip as the bitmap.  lengths /
 * length, append, cur_k/cur_v, page_min/page_max and packed/qscale/qmin (the
 * appended row's INT4 code) as tw_decode_attention_page_rows; phase as
 * tw_decode_attention_pages_phase.  P <= 8192, rec_stride >=
 * tw_twilight_union_record_words(P) and a multiple of 4, union_rec 16-byte
 * aligned; D = 128, 16-row pages, 16-bit K/V, R <= 8; max_rows bounds every
 * group's rows; workspace as tw_decode_attention for max_rows.  The
 * reference attends the GQA-group union rows (mp.py:239-279); the rows are
 * the same set. */
int tw_decode_attention_union(const void* q, const void* k_base, const void* v_base, int dtype, int G, int R, int D,
                              const uint32_t* union_rec, int64_t rec_stride, int P, int max_rows,
                              int64_t entry_stride_rows, int sink, int recent, int block_size, const int32_t* lengths,
                              int length, int append, const void* cur_k, const void* cur_v, float softmax_scale,
                              void* page_min, void* page_max, int64_t page_entry_stride, int meta_pages,
                              uint8_t* packed, void* qscale, void* qmin, int64_t quant_entry_stride, void* out,
                              void* workspace, size_t workspace_bytes, int phase, void* stream);
/* tw_decode_attention_union with the previous-token resident cache of the
 * Twilight cache (previous_token_resident_cache, twilight_offload_cache.py:
 * 2457-2608, 3323-3470; hit/miss mapping resident_gpu_mapping.py:14-144),
 * for slabs in host memory: the reference keeps the previous token's union
 * rows on the GPU and reads only the new rows from the host.  Here every
 * group keeps the rows of its last union in res_k/res_v [G][2][res_slots][16]
 * [D] (16-bit, HBM; two buffers alternating with the length's parity, a page
 * a slot at its union index, res_slots <= 65535), and res_map [G]
 * [res_map_pages] (int64, initialised to -1) = (length << 32) | (the page's
 * kept rows << 16) | slot: a kept row that the previous step kept too is
 * read from HBM, every other kept row from the slab, and every union page
 * read is stored for the next step.  res_stats [G][2] (nullable) accumulates
 * (hit rows, union rows).  The resident sink and recent windows (res_win_k,
 * res_win_v, res_win_state, ring_rows) as tw_decode_attention_pages_
 * resident.  Other arguments as tw_decode_attention_union. */
int tw_decode_attention_union_resident(const void* q, const void* k_base, const void* v_base, int dtype, int G,
                                       int R, int D, const uint32_t* union_rec, int64_t rec_stride, int P,
                                       int max_rows, int64_t entry_stride_rows, int sink, int recent,
                                       int block_size, const int32_t* lengths, int length, int append,
                                       const void* cur_k, const void* cur_v, float softmax_scale, void* res_k,
                                       void* res_v, int64_t* res_map, int res_slots, int res_map_pages,
                                       unsigned long long* res_stats, void* res_win_k, void* res_win_v,
                                       int32_t* res_win_state, int ring_rows, void* page_min, void* page_max,
                                       int64_t page_entry_stride, int meta_pages, uint8_t* packed, void* qscale,
                                       void* qmin, int64_t quant_entry_stride, void* out, void* workspace,
                                       size_t workspace_bytes, int phase, void* stream);
/* The Twilight union attention over page rows: the page-tile attention of
 * tw_decode_attention_pages(_ragged) where plan_pages / plan_counts are the
 * B0 union (tw_quest_select with k = b0_pages) and page_rows[g*plan_stride +
 * u] (tw_twilight_select_pages) says which rows of union page u are kept.
 * Every head attends every kept row (the GQA union of
 * twilight_offload_cache.py:1517-1614 with mp.py:239-279), the sink and
 * recent windows and the decode token; rows not kept are neither read nor
 * attended.  lengths (nullable) or length, append, cur_k / cur_v, the page
 * metadata of a completed page (page_min/page_max) and, with packed / qscale /
 * qmin [G][quant_entry_stride] (16-bit K), the appended row's INT4 code, as
 * tw_decode_attention_pages_ragged and tw_decode_attention_rows_append do.
 * D = 128, 16-row pages, 16-bit K/V, R <= 8; workspace as tw_decode_attention
 * for max_rows. */
int tw_decode_attention_page_rows(const void* q, const void* k_base, const void* v_base, int dtype, int G, int R,
                                  int D, const int32_t* plan_pages, const int32_t* plan_counts,
                                  const uint32_t* page_rows, int64_t plan_stride, int max_rows,
                                  int64_t entry_stride_rows, int sink, int recent, int block_size,
                                  const int32_t* lengths, int length, int append, const void* cur_k,
                                  const void* cur_v, float softmax_scale, void* page_min, void* page_max,
                                  int64_t page_entry_stride, int meta_pages, uint8_t* packed, void* qscale,
                                  void* qmin, int64_t quant_entry_stride, void* out, void* workspace,
                                  size_t workspace_bytes, void* stream);
/* Page-tile attention with a resident page cache in HBM, for slabs in host
 * memory.  Replaces the previous-token resident cache of the Twilight cache
 * (previous_token_resident_cache, twilight_offload_cache.py:2457-2608,
 * 3323-3470; hit/miss mapping resident_gpu_mapping.py:14-144), which keeps
 * the previous token's selected rows on the GPU and fetches only the misses
 * from the host.  Here every group keeps the K/V pages of its last union in
 * res_k/res_v [G][2][res_slots][16][D] (16-bit, HBM): a page the previous
 * step stored is read from there instead of the slab, and every union page
 * read (hit or miss) is stored into the buffer of this step's parity at its
 * union index, with res_map[g][page] = (length << 32) | index (int64,
 * [G][res_map_pages], initialised to -1).  res_stats [G][2] (nullable)
 * accumulates (hit pages, union pages).  lengths (device, per group) or,
 * when NULL, `length` for every group gives the window and the decode token
 * row, which is appended there from cur_k/cur_v when append != 0 -- the
 * semantics of tw_decode_attention_pages_ragged, as is the fused page
 * metadata update (page_min/page_max).  Union indexes at or above res_slots
 * are read from the slab and not stored.
 *   Resident windows (res_win_k nullable): res_win_k/res_win_v [G][sink +
 * ring_rows][D] (16-byte aligned; ring_rows a power of two >= recent) keep
 * each group's sink rows at [0, sink) and its latest ring_rows rows at sink
 * + (row & (ring_rows - 1)), and res_win_state [G][2] int32 (zeroed before
 * the first call, and again whenever the slab's rows change other than by
 * these launches' appends) records the history length the ring serves and
 * whether the sink rows are stored.  When the previous launch ran at
 * length - 1 with a decode row, both windows are read from HBM; otherwise
 * they are read from the slab and stored, so the next step reads them from
 * HBM.  The decode row goes into its ring slot at every launch.  The
 * reference's resident rows cover the sink and recent windows too
 * (twilight_offload_cache.py:3323-3330). */
int tw_decode_attention_pages_resident(const void* q, const void* k_base, const void* v_base, int dtype, int G,
                                       int R, int D, const int32_t* plan_pages, const uint8_t* plan_masks,
                                       const int32_t* plan_counts, int64_t plan_stride, int max_rows,
                                       int64_t entry_stride_rows, int sink, int recent, int block_size,
                                       const int32_t* lengths, int length, int append, const void* cur_k,
                                       const void* cur_v, float softmax_scale, void* res_k, void* res_v,
                                       int64_t* res_map, int res_slots, int res_map_pages,
                                       unsigned long long* res_stats, void* res_win_k, void* res_win_v,
                                       int32_t* res_win_state, int ring_rows, void* page_min, void* page_max,
                                       int64_t page_entry_stride, int meta_pages, void* out, void* workspace,
                                       size_t workspace_bytes, void* stream);
int tw_decode_attention(const void* q, const void* k_base, const void* v_base, int dtype, int G,
                        int R, int D, const int32_t* rows, const uint8_t* row_masks,
                        const int32_t* row_counts, int64_t rows_stride, int64_t entry_stride_rows,
                        const int32_t* cu_seqlens_k, int Hk, int window_left, int max_rows,
                        const void* cur_k, const void* cur_v, float softmax_scale, void* out,
                        void* workspace, size_t workspace_bytes, void* stream);
/* tw_decode_attention over a row list with the decode token's append fused:
 * the first block of every group also writes cur_k/cur_v[g] to row
 * append_position of entry g (0 <= append_position < entry_stride_rows), or,
 * when append_rows (int32 [G], device) is given, to row append_rows[g]
 * (rows outside the entry are skipped); the row list must not name it.
 * Optional (16-bit keys, D = 128): the decode-time metadata update of
 * tw_update_page_metadata for the appended row -- its INT4 code, scale and
 * minimum into packed / quant_scale / quant_min (row g * quant_entry_stride
 * + row) and, when it completes page p ((row - sink + 1) % 16 == 0,
 * p < meta_pages), that page's min/max into page_min / page_max (g *
 * page_entry_stride + p * 128).  Replaces the Twilight decode step's GQA
 * decode attention over the union rows (mp.py:239-279) followed by the
 * batched new-KV append (twilight_offload_cache.py:551-794). */
int tw_decode_attention_rows_append(const void* q, const void* k_base, const void* v_base, int dtype, int G, int R,
                                    int D, const int32_t* rows, const uint8_t* row_masks, const int32_t* row_counts,
                                    int64_t rows_stride, int64_t entry_stride_rows, int max_rows,
                                    const void* cur_k, const void* cur_v, int64_t append_position,
                                    const int32_t* append_rows, float softmax_scale, int sink, void* page_min,
                                    void* page_max, int64_t page_entry_stride, int meta_pages, uint8_t* packed,
                                    void* quant_scale, void* quant_min, int64_t quant_entry_stride, void* out,
                                    void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Head-wise K/V row gather into the attention layout.
 * Replaces the CPU index_select + H2D of update / update_layer_flat_ragged /
 * update_layer_gqa_group_ragged (quest_offload_cache.py:576-624,816-936;
 * twilight_offload_cache.py:2973-3101) and the mapped-host assembly kernel
 * launch_resident_zero_copy (resident_zero_copy.cu:44-65).
 *   src_k/src_v: row r at + r*D (HBM, or the device alias of mapped pinned
 *   host memory returned by tw_host_device_pointer).
 *   src_rows [n] int64 source rows (absolute, i.e. entry*Lmax + pos);
 *   dst_rows (nullable) [n] int64 destination rows (NULL: dst row = i, and
 *   n must not exceed dst_row_limit); dst_k/dst_v hold dst_row_limit rows.
 *   A pair whose source row is outside [0, src_row_limit) or whose
 *   destination row is outside [0, dst_row_limit) is not copied; the call
 *   then still completes and sets *error_flag (device int32, nullable) to 1.
 * Bit-exact copies.
 * ---------------------------------------------------------------------- */
int tw_gather_rows(const void* src_k, const void* src_v, int64_t src_row_limit,
                   const int64_t* src_rows, const int64_t* dst_rows, int64_t n, int64_t dst_row_limit, int D,
                   int elem_bytes, void* dst_k, void* dst_v, int32_t* error_flag, void* stream);

/* Group-union gather of the GQA group path: replaces the per-layer union
 * gather + H2D + current-token gap fill of update_layer_gqa_group_ragged
 * (twilight_offload_cache.py:2936-3101,3290-3310).  Entry of group g starts
 * at source row entry_row0 + g*entry_row_step (row = entry*Lmax + pos, the
 * slab layout of slab_cache.py:36-73).  Group g's rows[g*rows_stride + i],
 * i < row_counts[g] (device, clamped to max_count), then cur_k[g]/cur_v[g]
 * ([G][D]), are written back to back into dst ([dst_capacity][D]); group g
 * starts at sum_{h<g}(row_counts[h] + 1) and cu_seqlens[G+1] (int32,
 * device) receives those offsets (the varlen cu_seqlens_k of the attention).
 * Out-of-range rows are skipped and set *error_flag.  No host sync. */
int tw_gather_union(const void* src_k, const void* src_v, int64_t src_row_limit, int64_t entry_row0,
                    int64_t entry_row_step, const int32_t* rows, int64_t rows_stride, const int32_t* row_counts,
                    int G, int max_count, const void* cur_k, const void* cur_v, int D, int elem_bytes,
                    int64_t dst_capacity, void* dst_k, void* dst_v, int32_t* cu_seqlens, int32_t* error_flag,
                    void* stream);
/* tw_gather_union with the previous-token resident cache of the GQA-group
 * path (previous_token_resident_cache, twilight_offload_cache.py:2457-2608,
 * 3323-3470; hit/miss mapping resident_gpu_mapping.py:14-144, which maps the
 * current union onto the previous one and copies hits from the previous
 * snapshot): res_map [G][map_stride] (int64, initialised to -1; map_stride
 * above every position) holds (epoch << 32) | index of the step that last
 * packed each position, prev_k/prev_v [prev_capacity][D] that step's packed
 * output and prev_cu [G + 1] its cu_seqlens.  A union row whose entry names
 * epoch - 1 is copied from prev_k/prev_v (HBM) instead of the slab; the
 * entries of this step's rows then name epoch (this step's history length,
 * >= 1) and their index in dst.  res_stats [2] (nullable) accumulates (rows
 * copied from the previous step, union rows).  Other arguments as
 * tw_gather_union. */
int tw_gather_union_resident(const void* src_k, const void* src_v, int64_t src_row_limit, int64_t entry_row0,
                             int64_t entry_row_step, const int32_t* rows, int64_t rows_stride,
                             const int32_t* row_counts, int G, int max_count, const void* cur_k, const void* cur_v,
                             int D, int elem_bytes, int64_t dst_capacity, void* dst_k, void* dst_v,
                             int32_t* cu_seqlens, int32_t* error_flag, int64_t* res_map, int64_t map_stride,
                             int epoch, const void* prev_k, const void* prev_v, const int32_t* prev_cu,
                             int64_t prev_capacity, unsigned long long* res_stats, void* stream);

/* Per-query-head gather of the Quest paths: replaces the per-head CPU
 * index_select + H2D + current-token write of update (quest_offload_cache.py:
 * 576-637) and the layer-flat ragged pack (:816-936).  Head r of group g sees
 * [0, sink_end) ++ sel_pages[g][r][0..k) (ascending) expanded to block_size
 * rows ++ [recent_start, length) and then cur_k[g]/cur_v[g]; its row t goes
 * to dst row g*dst_g_stride + r*dst_r_stride + t*dst_t_stride (pack [1, Tmax,
 * R, D]: strides (.., 1, R); flat segments: ((R*(len+1)), len+1, 1)).  The
 * window is that of tw_quest_select.  All rows must land below dst_capacity. */
int tw_gather_heads(const void* src_k, const void* src_v, int64_t src_row_limit, int64_t entry_row0,
                    int64_t entry_row_step, const int32_t* sel_pages, int G, int R, int k, int sink, int recent,
                    int block_size, int length, const void* cur_k, const void* cur_v, int D, int elem_bytes,
                    int64_t dst_g_stride, int64_t dst_r_stride, int64_t dst_t_stride, int64_t dst_capacity,
                    void* dst_k, void* dst_v, int32_t* error_flag, void* stream);

/* Device address of pinned host memory allocated by hipHostMalloc (torch
 * pin_memory=True); replaces cudaHostGetDevicePointer in
 * resident_zero_copy.py:149-163. */
int tw_host_device_pointer(void* host_ptr, void** device_ptr);

/* ------------------------------------------------------------------------
 * Per-step append of the decode token.  Replaces _schedule_d2h
 * (quest_offload_cache.py:230-274) and the token-batched new-KV D2H
 * (twilight_offload_cache.py:551-794).  For each of n_entries entries,
 * row `position` of entry (first_entry + i) in dst_k/dst_v ([E][Lmax][D],
 * HBM or mapped pinned host) receives new_k[i]/new_v[i] ([n][D]).
 * ---------------------------------------------------------------------- */
int tw_append_kv(const void* new_k, const void* new_v, int n_entries, int D, int elem_bytes,
                 void* dst_k, void* dst_v, int64_t entry_stride_rows, int first_entry,
                 int64_t position, void* stream);

/* ------------------------------------------------------------------------
 * Element-wise steps of the graph-captured decode token around the sparse
 * path (16-bit activations).  No counterpart in the reference's path: they
 * stand for the HF modules the reference runs unpatched, with their rounding
 * steps (each element-wise op in fp32, rounded to the activation dtype).
 *   tw_add_rms_norm: h = h + delta (delta nullable), out = weight *
 *     (h * rsqrt(mean(h^2) + eps)) -- the decoder layer's residual add and
 *     LlamaRMSNorm; h [rows][H] updated in place.  H % 8 == 0, H <= 8192,
 *     16-byte aligned rows.
 *   tw_rope_qk: apply_rotary_pos_emb of q [Hq][D] and k [Hk][D] in place at
 *     the position *position (device int64) of the cos/sin tables
 *     [positions][D]; q32 (nullable) [Hq][D] receives q in fp32.
 *   tw_silu_mul: out[i] = silu(gate_up[i]) * gate_up[I + i] (LlamaMLP's
 *     act_fn(gate_proj(x)) * up_proj(x) over a fused gate/up projection).
 * ---------------------------------------------------------------------- */
int tw_add_rms_norm(void* h, const void* delta, const void* weight, float eps, void* out, int rows, int H,
                    int dtype, void* stream);
int tw_rope_qk(void* q, void* k, int Hq, int Hk, int D, const void* cos_table, const void* sin_table,
               const int64_t* position, float* q32, int dtype, void* stream);
int tw_silu_mul(const void* gate_up, void* out, int I, int dtype, void* stream);
/* tw_gemv: y [N] = x [K] . W[n][:] (+ bias [N], nullable) for one token,
 * W [N][K] row-major (nn.Linear's weight), fp32 accumulation, output in the
 * 16-bit dtype.  K % 8 == 0, K <= 32768, 16-byte aligned W and x. */
int tw_gemv(const void* W, const void* x, const void* bias, void* y, int N, int K, int dtype, void* stream);
/* The GEMV with the decoder layer's residual add + RMSNorm as its input:
 * x = RMSNorm(h_in + delta) as tw_add_rms_norm computes it (every block
 * normalises the row itself; delta nullable), h_out = h_in + delta (written
 * when delta is given; a buffer other than h_in and delta), then
 * y = x . W[n] (+ bias) as tw_gemv.  K % 8 == 0, K <= 8192.
 *   tw_rms_norm_gemv: y [N].
 *   tw_rms_norm_gemv_rope: W is the concatenated q/k/v projection
 *     [(Hq + Hk + Hv) * D][K]; y [N] gets q and k rotated at *position as
 *     tw_rope_qk does (q also to q32 [Hq][D], nullable).
 *   tw_rms_norm_gemv_silu: W is the concatenated gate/up projection [2I][K];
 *     y [I] = silu(gate) * up as tw_silu_mul does.
 * Same bits as the separate launches.  No counterpart in the reference's
 * path (the HF decoder layer's modules, run unpatched by the reference). */
int tw_rms_norm_gemv(const void* h_in, const void* delta, const void* norm_weight, float eps, void* h_out,
                     const void* W, const void* bias, void* y, int N, int K, int dtype, void* stream);
int tw_rms_norm_gemv_rope(const void* h_in, const void* delta, const void* norm_weight, float eps, void* h_out,
                          const void* W, const void* bias, void* y, int N, int K, int Hq, int Hk, int D,
                          const void* cos_table, const void* sin_table, const int64_t* position, float* q32,
                          int dtype, void* stream);
int tw_rms_norm_gemv_silu(const void* h_in, const void* delta, const void* norm_weight, float eps, void* h_out,
                          const void* W, const void* bias, void* y, int N, int K, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TWILIGHT_HIP_H */
