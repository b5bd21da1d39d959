/*
 * aspire_hip.h - C ABI of the MI355X (gfx950) mixed draft/verify paged-KV
 * attention library (libaspire_hip.so).
 *
 * Plain pointers, sizes and strides only. Every device entry point takes the
 * HIP stream to enqueue on (a hipStream_t passed as void*; NULL = the null
 * stream), never synchronises, and returns 0 on success or a nonzero
 * aspire_status code; aspire_last_error() then describes the failure (the
 * message is per host thread).
 *
 * Tensor conventions (all element strides, not bytes):
 *   q / out      [T, H_q, 128] bf16, head_dim contiguous
 *   kv_cache     [P, 2, 16, H_kv, 128] bf16: K at [:,0], V at [:,1]
 *   page lists   int32 CSR: kv_indptr (pages) + kv_indices (physical page ids)
 *   lse          [T, H_q] fp32, base-2 log-sum-exp
 */
#ifndef ASPIRE_HIP_H
#define ASPIRE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum aspire_status {
  ASPIRE_OK = 0,
  ASPIRE_ERR_INVALID = 1,     /* bad argument, shape or unsupported configuration */
  ASPIRE_ERR_CAPACITY = 2,    /* a workspace or plan capacity would be exceeded */
  ASPIRE_ERR_HIP = 3          /* a HIP runtime call failed */
};

/* Description of the last failure on this host thread ("" if none). */
const char* aspire_last_error(void);

/* Build identity: version, target and compile flags.
 * Replaces validate_flashinfer_patch (aspire/attention/flashinfer.py:14-60),
 * which checked the patched FlashInfer sources; the Python layer returns this
 * string and its sha256 in the same dict shape. */
const char* aspire_build_info(void);

/* KV tile (tokens) the attention kernel processes per step, the pad multiple
 * for the logits-dump stride. Replaces compute_max_cta_tile_kv
 * (aspire/attention/flashinfer.py:63-105). The kernel keeps the kv_idx < kv_len
 * guard on dump writes, so any stride >= max_seq_length is safe. */
int32_t aspire_max_kv_tile(void);

/* ---------------------------------------------------------------- (a1) -- */
/* Paged KV append. Replaces mylib::update_kv_padded
 * (aspire/attention/kv_ops.py:127-187) and its three launches: FlashInfer
 * get_seq_lens (kv_ops.py:141-143), get_batch_indices_positions_kernel
 * (kv_ops.py:144-156) and _append_paged_kv_cache_padded_kernel
 * (kv_ops.py:63-124), fused into one kernel.
 * Row b of the first num_seq rows (num_seq = len(kv_last_page_len)) owns the
 * append tokens [append_indptr[b], append_indptr[b+1]) and the pages
 * kv_page_indices[kv_page_indptr[b] : kv_page_indptr[b+1]];
 * append_indptr and kv_page_indptr hold at least num_seq + 1 entries.
 * Token i of row b lands at position kv_len_b - (append_indptr[b+1] - i) with
 * kv_len_b = max(pages_b - 1, 0) * page_size + kv_last_page_len[b]; tokens
 * with a negative position, of rows without pages, past kv_len_b, or covered
 * by no row are skipped. head_dim must be 128; k and v rows must be
 * contiguous per head (the reference raises ValueError otherwise). */
int aspire_paged_kv_append(const void* k, const void* v,
                           int64_t k_stride_n, int64_t k_stride_h,
                           int64_t v_stride_n, int64_t v_stride_h,
                           const int32_t* append_indptr,
                           const int32_t* kv_page_indices,
                           const int32_t* kv_page_indptr,
                           const int32_t* kv_last_page_len, int32_t num_seq,
                           void* kv_cache, int64_t cache_stride_p,
                           int64_t cache_stride_kv, int64_t cache_stride_t,
                           int64_t cache_stride_h, int32_t total_tokens,
                           int32_t num_heads, int32_t head_dim,
                           int32_t page_size, void* stream);

/* ---------------------------------------------------------------- (a2) -- */
/* Mixed draft/verify page list. Replaces build_unified_indices and
 * _copy_indices_kernel (aspire/models/sparse_draft_runner.py:92-153):
 * n_b = mode_flags[b] == 0 (DRAFT) ? draft_num_pages[b] : verify_num_pages[b];
 * indptr[0] = 0, indptr[b+1] = sum_{c<=b} n_c; the n_b entries read from the
 * flattened source table at b * width (draft or verify) are copied to
 * indices[indptr[b]]. When indptr_fill_to > batch + 1, entries
 * indptr[batch+1 : indptr_fill_to] are set to indptr[batch] (the padding-row
 * fill of aspire/backends/base.py:1253-1255). mode_flags_elem_size is 1, 4
 * or 8 (bool/uint8, int32, int64). Reads are bounded by draft_rows * width
 * and verify_rows * width; writes by indices_capacity (exceeding it sets no
 * error on the device: those entries are dropped). */
int aspire_build_mixed_page_list(const void* mode_flags, int32_t mode_flags_elem_size,
                                 const int32_t* draft_indices, int64_t draft_width,
                                 int64_t draft_rows,
                                 const int32_t* verify_indices, int64_t verify_width,
                                 int64_t verify_rows,
                                 const int32_t* draft_num_pages,
                                 const int32_t* verify_num_pages, int32_t batch,
                                 int32_t* paged_kv_indices, int64_t indices_capacity,
                                 int32_t* paged_kv_indptr, int32_t indptr_fill_to,
                                 void* stream);

/* Per-(row, kv head) page lists: the consumer of the key-mean (B) selection,
 * which has no reference code (the BASELINE config-2 refresh layer feeding the
 * following sparse layers). Segment s = b * num_kv_heads + g takes
 * selected_counts[s] entries of row s of `selected` ([batch * num_kv_heads,
 * selected_width], the KeyMeanPageSelector output) when row b drafts, and
 * verify_num_pages[b] entries of verify row b otherwise: once per head, or,
 * with share_verify, once per row with all the row's heads starting at that
 * list. paged_kv_indptr[s] receives segment s's first entry and
 * paged_kv_indptr[batch * num_kv_heads] the total (without sharing this is the
 * running count, the per-head form of aspire_build_mixed_page_list's indptr);
 * entries up to indptr_fill_to repeat the total. Same bounds and error rules
 * as aspire_build_mixed_page_list. */
int aspire_build_head_page_lists(const void* mode_flags, int32_t mode_flags_elem_size,
                                 const int32_t* selected, int64_t selected_width,
                                 const int32_t* selected_counts, const int32_t* verify_indices,
                                 int64_t verify_width, int64_t verify_rows,
                                 const int32_t* verify_num_pages, int32_t batch, int32_t num_kv_heads,
                                 int32_t share_verify, int32_t* paged_kv_indices, int64_t indices_capacity,
                                 int32_t* paged_kv_indptr, int32_t indptr_fill_to, void* stream);

/* ---------------------------------------------------------------- (a7) -- */
/* Work plan for the mixed attention kernel. Replaces the patched FlashInfer
 * TwoStageHolisticPlan (third_party/flashinfer/aspire.patch:108-288) behind
 * HolisticAttentionWrapper.plan / plan_host
 * (aspire/attention/holistic_wrapper.py:200-342).
 * The plan lives at fixed offsets of a device int workspace (so a captured
 * run() replays with new plans); aspire_plan_build fills a host (pinned)
 * mirror with no HIP calls and aspire_plan_upload copies its live segments
 * asynchronously on the given stream. */
typedef struct aspire_plan_layout {
  int32_t num_waves;          /* persistent waves per row-tile class kernel */
  int32_t max_items;          /* work items per class */
  int32_t max_merge;          /* split segments needing a merge */
  int32_t head_dim;           /* 128 */
  int64_t partial_rows_cap;   /* fp32 partial rows (head_dim + 1 floats each) */
  int64_t int_ws_bytes;       /* bytes of the int workspace the layout uses */
  int64_t float_ws_bytes;     /* bytes of the float workspace the layout uses */
} aspire_plan_layout;

typedef struct aspire_plan_info {
  int32_t num_items[3];       /* per row-tile class (<=16, <=32, <=48 rows) */
  int32_t num_merge;
  int64_t partial_rows;
  int32_t num_segments;       /* (row, kv head) segments with queries */
  int32_t max_rows;           /* largest q_len * group of any segment */
  int64_t total_pages;        /* page-heads the plan streams */
  int64_t live_bytes;         /* bytes the upload copies */
  int32_t split_rows;         /* rows cut into query tiles (q_len * group > 48): no logits dump */
} aspire_plan_info;

/* num_cus <= 0 queries the current device. waves_per_cu <= 0 uses 4 (one wave per SIMD). */
int aspire_plan_layout_init(int32_t num_cus, int32_t waves_per_cu,
                            int64_t int_ws_bytes, int64_t float_ws_bytes,
                            int32_t head_dim, aspire_plan_layout* out);

/* Rows b in [0, batch) have queries [qo_indptr[b], qo_indptr[b+1]) (host
 * arrays). per_head_lists == 0: kv_indptr has batch+1 entries and kv_len batch
 * entries (one page list per row, shared by its kv heads); otherwise
 * batch*num_kv_heads+1 and batch*num_kv_heads, one list per (row, kv head),
 * segment index b*num_kv_heads + g. A row with q_len * group > 48 (a prefill
 * chunk; group = num_qo_heads / num_kv_heads) is cut into query tiles of
 * 48 / group tokens, each streaming only the keys up to its last token when
 * causal (replaces BatchPrefillWithPagedKVCacheWrapper's plan as well). */
int aspire_plan_build(const aspire_plan_layout* layout, const int32_t* qo_indptr,
                      const int32_t* kv_indptr, const int32_t* kv_len, int32_t batch,
                      int32_t per_head_lists, int32_t num_qo_heads,
                      int32_t num_kv_heads, int32_t page_size, int32_t causal,
                      void* host_buf, int64_t host_buf_bytes,
                      aspire_plan_info* info);

/* The plan of aspire_plan_build from explicit (row, kv head) segments, for
 * page lists that are neither one per row nor laid end to end per head (no
 * reference counterpart: the per-head lists of the key-mean selection, with
 * verify rows sharing one list). Segment s = b * num_kv_heads + g streams
 * seg_kv_len[s] tokens of the seg_pages[s] entries at kv_indices[seg_start[s]].
 * When every row's heads have the same length the plan is head-aligned: rows
 * whose heads share one start stage their pages through LDS like row lists,
 * rows with a list per head load their own head's rows. */
int aspire_plan_build_segments(const aspire_plan_layout* layout, const int32_t* qo_indptr,
                               const int32_t* seg_start, const int32_t* seg_pages, const int32_t* seg_kv_len,
                               int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads, int32_t page_size,
                               int32_t causal, void* host_buf, int64_t host_buf_bytes, aspire_plan_info* info);

int aspire_plan_upload(const aspire_plan_layout* layout, const aspire_plan_info* info,
                       const void* host_buf, void* dev_buf, void* stream);

/* ------------------------------------------------------- (a4, a5, a6) -- */
/* Mixed draft/verify attention over a plan. Replaces
 * HolisticAttentionWrapper.run (aspire/attention/holistic_wrapper.py:344-386)
 * and the patched BatchPagedAttentionPersistent<64,16,...> kernel it runs
 * (aspire.patch:18-21), including the split-KV merge (aspire.patch:81-85,
 * 257-273) and, when dump_kind != 0, the logits-dump variant bound at the
 * refresh layer (aspire/backends/base.py:452-514, jit_kernels.py:74-96,
 * 182-193, 247-256). page_scores != NULL adds the per-KV-head key-mean page
 * score of BASELINE config 2 (no reference counterpart). */
typedef struct aspire_attention_args {
  const void* q; int64_t q_stride_t; int64_t q_stride_h;
  const void* kv_cache; int64_t cache_stride_p; int64_t cache_stride_kv;
  int64_t cache_stride_t; int64_t cache_stride_h;
  const int32_t* kv_indices;
  void* out; int64_t out_stride_t; int64_t out_stride_h;
  float* lse;                     /* [T, H_q] contiguous, or NULL */
  const void* plan_dev;           /* device int workspace holding the plan */
  float* float_ws;                /* device float workspace (partials) */
  int32_t num_qo_heads; int32_t num_kv_heads; int32_t head_dim; int32_t page_size;
  float sm_scale; int32_t causal;
  int32_t class_mask;             /* bit c launches row-tile class c; 7 = all (graph-safe) */
  int32_t launch_merge;           /* 0 skips the merge launch (no split segment) */
  /* logits dump: kind 0 none, 1 last_token (1 slot), 2 first_last (2 slots) */
  void* dump; int32_t dump_kind; int32_t dump_dtype; /* 0 fp16, 1 fp32 */
  int64_t dump_kv_stride; int32_t dump_num_heads;
  const int32_t* dump_mode_flags; /* per row, 0 disables; NULL = all rows */
  float* page_scores; int64_t page_score_stride; /* [segments, stride] or NULL */
  int32_t partial_nt;             /* 1: store split-KV partials non-temporally (short plans,
                                     at most 64 page-heads per wave; no reference counterpart);
                                     0 (zero-initialised callers): plain stores */
} aspire_attention_args;

int aspire_attention_run(const aspire_plan_layout* layout,
                         const aspire_attention_args* args, void* stream);

/* Size of the static device scratch of aspire_attention_run_static (bytes per
 * GPU): 64 MiB, room for 130,055 fp32 partial rows. */
#define ASPIRE_STATIC_SCRATCH_BYTES (64u << 20)

/* aspire_attention_run without any device allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments and results as aspire_attention_run, except that
 * args->float_ws must be NULL: the split-KV partials live in a static device
 * array of ASPIRE_STATIC_SCRATCH_BYTES that each GPU the library runs on holds
 * until the process ends. The layout must have been built with
 * float_ws_bytes <= ASPIRE_STATIC_SCRATCH_BYTES (ASPIRE_ERR_CAPACITY
 * otherwise), so every plan built from it fits. The stream must belong to the
 * current device. Nothing needs clearing between calls (every partial row the
 * merge reads is written first), but all calls on one GPU share the array:
 * calls that overlap on one GPU (two streams, or two host threads) race. */
int aspire_attention_run_static(const aspire_plan_layout* layout,
                                const aspire_attention_args* args, void* stream);

/* ---------------------------------------------------------------- (a6) -- */
/* Standalone merge of num_states partial states (FlashInfer merge_states
 * semantics, base-2 lse): v [num_states, rows, head_dim] fp32, s
 * [num_states, rows] fp32 -> v_out [rows, head_dim] (out_dtype 0 fp32,
 * 1 bf16), s_out [rows]. */
int aspire_merge_states(const float* v, const float* s, int32_t num_states,
                        int64_t rows, int32_t head_dim, void* v_out,
                        int32_t out_dtype, float* s_out, void* stream);

/* ---------------------------------------------------------------- (a3) -- */
/* Reference page scoring (R). slots == 2 replaces
 * PageSelectorFirstLastAvg.select / select_subset
 * (aspire/backends/page_selector.py:206-233) and _select_first_last_impl
 * (163-181); slots == 1 replaces PageSelector.select / select_subset (140-157)
 * and _select_impl (110-130). Page score j of row r (row_ids[r] or r):
 *   sum_{t in page j, t < max_seq_length} sum_{slot} max_h
 *     exp2(nan_to_num(fp32(fp16(dump * sm_scale_log2e)) - lse[q_slot, h]))
 *   + (-j * 1e-7f)
 * where q_slot is the row's first query (slot 0 of 2) or last query, for
 * j < num_pages[row], written to scores[r * score_stride + j]. The dump is
 * fp16 [bsz, n_heads, slots, kv_stride]. */
int aspire_select_first_last_scores(const void* dump, int64_t kv_stride, int32_t n_heads,
                                    int32_t bsz, int32_t max_seq_length,
                                    const float* lse, int32_t lse_rows,
                                    const int32_t* qo_indptr, const int32_t* num_pages,
                                    const int32_t* row_ids, int32_t rows,
                                    int32_t page_size, float sm_scale_log2e,
                                    float* scores, int64_t score_stride, int32_t slots,
                                    void* stream);

/* Top-k page selection for rows (R) or (row, kv head) segments (B).
 * Replaces _finalize_scores (page_selector.py:79-108) and
 * compute_valid_counts (52-62). For segment s (table row = row_ids[s /
 * segs_per_row] or s / segs_per_row): pages j < n = num_pages[that row] with
 * j >= n - L forced in; k_s = valid count (count_mode 0: min(n, subset);
 * 1: min(n, min_pages); 2: clamp(ceil(fp32(n) * pct / 100), min(n,
 * min_pages), min(n, subset))); the k_s best pages are looked up in the
 * table and written to selected[s * sel_stride + 0 .. k_s) in ascending
 * physical (order 0, the reference rule) or logical (order 1) page order,
 * zeros up to sel_width; valid[s] = k_s (if valid != NULL). */
int aspire_select_topk(const float* scores, int64_t score_stride, const int32_t* num_pages,
                       const int32_t* row_ids, int32_t segments, int32_t segs_per_row,
                       int32_t L, int32_t count_mode, int32_t subset, int32_t min_pages,
                       float pct, const int32_t* block_table, int64_t table_stride,
                       int32_t order, int32_t* selected, int64_t sel_stride,
                       int32_t sel_width, int32_t* valid, void* stream);

/* ------------------------------------------------------------------ host plan
 * Native host mirror of the per-step plan arrays. Replaces HostPlanState
 * (aspire/backends/host_plan.py:30-306): HostPlanConfig becomes
 * aspire_host_plan_config, reset_all / reset_slots become
 * aspire_host_plan_reset, build_step becomes aspire_host_plan_step. Host
 * memory only; no device work and no synchronisation. */
enum {
  ASPIRE_DRAFT_REPLAN = 0,      /* 'replan' (host_plan.py:38-39) */
  ASPIRE_DRAFT_SINK_RECENT = 1, /* 'sink_recent' */
  ASPIRE_DRAFT_GATED = 2,       /* 'gated' */
  ASPIRE_FULL_NONE = 0,         /* full_kind None: no dump wrapper */
  ASPIRE_FULL_MIRROR = 1,       /* 'mirror': dump wrapper reuses the mixed arrays */
  ASPIRE_FULL_EFFECTIVE = 2     /* 'effective_full' */
};

typedef struct aspire_host_plan_config {
  int32_t page_size;
  int32_t max_batch;
  int32_t draft_kind;        /* ASPIRE_DRAFT_* */
  int32_t full_kind;         /* ASPIRE_FULL_* */
  int32_t subset_cache_size;
  int32_t table_width;
  int32_t min_draft_pages;   /* < 0: None */
  float draft_percent;       /* < 0: None (evaluated in fp32, as the device does) */
  int32_t valid_floor_l;
  int32_t pages_per_slot;    /* > 0: static arange index layout for 'effective_full' */
} aspire_host_plan_config;

/* Mirror state, caller-owned: max_batch entries each. */
typedef struct aspire_host_plan_state {
  int64_t* draft_num_pages;
  uint8_t* prev_verify;
} aspire_host_plan_state;

/* Pre-step row state from the scheduler (build_step's keyword arguments). */
typedef struct aspire_host_plan_inputs {
  int32_t batch;               /* rows this step (<= max_batch) */
  const uint8_t* verify;       /* [batch] */
  const uint8_t* finished;     /* [batch] */
  const int64_t* draft_counts; /* [batch] */
  const int64_t* seq_lens;     /* [batch] */
  int64_t total_tokens;
  int64_t bucket_tokens;
} aspire_host_plan_inputs;

/* Rendered arrays. qo_indptr / kv_indptr / full_kv_indptr hold max_batch + 2
 * entries and kv_len / full_kv_len max_batch + 1 (padding rows filled as the
 * reference does); per-row arrays hold batch entries; refresh_rows / spill_rows
 * (optional) hold up to max_batch; sample_indices / position_indices
 * (optional) up to token_capacity. */
typedef struct aspire_host_plan_outputs {
  int32_t* qo_indptr;
  int32_t* kv_indptr;
  int32_t* kv_len;
  int32_t* full_kv_indptr;     /* 'effective_full' only */
  int32_t* full_kv_len;        /* 'effective_full' only */
  int64_t* dec;
  int64_t* verify_num_pages;
  int64_t* effective_num_pages;
  int64_t* last_page_len;
  int64_t* input_pos;
  int64_t* sample_indices;
  int64_t* position_indices;
  int64_t token_capacity;
  int64_t* refresh_rows;
  int64_t* spill_rows;
  int32_t n_refresh;           /* written */
  int32_t n_spill;             /* written */
} aspire_host_plan_outputs;

/* reset_all (slot_ids == NULL: rows 0..n-1, every verify flag cleared) or
 * reset_slots (host_plan.py:138-151): seeds draft_num_pages from each row's
 * page count. */
int aspire_host_plan_reset(const aspire_host_plan_config* cfg, int64_t* draft_num_pages,
                           uint8_t* prev_verify, const int64_t* slot_ids,
                           const int64_t* seq_lens, int32_t n);

/* build_step (host_plan.py:155-306): advances the state by one step and
 * renders the arrays. ASPIRE_ERR_INVALID (state left as the reference leaves
 * it) when the token total disagrees with the scheduler's. */
int aspire_host_plan_step(const aspire_host_plan_config* cfg, aspire_host_plan_state* state,
                          const aspire_host_plan_inputs* in, aspire_host_plan_outputs* out);

/* ------------------------------------------------------ qk norm + rope + append
 * One launch for the per-layer q / k preparation of the mixed forward
 * (aspire/models/sparse_draft_transformer.py:149-171): optional q / k RMSNorm
 * (transformer.py:505-516) with the rotary permute (transformer.py:360-364),
 * interleaved RoPE (the mylib::rope op, mixed_transformer.py:159-198, i.e.
 * FlashInfer apply_rope_inplace / apply_llama31_rope_inplace with
 * interleave=True), and optionally the paged append of the rotated k and of v
 * (mylib::update_kv_padded, kv_ops.py:127-187). q is rewritten in place; k
 * too when write_k. Without norm weights and without a cache this is exactly
 * mylib::rope. bf16, head_dim 128. */
typedef struct aspire_rope_args {
  void* q;                      /* [T, Hq, 128] bf16, in place */
  int64_t q_stride_t, q_stride_h;
  int32_t num_qo_heads;
  void* k;                      /* [T, Hkv, 128] bf16 */
  int64_t k_stride_t, k_stride_h;
  int32_t num_kv_heads;
  const void* v;                /* [T, Hkv, 128] bf16 (append only; may be NULL) */
  int64_t v_stride_t, v_stride_h;
  int32_t total_tokens;
  int32_t head_dim;
  const void* q_norm_weight;    /* [128] bf16, NULL: no norm (and no permute) */
  const void* k_norm_weight;
  float norm_eps;
  int32_t permute;              /* permute to the interleaved layout after the norm */
  float rope_theta, rope_scale;
  int32_t llama31;              /* Llama 3.1 frequency smoothing */
  float low_freq_factor, high_freq_factor, old_context_len;
  const int32_t* indptr;        /* rows of tokens: [num_rows + 1] (the append indptr) */
  const int32_t* offsets;       /* [num_rows] position of each row's first token */
  int32_t num_rows;
  void* kv_cache;               /* NULL: no append */
  int64_t cache_stride_p, cache_stride_kv, cache_stride_t, cache_stride_h;
  int32_t page_size;
  const int32_t* kv_page_indices;
  const int32_t* kv_page_indptr;
  const int32_t* kv_last_page_len;
  int32_t num_seq;              /* rows of the append (a prefix of the rope rows) */
  int32_t write_k;              /* also rewrite k in place */
} aspire_rope_args;

int aspire_qk_norm_rope_append(const aspire_rope_args* args, void* stream);

/* The head_dim / 2 fp32 rotary frequencies the kernel uses (host only):
 * theta^(-2i/head_dim) / rope_scale, or the Llama 3.1 smoothing. */
int aspire_rope_frequencies(int32_t head_dim, float rope_theta, float rope_scale, int32_t llama31,
                            float low_freq_factor, float high_freq_factor, float old_context_len,
                            float* out);

/* ------------------------------------------------ decode-step row operations
 * The per-token steps a decode step runs between the GEMMs, used by the full
 * decode step. One workgroup per row, no scratch memory.
 *
 * aspire_add_rms_norm: with delta, x[r] += delta[r] (bf16) first
 * (h = x + attn_out, aspire/models/sparse_draft_transformer.py:232-238); then
 * out[r] = RMSNorm(x[r]) * weight as transformer.py:505-516 computes it in
 * bf16. dim % 8 == 0, dim <= 8192, 16-byte aligned rows; out must not overlap
 * x or delta. */
int aspire_add_rms_norm(void* x, int64_t x_stride, const void* delta, int64_t delta_stride,
                        const void* weight, void* out, int64_t out_stride, int32_t rows, int32_t dim,
                        float eps, void* stream);

/* SwiGLU's elementwise step, FeedForward.forward (transformer.py:498-499):
 * out[t, i] = bf16(bf16(silu(gate_up[t, i])) * gate_up[t, inter + i]), the
 * gate (w1) and up (w3) projections side by side in one row. */
int aspire_silu_mul(const void* gate_up, int64_t gate_up_stride, void* out, int64_t out_stride,
                    int32_t rows, int32_t inter, void* stream);

/* Greedy token pick (the top_k == 0 branch of TransformerSparseDraft.unified_forward,
 * sparse_draft_transformer.py:276-286): ids[r] = the first index of the
 * maximum of the bf16 row logits[r, :vocab] (torch.argmax). */
int aspire_argmax_rows(const void* logits, int64_t stride, int32_t rows, int32_t vocab, int64_t* ids,
                       void* stream);

/* ------------------------------------------------------ (f3) prefill
 * Chunked-prefill paged attention: replaces the attention FlashInfer's
 * BatchPrefillWithPagedKVCacheWrapper runs for prompt chunks
 * (aspire/models/sparse_draft_runner.py:199-209; the chunk loop of encode_slots,
 * aspire/backends/base.py:1559-1674). Row b's queries [qo_indptr[b], qo_indptr[b+1])
 * attend the first kv_len_b tokens of its pages kv_indices[kv_indptr[b] ..
 * kv_indptr[b+1]) (kv_len_b = max(pages - 1, 0) * 16 + kv_last_page_len[b]), bottom-right
 * causal when causal != 0; out and the base-2 lse as aspire_attention_run writes them.
 * Work is split into query blocks of block_tokens tokens per (row, kv head):
 * block_indptr[b] = sum over rows c < b of ceil(q_len_c / block_tokens), total_blocks =
 * block_indptr[num_rows]; all index arrays are device arrays. No workspace. */
typedef struct aspire_prefill_args {
  const void* q; int64_t q_stride_t; int64_t q_stride_h;
  const void* kv_cache; int64_t cache_stride_p; int64_t cache_stride_kv;
  int64_t cache_stride_t; int64_t cache_stride_h;
  const int32_t* kv_indices; const int32_t* kv_indptr; const int32_t* kv_last_page_len;
  const int32_t* qo_indptr; const int32_t* block_indptr;
  int32_t num_rows; int32_t total_blocks; int32_t block_tokens;
  void* out; int64_t out_stride_t; int64_t out_stride_h;
  float* lse;                      /* [T, H_q] or NULL */
  int32_t num_qo_heads; int32_t num_kv_heads; int32_t head_dim; int32_t page_size;
  float sm_scale; int32_t causal;
} aspire_prefill_args;

/* Tokens per query block for a head configuration: the workgroup's query rows (128 in
 * the default build: 4 waves x 32) / (num_qo_heads / num_kv_heads), or 0 when the GQA
 * group does not divide a wave's query rows (32 in the default build). Host only. */
int aspire_prefill_block_tokens(int32_t num_qo_heads, int32_t num_kv_heads);

int aspire_prefill_run(const aspire_prefill_args* args, void* stream);

/* ------------------------------------------------------ (f4) sampling
 * Token sampling and speculative verification. One workgroup per row or request; the
 * uniforms of every draw are explicit device inputs (the Python layer draws them with
 * torch's generator, so a run is reproducible and graph-capturable). */

/* local_topk_candidates (aspire/engine/sampling.py:6-29) on one rank: the top_k
 * (1..1024) largest bf16 logits of each row, descending (ties: lower id first), into
 * values [rows, top_k] bf16 and ids [rows, top_k] (+ vocab_start); rows narrower than
 * top_k are padded with -inf / id 0 as the reference pads a narrow vocabulary shard. */
int aspire_topk_candidates(const void* logits, int64_t stride, int32_t rows, int32_t vocab, int32_t top_k,
                           int64_t vocab_start, void* values, int64_t* ids, void* stream);

/* LogitsPipe([Temperature(), Softmax(), TopP()]) behind mylib::logit_process
 * (aspire/models/sparse_draft_runner.py:527-554): per row of width (<= 4096) values
 * (values_dtype 0 bf16, 1 fp32), probs = softmax(values / temperature) in fp32 (no
 * temperature when <= 0), then top-p renormalisation when 0 < top_p < 1: the smallest
 * set of the largest probabilities whose sum reaches top_p (every probability equal to
 * its smallest member included) is kept and divided by its sum, the rest set to 0. */
int aspire_logits_pipe(const void* values, int32_t values_dtype, int64_t stride, int32_t rows, int32_t width,
                       float temperature, float top_p, float* probs, int64_t out_stride, void* stream);

/* FlashInfer sampling_from_probs (called at aspire/engine/runtime.py:709,748): out[r] =
 * the first index whose inclusive prefix sum of probs[r] exceeds uniforms[r] * sum
 * (uniforms in [0, 1)); the last positive index if rounding leaves none. */
int aspire_sampling_from_probs(const float* probs, int64_t stride, int32_t rows, int32_t vocab,
                               const float* uniforms, int32_t* out, void* stream);

/* FlashInfer chain_speculative_sampling (called at aspire/engine/sampling.py:84-86):
 * draft_probs [rows, num_spec, vocab], draft_token_ids [rows, num_spec], target_probs
 * [rows, num_spec + 1, vocab], uniforms [rows, num_spec + 1], all contiguous. Draft i
 * is accepted while uniforms[r, i] * q_i(x_i) < p_i(x_i); at the first rejection j a
 * token is drawn (with uniforms[r, num_spec]) from max(0, p_j - q_j) normalised (from
 * p_j if that is all zero), after a full acceptance from p_{num_spec}.
 * output_token_ids [rows, num_spec + 1]: accepted drafts, the drawn token, then -1;
 * emitted_num[r] = j; accepted_num[r] (optional) = the positions that pass the test on
 * their own, chain or not. */
int aspire_chain_speculative_sampling(const float* draft_probs, const int32_t* draft_token_ids,
                                      const float* target_probs, int32_t rows, int32_t num_spec, int32_t vocab,
                                      const float* uniforms, int32_t* output_token_ids, int32_t* accepted_num,
                                      int32_t* emitted_num, void* stream);

/* verify_topk_speculation (aspire/engine/sampling.py:46-98) in one launch: the chain
 * rule over each position's local vocabulary of the target's top_k candidates plus one
 * entry for tokens outside them. draft_probs / draft_ids [requests, max_draft, top_k],
 * draft_tokens [requests, max_draft] int32, draft_counts [requests] int32, target_probs /
 * target_ids [requests, max_draft + 1, top_k], uniforms [requests, max_draft + 1];
 * output [requests, max_draft + 1] int64 (vocabulary ids, -1 past the emitted tokens),
 * emitted [requests] int32 (accepted drafts). max_draft <= 64, top_k <= 1024. */
int aspire_verify_topk_speculation(const float* draft_probs, const int64_t* draft_ids, const int32_t* draft_tokens,
                                   const int32_t* draft_counts, const float* target_probs, const int64_t* target_ids,
                                   const float* uniforms, int32_t requests, int32_t max_draft, int32_t top_k,
                                   int64_t* output, int32_t* emitted, void* stream);

/* ----------------------------------------------------------------- (d) -- */
/* HBM calibration (no reference counterpart: the measurement row asks for the
 * bandwidth achieved on the box, measured with a streaming kernel, beside the
 * published peak). mode 0 reads `bytes` of src once as 1 KiB rows, one 128-bit
 * non-temporal buffer load per lane (the attention kernel's staged K/V access),
 * in_flight rows per wave; dst is a sink of at least workgroups * 1024 bytes
 * that a store reaches only under a data-dependent condition. mode 1 copies
 * `bytes` of src to dst (dst_bytes >= bytes) with in_flight 16-byte chunks per
 * thread. in_flight is 1, 2, 4, 8 or 16; bytes is a multiple of 1024; src and
 * dst are 16-byte aligned; `workgroups` 256-thread workgroups stride over the
 * buffer. Time it with events on `stream`: GB/s = bytes (x2 for the copy) /
 * time; the best grid depends on in_flight, so sweep both. */
int aspire_bandwidth_probe(int32_t mode, const void* src, int64_t bytes, void* dst, int64_t dst_bytes,
                           int32_t workgroups, int32_t in_flight, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ASPIRE_HIP_H */
