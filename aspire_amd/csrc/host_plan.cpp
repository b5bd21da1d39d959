// (a7) Host mirror of the per-step plan arrays, native.
//
// The reference keeps the lengths that drive the attention plan in NumPy on
// the host and renders qo_indptr / kv_indptr / kv_len (and the dump wrapper's
// full-context arrays) every step without a device readback
// (aspire/backends/host_plan.py:154-306). This is the same bookkeeping as one
// C++ pass over the rows: integer arithmetic only, plus the one fp32 ceil of
// the draft-percent rule, evaluated in fp32 exactly as the device does.
#include <cmath>
#include <cstdint>
#include <cstring>

#include "common.h"

namespace aspire {
namespace {

inline int64_t num_pages_of(int64_t len, int64_t page) { return (len + page - 1) / page; }

inline int64_t last_page_len_of(int64_t len, int64_t page) { return len > 0 ? (len - 1) % page + 1 : 0; }

// PageSelector.compute_valid_counts (page_selector.py:52-62) with the floor
// the host mirror passes (host_plan.py:92-118); the sink+recent family caps at
// the subset size (host_plan.py:96-99).
int64_t valid_count(const aspire_host_plan_config& c, int64_t np, bool seeding) {
  if (!seeding && c.draft_kind == ASPIRE_DRAFT_SINK_RECENT) return np < c.subset_cache_size ? np : c.subset_cache_size;
  const int64_t hi = np < c.subset_cache_size ? np : c.subset_cache_size;
  if (c.draft_percent < 0.f) {
    if (c.min_draft_pages >= 0) return np < c.min_draft_pages ? np : c.min_draft_pages;
    return hi;
  }
  const int64_t floor_pages = c.min_draft_pages >= 0 ? c.min_draft_pages : c.valid_floor_l;
  const int64_t lo = np < floor_pages ? np : floor_pages;
  const float t = std::ceil(static_cast<float>(np) * c.draft_percent / 100.0f);
  const int64_t target = static_cast<int64_t>(t);
  const int64_t a = target > lo ? target : lo;  // numpy clip = min(max(x, lo), hi)
  return a < hi ? a : hi;
}

}  // namespace
}  // namespace aspire

extern "C" int aspire_host_plan_reset(const aspire_host_plan_config* cfg, int64_t* draft_num_pages,
                                      uint8_t* prev_verify, const int64_t* slot_ids, const int64_t* seq_lens,
                                      int32_t n) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(cfg && draft_num_pages && prev_verify && (n == 0 || seq_lens), "null argument");
  ASPIRE_CHECK_ARG(cfg->page_size > 0 && cfg->max_batch >= 0, "bad config");
  ASPIRE_CHECK_ARG(n >= 0 && (slot_ids != nullptr || n <= cfg->max_batch), "too many rows");
  for (int32_t i = 0; i < n; ++i) {
    const int64_t slot = slot_ids ? slot_ids[i] : i;
    ASPIRE_CHECK_ARG(slot >= 0 && slot < cfg->max_batch, "slot id out of range");
    draft_num_pages[slot] = valid_count(*cfg, num_pages_of(seq_lens[i], cfg->page_size), true);
    prev_verify[slot] = 0;
  }
  // reset_all (no slot ids) also clears every verify flag (host_plan.py:140-144)
  if (!slot_ids) std::memset(prev_verify, 0, size_t(cfg->max_batch));
  return ASPIRE_OK;
}

extern "C" int aspire_host_plan_step(const aspire_host_plan_config* cfg, aspire_host_plan_state* st,
                                     const aspire_host_plan_inputs* in, aspire_host_plan_outputs* out) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(cfg && st && in && out, "null argument");
  const aspire_host_plan_config& c = *cfg;
  const int32_t mb = in->batch;
  const int64_t P = c.page_size;
  ASPIRE_CHECK_ARG(P > 0, "page_size must be positive");
  ASPIRE_CHECK_ARG(mb >= 0 && mb <= c.max_batch, "batch exceeds max_batch");
  ASPIRE_CHECK_ARG(st->draft_num_pages && st->prev_verify, "null state");
  ASPIRE_CHECK_ARG(mb == 0 || (in->verify && in->finished && in->draft_counts && in->seq_lens), "null input");
  ASPIRE_CHECK_ARG(out->qo_indptr && out->kv_indptr && out->kv_len && out->dec && out->verify_num_pages &&
                       out->effective_num_pages && out->last_page_len && out->input_pos,
                   "null output");
  ASPIRE_CHECK_ARG(c.draft_kind >= 0 && c.draft_kind <= 2 && c.full_kind >= 0 && c.full_kind <= 2,
                   "unknown draft_kind / full_kind");
  const int32_t nq = c.max_batch + 2;  // qo / kv indptr length (the padding row included)
  const int32_t nl = c.max_batch + 1;  // kv_len length

  // Per-row lengths at plan time (host_plan.py:181-199): decode tokens, the
  // target cache length after the append, the draft cache length, and the
  // length each row's attention sees.
  for (int32_t b = 0; b < mb; ++b) {
    const bool verify = in->verify[b] != 0;
    const bool active = in->finished[b] == 0;
    const int64_t d = in->draft_counts[b];
    const int64_t dec = verify ? d + 1 : (active ? 1 : 0);
    const int64_t cachelens = in->seq_lens[b] + d - (verify ? d : 0) + dec;
    const int64_t draft_cachelens = in->seq_lens[b] + d + (verify ? 0 : 1);
    const int64_t eff = verify ? cachelens : draft_cachelens;
    out->dec[b] = dec;
    out->verify_num_pages[b] = num_pages_of(cachelens, P);
    out->effective_num_pages[b] = num_pages_of(eff, P);
    out->last_page_len[b] = last_page_len_of(eff, P);
    out->input_pos[b] = verify ? cachelens - dec : draft_cachelens - 1;
  }

  // Draft-table page counts per refresh family (host_plan.py:201-231).
  int32_t n_refresh = 0, n_spill = 0;
  if (c.draft_kind != ASPIRE_DRAFT_GATED) {
    for (int32_t b = 0; b < mb; ++b) st->draft_num_pages[b] = valid_count(c, out->verify_num_pages[b], false);
  } else {
    for (int32_t b = 0; b < c.max_batch; ++b) {
      if (!st->prev_verify[b]) continue;
      if (b >= mb) {
        set_error("aspire_host_plan_step: row %d verified last step but the batch is now %d rows", b, mb);
        return ASPIRE_ERR_INVALID;
      }
      st->draft_num_pages[b] = valid_count(c, out->verify_num_pages[b], false);
      if (out->refresh_rows) out->refresh_rows[n_refresh] = b;
      ++n_refresh;
    }
    // A draft token opening a new page is appended to every table that was
    // not refreshed this step, while the table has room.
    for (int32_t b = 0; b < mb; ++b) {
      const bool verify = in->verify[b] != 0;
      const int64_t draft_cachelens = in->seq_lens[b] + in->draft_counts[b] + (verify ? 0 : 1);
      const bool crossed = !verify && out->dec[b] > 0 && (draft_cachelens - 1) % P == 0;
      if (!crossed || st->prev_verify[b] || st->draft_num_pages[b] >= c.table_width) continue;
      st->draft_num_pages[b] += 1;
      if (out->spill_rows) out->spill_rows[n_spill] = b;
      ++n_spill;
    }
  }
  out->n_refresh = n_refresh;
  out->n_spill = n_spill;

  // Plan arrays (host_plan.py:233-251): padding rows take the bucket / last
  // indptr value and a zero length.
  int64_t q = 0, k = 0;
  out->qo_indptr[0] = 0;
  out->kv_indptr[0] = 0;
  for (int32_t b = 0; b < mb; ++b) {
    const bool draft = in->verify[b] == 0;
    const int64_t pages = draft ? st->draft_num_pages[b] : out->verify_num_pages[b];
    q += out->dec[b];
    k += pages;
    out->qo_indptr[b + 1] = static_cast<int32_t>(q);
    out->kv_indptr[b + 1] = static_cast<int32_t>(k);
    out->kv_len[b] = static_cast<int32_t>((pages > 1 ? pages - 1 : 0) * P + out->last_page_len[b]);
  }
  for (int32_t i = mb + 1; i < nq; ++i) {
    out->qo_indptr[i] = static_cast<int32_t>(in->bucket_tokens);
    out->kv_indptr[i] = static_cast<int32_t>(k);
  }
  for (int32_t i = mb; i < nl; ++i) out->kv_len[i] = 0;
  if (q != in->total_tokens) {
    set_error("host plan mirror diverged: token total %lld != scheduler total %lld", (long long)q,
              (long long)in->total_tokens);
    return ASPIRE_ERR_INVALID;
  }

  // Token-level metadata (host_plan.py:255-262): per token, its row and its
  // index within the row.
  if (out->sample_indices || out->position_indices) {
    ASPIRE_CHECK_ARG(out->token_capacity >= q, "token arrays smaller than the step's tokens");
    int64_t t = 0;
    for (int32_t b = 0; b < mb; ++b)
      for (int64_t j = 0; j < out->dec[b]; ++j, ++t) {
        if (out->sample_indices) out->sample_indices[t] = b;
        if (out->position_indices) out->position_indices[t] = j;
      }
  }

  // Dump wrapper arrays over the effective (full) context (host_plan.py:280-303).
  if (c.full_kind == ASPIRE_FULL_EFFECTIVE) {
    ASPIRE_CHECK_ARG(out->full_kv_indptr && out->full_kv_len, "null full-context output");
    int64_t f = 0;
    out->full_kv_indptr[0] = 0;
    for (int32_t b = 0; b < mb; ++b) {
      const int64_t ep = out->effective_num_pages[b];
      f = c.pages_per_slot > 0 ? int64_t(b + 1) * c.pages_per_slot : f + ep;
      out->full_kv_indptr[b + 1] = static_cast<int32_t>(f);
      out->full_kv_len[b] = static_cast<int32_t>((ep > 1 ? ep - 1 : 0) * P + out->last_page_len[b]);
    }
    for (int32_t i = mb + 1; i < nq; ++i) out->full_kv_indptr[i] = static_cast<int32_t>(f);
    for (int32_t i = mb; i < nl; ++i) out->full_kv_len[i] = 0;
  }

  for (int32_t b = 0; b < mb; ++b) st->prev_verify[b] = in->verify[b] != 0;
  return ASPIRE_OK;
}
