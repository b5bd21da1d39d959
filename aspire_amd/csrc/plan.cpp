// (a7) Host planner for the mixed attention kernel.
//
// The attention kernel is persistent: each row-tile class (<=16, <=32, <=48
// query rows per (row, kv head) segment) runs a fixed grid of `num_waves`
// waves, and wave w processes the work items items[indptr[w] .. indptr[w+1]).
// The plan lives at fixed offsets of the device int workspace, so a run()
// captured in a HIP graph replays correctly after any later plan.
//
// Decomposition (stream-K): the segments of a class are laid end to end as a
// sequence of pages; slot j takes the contiguous range [j*T/S, (j+1)*T/S). A
// segment cut by a range boundary is split into pieces that write fp32
// partial (o, lse) rows; a merge item per split (row, kv head) combines them.
// This balances HBM traffic per wave exactly and creates at most two split
// pieces per slot, unlike a fixed chunk length. When every row's kv heads
// attend the same number of tokens, a slot is a group of num_kv_heads
// consecutive waves and a segment is a whole row: wave g of the group streams
// kv head g over the same page range at the same time. Rows whose heads share
// one list then stage the pages through LDS; rows with a list per head (the
// key-mean selection) read their own head's rows directly (their items carry
// kItemDirect). Otherwise a slot is one wave and a segment one (row, kv head).
#include <algorithm>
#include <cstring>
#include <vector>

#include "common.h"

namespace aspire {
namespace {

constexpr int kMinPagesPerWave = 8;
// Stream-K cost units of one page-head, in quarters: an item staged for the workgroup's heads
// (32 for 2- and 3-tile items, 33 for 1-tile items) and an item reading its own head's list
// (direct: 48). Per-wave finish times of config-4 launches (fitted per class) showed 1-tile
// pages about 3-10% slower than 3-tile pages in a joint launch, whose tiles run on two waves
// of the head; sweeping the 1-tile weight (32-35) gave 33 at every draft fraction, and the
// 3-tile weight (28-40) 32. With the slack softmax (3-tile items 5% faster) 33/32/32 stayed
// best against 3-tile 30 or 34, 2- and 3-tile 31 and 1-tile 34 on configs 1 and 4. The
// direct weight comes from a sweep of 40-52 on configs 3 and 4.
#ifndef ASPIRE_DIRECT_PAGE_COST
#define ASPIRE_DIRECT_PAGE_COST 48
#endif
#ifndef ASPIRE_C1_PAGE_COST
#define ASPIRE_C1_PAGE_COST 33
#endif
#ifndef ASPIRE_C2_PAGE_COST
#define ASPIRE_C2_PAGE_COST 32
#endif
#ifndef ASPIRE_C3_PAGE_COST
#define ASPIRE_C3_PAGE_COST 32
#endif
constexpr int64_t kDirectPageCost = ASPIRE_DIRECT_PAGE_COST;
constexpr int64_t kSharedPageCost[3] = {ASPIRE_C1_PAGE_COST, ASPIRE_C2_PAGE_COST, ASPIRE_C3_PAGE_COST};

struct Segment {
  int32_t q_start, q_len, kv_len, list_base, npages, bg, rows;
  int32_t seg0;    // segment index of kv head (bg & 255), for per-head list starts
  int32_t direct;  // kItemDirect for rows whose heads read different lists
};

struct Piece {
  int64_t slot, pb, pe;  // slot and the segment's pages [pb, pe) it streams
};

struct Scratch {
  std::vector<Segment> segs[3];
  std::vector<Piece> pieces;
  std::vector<std::pair<int32_t, WorkItem>> citems[3];
  std::vector<int32_t> start, pages;
  std::vector<std::pair<int32_t, WorkItem>> items;
  std::vector<MergeItem> merges;
  std::vector<int32_t> counts;
};

int cached_cu_count() {
  static thread_local int dev_cached = -1;
  static thread_local int cus = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (dev != dev_cached) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return -1;
    dev_cached = dev;
  }
  return cus;
}

}  // namespace
}  // namespace aspire

extern "C" int aspire_plan_layout_init(int32_t num_cus, int32_t waves_per_cu, int64_t int_ws_bytes,
                                       int64_t float_ws_bytes, int32_t head_dim,
                                       aspire_plan_layout* out) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(out != nullptr, "null layout");
  ASPIRE_CHECK_ARG(head_dim == kHeadDim, "head_dim must be 128");
  if (num_cus <= 0) {
    num_cus = cached_cu_count();
    if (num_cus <= 0) return fail(ASPIRE_ERR_HIP, "aspire_plan_layout_init: cannot query CU count");
  }
  // One wave per SIMD: measured best on MI355X for every row-tile mix (with
  // more waves per CU they contend for HBM and the long wide-row workloads
  // lose up to 10%).
  if (waves_per_cu <= 0) waves_per_cu = 4;
  int32_t waves = num_cus * waves_per_cu;
  waves = (waves + kAttnWavesPerBlock - 1) / kAttnWavesPerBlock * kAttnWavesPerBlock;
  aspire_plan_layout L;
  L.num_waves = waves;
  L.max_items = 4 * waves + 8192;
  L.max_merge = 8 * waves + 16384;  // a split segment may be cut into up to 4 row ranges
  L.head_dim = head_dim;
  PlanOffsets o = plan_offsets(L);
  while (o.total * 4 > int_ws_bytes && L.max_items > waves + 64) {
    L.max_items = (L.max_items + waves) / 2;
    L.max_merge = (L.max_merge + waves) / 2;
    o = plan_offsets(L);
  }
  if (o.total * 4 > int_ws_bytes)
    return fail(ASPIRE_ERR_CAPACITY, "aspire_plan_layout_init: int workspace too small");
  L.int_ws_bytes = o.total * 4;
  L.partial_rows_cap = float_ws_bytes / (int64_t(head_dim + 1) * 4);
  L.float_ws_bytes = L.partial_rows_cap * (head_dim + 1) * 4;
  if (L.partial_rows_cap <= 0)
    return fail(ASPIRE_ERR_CAPACITY, "aspire_plan_layout_init: float workspace too small");
  *out = L;
  return ASPIRE_OK;
}

namespace aspire {
namespace {

Scratch& scratch() {
  static thread_local Scratch sc;
  return sc;
}

// Segments: per_head ? (row b, kv head g) at index b * num_kv_heads + g : row b, each with
// its list start (kv_indices offset), list pages and kv length.
int plan_core(const aspire_plan_layout* layout, const int32_t* qo_indptr, const int32_t* seg_start,
              const int32_t* seg_pages, const int32_t* seg_kv_len, int32_t batch, bool per_head,
              int32_t num_qo_heads, int32_t num_kv_heads, int32_t causal, void* host_buf, aspire_plan_info* info) {
  const int group = num_qo_heads / num_kv_heads;
  const aspire_plan_layout& L = *layout;
  const PlanOffsets off = plan_offsets(L);
  const int W = L.num_waves;

  Scratch& sc = scratch();
  for (auto& s : sc.segs) s.clear();
  sc.items.clear();
  sc.merges.clear();

  // Head-aligned planning: the stream-K unit is a whole page (all kv heads)
  // and a slot is a group of num_kv_heads consecutive waves, wave g of the
  // group streaming kv head g. Every head of a page is then read at about the
  // same time by waves dispatched together, which keeps a shared page's 64 KB
  // of DRAM traffic together. It needs every row's heads to attend the same
  // number of tokens; otherwise each (row, kv head) is a segment of its own
  // with single-wave slots.
  bool uniform = true;
  if (per_head)
    for (int b = 0; b < batch && uniform; ++b)
      for (int g = 1; g < num_kv_heads; ++g)
        if (seg_kv_len[b * num_kv_heads + g] != seg_kv_len[b * num_kv_heads]) {
          uniform = false;
          break;
        }
  const bool aligned = uniform && W % num_kv_heads == 0;
  const int hpu = aligned ? num_kv_heads : 1;
  int max_rows = 0;
  int num_segments = 0;
  int split_rows = 0;
  // A row longer than one 3-tile item (q_len * group > 48, e.g. a prefill
  // chunk) is cut into query tiles of tile_q tokens. Each tile is planned as a
  // row of its own whose keys end at the tile's last token: with
  // kv_len' = kv_len - q_len + t0 + q_len', the kernel's causal limit
  // kv_len' - q_len' + j equals the row's limit kv_len - q_len + (t0 + j), and
  // the tile streams only the pages below it. Without the causal mask every
  // tile sees the whole row.
  const int tile_q = std::max(1, 16 * kMaxRowTiles / group);
  for (int b = 0; b < batch; ++b) {
    const int q_len = qo_indptr[b + 1] - qo_indptr[b];
    if (q_len <= 0) continue;
    if (q_len * group > 16 * kMaxRowTiles) ++split_rows;
    for (int t0 = 0; t0 < q_len; t0 += tile_q) {
      const int tq = std::min(tile_q, q_len - t0);
      const int rows = tq * group;
      max_rows = std::max(max_rows, rows);
      const int cls = (rows - 1) / 16;
      for (int g = 0; g < num_kv_heads; g += hpu) {
        const int s = per_head ? b * num_kv_heads + g : b;
        const int kvl_row = seg_kv_len[s];
        if (kvl_row < 0) {
          set_error("aspire_plan_build: segment %d has negative length", s);
          return ASPIRE_ERR_INVALID;
        }
        const int kvl = causal && tq < q_len ? std::max(kvl_row - q_len + t0 + tq, 0) : kvl_row;
        const int np = (kvl + kPage - 1) / kPage;
        // every head the segment covers must hold the pages in its list
        bool shared = true;
        for (int gg = 0; gg < (per_head ? hpu : 1); ++gg) {
          const int sg = s + gg;
          if (seg_pages[sg] < 0 || np > seg_pages[sg]) {
            set_error("aspire_plan_build: segment %d needs %d pages but its list holds %d", sg, np,
                      seg_pages[sg]);
            return ASPIRE_ERR_INVALID;
          }
          if (seg_start[sg] != seg_start[s]) shared = false;
        }
        const int32_t direct = (hpu > 1 && !shared) ? kItemDirect : 0;
        sc.segs[cls].push_back(Segment{qo_indptr[b] + t0, tq, kvl, seg_start[s], np, (b << 8) | g, rows,
                                       per_head ? s : -1, direct});
        num_segments += hpu;
      }
    }
  }

  int32_t* buf = static_cast<int32_t*>(host_buf);
  int64_t partial_rows = 0;
  int64_t total_pages = 0;
  int num_items[3] = {0, 0, 0};
  // One kernel launch runs every class: each wave takes its class-1 items, then its class-2,
  // then its class-3 items. The classes are planned as one stream-K sequence in cost units
  // (class by class, segments in row order), so a slot streams one contiguous range of that
  // sequence and a long row is split about as often as its share of the whole launch needs,
  // not once per slot of its class.
  auto page_cost = [&](int c, bool direct) -> int64_t { return direct ? kDirectPageCost : kSharedPageCost[c]; };
  int64_t T = 0, T_pages = 0;
  for (int c = 0; c < 3; ++c)
    for (const auto& s : sc.segs[c]) {
      T += int64_t(s.npages) * page_cost(c, s.direct != 0);
      T_pages += s.npages;
    }
  total_pages = T_pages * hpu;
  const int64_t slots = W / hpu;
  // Slots actually used: enough that each streams >= kMinPagesPerWave pages.
  int64_t s_eff = std::max<int64_t>(1, std::min<int64_t>(slots, T_pages / kMinPagesPerWave));
  // Shrink until the split pieces' partial rows fit the float workspace.
  for (;;) {
    for (auto& v : sc.citems) v.clear();
    sc.merges.clear();
    int64_t pr = 0;
    int64_t seg_off = 0;
    int zero_rr = 0;
    for (int c = 0; c < 3; ++c) {
      auto& out = sc.citems[c];
      for (const auto& s : sc.segs[c]) {
        if (s.npages == 0) {
          const int64_t slot = zero_rr++ % s_eff;
          for (int gg = 0; gg < hpu; ++gg) {
            const int32_t base = s.seg0 >= 0 ? seg_start[s.seg0 + gg] : s.list_base;
            WorkItem it{s.q_start, s.q_len | s.direct, s.kv_len, base, 0, 0, s.bg + gg, -1};
            out.emplace_back(static_cast<int32_t>(slot * hpu + gg), it);
          }
          continue;
        }
        // Page p of the segment sits at cost position a + p * wt and belongs to the slot
        // holding that position: slot j holds positions [floor(j*T/s_eff), floor((j+1)*T/s_eff)).
        const int64_t wt = page_cost(c, s.direct != 0);
        const int64_t a = seg_off, e = seg_off + int64_t(s.npages) * wt;
        auto slot_of = [&](int64_t x) {  // largest j with floor(j*T/s_eff) <= x
          int64_t j = (x * s_eff) / T;
          while (j > 0 && (j * T) / s_eff > x) --j;
          while (j + 1 < s_eff && ((j + 1) * T) / s_eff <= x) ++j;
          return j;
        };
        auto first_page_at = [&](int64_t x) {  // first page whose position is >= x
          return x <= a ? int64_t(0) : std::min<int64_t>(s.npages, (x - a + wt - 1) / wt);
        };
        const int64_t j_lo = slot_of(a), j_hi = slot_of(e - wt);
        sc.pieces.clear();
        for (int64_t j = j_lo; j <= j_hi; ++j) {
          const int64_t pb = first_page_at((j * T) / s_eff);
          const int64_t pe = j == j_hi ? s.npages : first_page_at(((j + 1) * T) / s_eff);
          if (pe > pb) sc.pieces.push_back({j, pb, pe});
        }
        const int pieces = static_cast<int>(sc.pieces.size());
        // partial rows: head gg's pieces are contiguous, first[gg] + k * rows
        const int64_t first = pr;
        if (pieces > 1) pr += int64_t(hpu) * pieces * s.rows;
        for (int k = 0; k < pieces; ++k) {
          const Piece& pc = sc.pieces[k];
          for (int gg = 0; gg < hpu; ++gg) {
            const int64_t prow = pieces > 1 ? first + (int64_t(gg) * pieces + k) * s.rows : -1;
            const int32_t base = s.seg0 >= 0 ? seg_start[s.seg0 + gg] : s.list_base;
            WorkItem it{s.q_start, s.q_len | s.direct, s.kv_len, base, static_cast<int32_t>(pc.pb),
                        static_cast<int32_t>(pc.pe), s.bg + gg, static_cast<int32_t>(prow)};
            out.emplace_back(static_cast<int32_t>(pc.slot * hpu + gg), it);
          }
        }
        if (pieces > 1) {
          // row ranges small enough for the merge kernel's piece groups
          const int span = pieces > 2 * kMergeChunk ? kMergeRows / 4
                           : pieces > kMergeChunk   ? kMergeRows / 2
                                                    : kMergeRows;
          for (int gg = 0; gg < hpu; ++gg)
            for (int r0 = 0; r0 < s.rows; r0 += span)
              sc.merges.push_back(MergeItem{s.q_start, s.q_len, s.bg + gg,
                                            static_cast<int32_t>(first + int64_t(gg) * pieces * s.rows),
                                            pieces, s.rows, r0, std::min(span, s.rows - r0)});
        }
        seg_off = e;
      }
    }
    if (pr <= L.partial_rows_cap || s_eff == 1) {
      if (pr > L.partial_rows_cap)
        return fail(ASPIRE_ERR_CAPACITY, "aspire_plan_build: float workspace too small");
      partial_rows = pr;
      break;
    }
    s_eff = std::max<int64_t>(1, s_eff / 2);
  }
  for (int c = 0; c < 3; ++c) {
    const auto& citems = sc.citems[c];
    if (static_cast<int64_t>(citems.size()) > L.max_items) {
      set_error("aspire_plan_build: class %d needs %zu work items, capacity %d", c, citems.size(),
                L.max_items);
      return ASPIRE_ERR_CAPACITY;
    }
    // CSR by wave (stable: keeps each wave's pieces in page order).
    sc.counts.assign(W + 1, 0);
    for (const auto& pi : citems) sc.counts[pi.first + 1]++;
    for (int w = 0; w < W; ++w) sc.counts[w + 1] += sc.counts[w];
    int32_t* indptr = buf + off.indptr[c];
    std::memcpy(indptr, sc.counts.data(), sizeof(int32_t) * (W + 1));
    WorkItem* items = reinterpret_cast<WorkItem*>(buf + off.items[c]);
    for (const auto& pi : citems) items[sc.counts[pi.first]++] = pi.second;
    num_items[c] = static_cast<int>(citems.size());
  }
  if (static_cast<int64_t>(sc.merges.size()) > L.max_merge) {
    set_error("aspire_plan_build: %zu merge items, capacity %d", sc.merges.size(), L.max_merge);
    return ASPIRE_ERR_CAPACITY;
  }
  if (!sc.merges.empty())
    std::memcpy(buf + off.merge, sc.merges.data(), sizeof(MergeItem) * sc.merges.size());
  std::memset(buf + off.header, 0, 32 * sizeof(int32_t));
  buf[off.header + 0] = num_items[0];
  buf[off.header + 1] = num_items[1];
  buf[off.header + 2] = num_items[2];
  buf[off.header + 3] = static_cast<int32_t>(sc.merges.size());
  buf[off.header + 4] = hpu;  // kv heads per slot (waves of a slot share pages)

  info->num_items[0] = num_items[0];
  info->num_items[1] = num_items[1];
  info->num_items[2] = num_items[2];
  info->num_merge = static_cast<int32_t>(sc.merges.size());
  info->partial_rows = partial_rows;
  info->num_segments = num_segments;
  info->max_rows = max_rows;
  info->split_rows = split_rows;
  info->total_pages = total_pages;
  info->live_bytes = (off.items[0] + int64_t(num_items[0] + num_items[1] + num_items[2]) * 8 +
                      int64_t(sc.merges.size()) * 8) *
                     4;
  return ASPIRE_OK;
}

int check_common(const aspire_plan_layout* layout, const int32_t* qo_indptr, int32_t batch, int32_t num_qo_heads,
                 int32_t num_kv_heads, int32_t page_size, const void* host_buf, int64_t host_buf_bytes,
                 const aspire_plan_info* info, const char* fn) {
  if (!layout || !host_buf || !info) {
    set_error("%s: null argument", fn);
    return ASPIRE_ERR_INVALID;
  }
  const char* msg = nullptr;
  if (batch < 0) msg = "negative batch";
  else if (batch >= (1 << 23)) msg = "batch too large";
  else if (batch > 0 && !qo_indptr) msg = "null plan array";
  else if (page_size != kPage) msg = "page_size must be 16";
  else if (num_kv_heads <= 0 || num_kv_heads >= 256) msg = "num_kv_heads must be in [1, 255]";
  else if (num_qo_heads <= 0 || num_qo_heads % num_kv_heads != 0) msg = "num_qo_heads must be a multiple of num_kv_heads";
  // a query token's GQA group is the smallest row unit: it must fit one 3-tile item
  else if (num_qo_heads / num_kv_heads > 16 * kMaxRowTiles) msg = "num_qo_heads / num_kv_heads must be at most 48";
  else if (host_buf_bytes < plan_offsets(*layout).total * 4) msg = "host plan buffer smaller than the layout";
  if (msg) {
    set_error("%s: %s", fn, msg);
    return ASPIRE_ERR_INVALID;
  }
  return ASPIRE_OK;
}

}  // namespace
}  // namespace aspire

extern "C" int aspire_plan_build(const aspire_plan_layout* layout, const int32_t* qo_indptr,
                                 const int32_t* kv_indptr, const int32_t* kv_len, int32_t batch,
                                 int32_t per_head_lists, int32_t num_qo_heads,
                                 int32_t num_kv_heads, int32_t page_size, int32_t causal,
                                 void* host_buf, int64_t host_buf_bytes, aspire_plan_info* info) {
  using namespace aspire;
  int rc = check_common(layout, qo_indptr, batch, num_qo_heads, num_kv_heads, page_size, host_buf, host_buf_bytes,
                        info, "aspire_plan_build");
  if (rc != ASPIRE_OK) return rc;
  ASPIRE_CHECK_ARG(batch == 0 || (kv_indptr && kv_len), "null plan array");
  const int64_t n = per_head_lists ? int64_t(batch) * num_kv_heads : batch;
  Scratch& sc = scratch();
  sc.start.resize(std::max<int64_t>(n, 1));
  sc.pages.resize(std::max<int64_t>(n, 1));
  for (int64_t s = 0; s < n; ++s) {
    sc.start[s] = kv_indptr[s];
    sc.pages[s] = kv_indptr[s + 1] - kv_indptr[s];
  }
  return plan_core(layout, qo_indptr, sc.start.data(), sc.pages.data(), kv_len, batch, per_head_lists != 0,
                   num_qo_heads, num_kv_heads, causal, host_buf, info);
}

extern "C" int aspire_plan_build_segments(const aspire_plan_layout* layout, const int32_t* qo_indptr,
                                          const int32_t* seg_start, const int32_t* seg_pages,
                                          const int32_t* seg_kv_len, int32_t batch, int32_t num_qo_heads,
                                          int32_t num_kv_heads, int32_t page_size, int32_t causal,
                                          void* host_buf, int64_t host_buf_bytes, aspire_plan_info* info) {
  using namespace aspire;
  int rc = check_common(layout, qo_indptr, batch, num_qo_heads, num_kv_heads, page_size, host_buf, host_buf_bytes,
                        info, "aspire_plan_build_segments");
  if (rc != ASPIRE_OK) return rc;
  ASPIRE_CHECK_ARG(batch == 0 || (seg_start && seg_pages && seg_kv_len), "null plan array");
  return plan_core(layout, qo_indptr, seg_start, seg_pages, seg_kv_len, batch, true, num_qo_heads, num_kv_heads,
                   causal, host_buf, info);
}

extern "C" int aspire_plan_upload(const aspire_plan_layout* layout, const aspire_plan_info* info,
                                  const void* host_buf, void* dev_buf, void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(layout && info && host_buf && dev_buf, "null argument");
  const PlanOffsets off = plan_offsets(*layout);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const char* h = static_cast<const char*>(host_buf);
  char* d = static_cast<char*>(dev_buf);
  // Header and the three indptr arrays are contiguous.
  ASPIRE_CHECK_HIP(hipMemcpyAsync(d, h, off.items[0] * 4, hipMemcpyHostToDevice, s));
  for (int c = 0; c < 3; ++c) {
    const int64_t n = int64_t(info->num_items[c]) * 8 * 4;
    if (n > 0)
      ASPIRE_CHECK_HIP(hipMemcpyAsync(d + off.items[c] * 4, h + off.items[c] * 4, n,
                                      hipMemcpyHostToDevice, s));
  }
  const int64_t nm = int64_t(info->num_merge) * 8 * 4;
  if (nm > 0)
    ASPIRE_CHECK_HIP(
        hipMemcpyAsync(d + off.merge * 4, h + off.merge * 4, nm, hipMemcpyHostToDevice, s));
  return ASPIRE_OK;
}
