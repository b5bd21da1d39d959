// (a3) Page scoring and top-k page selection.
//
// first_last_scores: applies the reference selector's element-wise chain in the
// same precision (fp16 product, fp32 subtraction, nan_to_num, exp2, max over
// heads, sum over the query slots) and reduces each page's tokens, reading only
// pages below the row's page count. exp2 is monotonic, so max_h exp2(n_h) ==
// exp2(max_h n_h): the kernel takes the max of the fp32 differences and calls
// exp2 once per token and slot. nan_to_num needs no code: fmaxf drops NaN
// (the reference maps it to -inf, whose exp2 is 0 and never wins the max over
// values >= 0), and exp2(+-inf) equals exp2(+-FLT_MAX) in fp32.
//   * page 16, 8-aligned strides: 2 threads per page, one 16-byte load per
//     (head, slot) and thread, 32 pages per one-wave workgroup;
//   * other page sizes (1..16): 16 lanes per page, one token per lane.
//
// topk: one workgroup per row / (row, kv head) segment. Scores become
// order-preserving uint32 keys held in registers; a radix select over three
// digits (LDS histograms, one workgroup-wide scan per digit) finds the k-th
// largest key, and an ordered compaction (one exclusive scan of per-thread
// counts) keeps every larger key plus the lowest-index ties, emitting logical
// pages in ascending order. When the reference's order is requested they are
// sorted by physical page id: skipped when the ids are already ascending, a
// rank sort up to 4 x (threads) pages, bitonic beyond.
#include <algorithm>

#include "common.h"

namespace aspire {
namespace {

constexpr int kMaxSel = 2048;

struct ScoreParams {
  const _Float16* dump;
  int64_t kv_stride;
  int n_heads, max_seq;
  const float* lse;
  int lse_rows;
  const int32_t* qo_indptr;
  const int32_t* num_pages;
  const int32_t* row_ids;
  int page_size;
  float c;
  float* scores;
  int64_t score_stride;
  int slots, pages;
};

__device__ __forceinline__ float chain_diff(_Float16 logit, float c, float lse) {
  const _Float16 prod = static_cast<_Float16>(static_cast<float>(logit) * c);
  return static_cast<float>(prod) - lse;
}

// Pages per workgroup of the page-size-16 scores kernel (two threads per page, one wave):
// measured 30.2 us against 32.0 for 128 pages in 256-thread workgroups at refresh scale.
constexpr int kScPages = 32;

__device__ __forceinline__ int slot_qrow(const ScoreParams& p, int row, int slot, int slots) {
  const int max_q = max(p.lse_rows - 1, 0);
  const int first = min(max(p.qo_indptr[row], 0), max_q);
  const int last = min(max(p.qo_indptr[row + 1] - 1, 0), max_q);
  return (slot == 0 && slots == 2) ? first : last;
}

// Page size 16: thread pair (2i, 2i+1) covers page blockIdx.y * kScPages + i.
template <int SLOTS>
__global__ __launch_bounds__(2 * kScPages) void first_last_scores_p16_kernel(ScoreParams p) {
  const int rl = blockIdx.x;
  const int row = p.row_ids ? p.row_ids[rl] : rl;
  const int np = p.num_pages[row];
  const int j = blockIdx.y * kScPages + (threadIdx.x >> 1);
  if (j >= np || j >= p.pages) return;  // both threads of a page leave together
  const int t0 = j * 16 + (threadIdx.x & 1) * 8;
  float tok[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) tok[e] = 0.f;
  if (t0 < p.max_seq) {  // max_seq % 8 == 0: all 8 tokens are in range
#pragma unroll
    for (int slot = 0; slot < SLOTS; ++slot) {
      const int qrow = slot_qrow(p, row, slot, SLOTS);
      const float* lse = p.lse + int64_t(qrow) * p.n_heads;
      const _Float16* base = p.dump + (int64_t(row) * p.n_heads * SLOTS + slot) * p.kv_stride + t0;
      float mx[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) mx[e] = -__builtin_huge_valf();
#pragma unroll 8
      for (int h = 0; h < p.n_heads; ++h) {
        const uint4 raw = *reinterpret_cast<const uint4*>(base + int64_t(h) * SLOTS * p.kv_stride);
        const float l = lse[h];
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint16_t bits = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
          mx[e] = fmaxf(mx[e], chain_diff(__builtin_bit_cast(_Float16, bits), p.c, l));
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) tok[e] += exp2f(mx[e]);
    }
  }
  float sum = ((tok[0] + tok[1]) + (tok[2] + tok[3])) + ((tok[4] + tok[5]) + (tok[6] + tok[7]));
  sum += __shfl_xor(sum, 1, 64);
  if ((threadIdx.x & 1) == 0) {
    const float bias = -static_cast<float>(j) * 1e-7f;
    p.scores[int64_t(rl) * p.score_stride + j] = sum + bias;
  }
}

// Any page size in [1, 16]: 16 lanes per page, one token per lane.
__global__ __launch_bounds__(256) void first_last_scores_kernel(ScoreParams p) {
  const int rl = blockIdx.x;
  const int row = p.row_ids ? p.row_ids[rl] : rl;
  const int np = p.num_pages[row];
  const int j = blockIdx.y * 16 + (threadIdx.x >> 4);
  if (j >= np || j >= p.pages) return;  // all 16 lanes of a page leave together
  const int t = j * p.page_size + (threadIdx.x & 15);
  float tok = 0.f;
  if (t < p.max_seq && (threadIdx.x & 15) < p.page_size) {
    for (int slot = 0; slot < p.slots; ++slot) {
      const int qrow = slot_qrow(p, row, slot, p.slots);
      float mx = -__builtin_huge_valf();
      for (int h = 0; h < p.n_heads; ++h) {
        const _Float16 lg = p.dump[(int64_t(row * p.n_heads + h) * p.slots + slot) * p.kv_stride + t];
        mx = fmaxf(mx, chain_diff(lg, p.c, p.lse[int64_t(qrow) * p.n_heads + h]));
      }
      tok += exp2f(mx);
    }
  }
  float sum = tok;
  sum += __shfl_xor(sum, 1, 64);
  sum += __shfl_xor(sum, 2, 64);
  sum += __shfl_xor(sum, 4, 64);
  sum += __shfl_xor(sum, 8, 64);
  if ((threadIdx.x & 15) == 0) {
    const float bias = -static_cast<float>(j) * 1e-7f;
    p.scores[int64_t(rl) * p.score_stride + j] = sum + bias;
  }
}

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct TopkParams {
  const float* scores;
  int64_t score_stride;
  const int32_t* num_pages;
  const int32_t* row_ids;
  int segs_per_row;
  int L;
  int count_mode, subset, min_pages;
  float pct;
  const int32_t* table;
  int64_t table_stride;
  int order;
  int32_t* selected;
  int64_t sel_stride;
  int sel_width;
  int32_t* valid;
};

// Pages a segment of n pages keeps (page_selector.py:52-62): the budget, the minimum, or
// the percentage clamped between them.
__device__ __forceinline__ int segment_take(const TopkParams& p, int n) {
  int k;
  if (p.count_mode == 0) {
    k = min(n, p.subset);
  } else if (p.count_mode == 1) {
    k = min(n, p.min_pages);
  } else {
    const int lo = min(n, p.min_pages), hi = min(n, p.subset);
    const float t = ceilf((static_cast<float>(n) * p.pct) / 100.0f);
    k = min(max(static_cast<int>(t), lo), hi);
  }
  return max(k, 0);
}

// One workgroup per segment (a row or a (row, kv head)); thread t holds the keys of pages
// PER t .. PER t + PER - 1 in registers (THREADS x PER >= the score stride: 256 x 8 up to
// 2,048 pages, 1,024 x 12 up to 12,288). The k-th largest key comes from a radix select over
// 11-, 11- and 10-bit digits (bits 31..21, 20..10, 9..0): each pass counts the keys that
// match the digits chosen so far in an LDS histogram of 2,048 bins, and one workgroup-wide
// scan over the bins in descending order finds the digit whose bin holds the k-th key. A
// pass whose bin holds exactly the keys still needed ends the search (every key >= the
// bin's lowest value is taken). The compaction is one workgroup-wide exclusive scan of each
// thread's (keys above, ties) counts: a thread writes its taken pages at its offset, in page
// order, ties by lowest page first.
constexpr int kTbBins = 2048;

// Exclusive prefix sum of v over the workgroup's threads in index order (inclusive
// shuffles within each wave, wave totals through LDS); *total gets the sum of all.
template <int THREADS>
__device__ __forceinline__ uint32_t tb_exclusive_scan(uint32_t v, uint32_t* wtot, uint32_t* total) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  uint32_t inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_up(inc, d, 64);
    if (lane >= d) inc += o;
  }
  if (lane == 63) wtot[w] = inc;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int i = 0; i < THREADS / 64; ++i) {
    const uint32_t x = wtot[i];
    before += i < w ? x : 0u;
    all += x;
  }
  __syncthreads();  // wtot is reused by the next scan
  *total = all;
  return before + inc - v;
}

template <int THREADS, int PER>
__global__ __launch_bounds__(THREADS) void topk_block_kernel(TopkParams p) {
  constexpr int BPT = kTbBins / THREADS;  // histogram bins per thread
  static_assert(BPT * THREADS == kTbBins && THREADS * PER < 65536, "bins split evenly; counts pack into 16 bits");
  __shared__ uint32_t hist[kTbBins];
  __shared__ __align__(16) int32_t sel[kMaxSel];
  __shared__ uint32_t wtot[THREADS / 64];
  __shared__ uint32_t pick[3];  // bin, keys in higher bins, keys in the bin
  const int s = blockIdx.x;
  const int t = threadIdx.x;
  const int rl = s / p.segs_per_row;
  const int row = p.row_ids ? p.row_ids[rl] : rl;
  const int n = min(max(p.num_pages[row], 0), static_cast<int>(p.score_stride));
  const int k = segment_take(p, n);
  const int kk = min(min(k, kMaxSel), p.sel_width);
  const float* sc = p.scores + int64_t(s) * p.score_stride;
  const int forced_from = n - p.L;
  const uint32_t inf_key = order_key(__builtin_huge_valf());
  const int last = max(n - 1, 0);
  const int j0 = PER * t;
  // unconditional loads (clamped index): all in flight at once
  float v[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) v[e] = sc[min(j0 + e, last)];
  for (int i = t; i < kTbBins; i += THREADS) hist[i] = 0u;
  uint32_t key[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) key[e] = j0 + e >= forced_from ? inf_key : order_key(v[e]);

  // thr and need_eq: take every page with key > thr, and the first need_eq pages with key == thr
  uint32_t thr = 0u;
  int need_eq = n;  // kk == n: every page is taken
  uint32_t total = 0u;
  if (kk > 0 && kk < n) {
    uint32_t prefix = 0u, hi_mask = 0u;
    int need = kk;
    bool exact = false;
    __syncthreads();  // histogram cleared
#pragma unroll
    for (int pass = 0; pass < 3; ++pass) {
      const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
      const uint32_t dmask = pass == 2 ? 1023u : 2047u;
#pragma unroll
      for (int e = 0; e < PER; ++e)
        if (j0 + e < n && (key[e] & hi_mask) == prefix) atomicAdd(&hist[(key[e] >> shift) & dmask], 1u);
      __syncthreads();
      // thread t reads (and clears for the next pass) bins dmask - BPT t - i, i < BPT: the
      // workgroup's threads in index order cover the bins in descending order
      uint32_t c[BPT];
      uint32_t local = 0u;
#pragma unroll
      for (int i = 0; i < BPT; ++i) {
        const int b = int(dmask) - BPT * t - i;
        c[i] = b >= 0 ? hist[b] : 0u;
        if (b >= 0) hist[b] = 0u;
        local += c[i];
      }
      uint32_t above = tb_exclusive_scan<THREADS>(local, wtot, &total);
      if (above < uint32_t(need) && above + local >= uint32_t(need)) {
#pragma unroll
        for (int i = 0; i < BPT; ++i) {
          if (above + c[i] >= uint32_t(need)) {
            pick[0] = uint32_t(int(dmask) - BPT * t - i);
            pick[1] = above;
            pick[2] = c[i];
            break;
          }
          above += c[i];
        }
      }
      __syncthreads();
      const uint32_t b = pick[0];
      need -= int(pick[1]);
      const int in_bin = int(pick[2]);
      prefix |= b << shift;
      hi_mask |= dmask << shift;
      if (in_bin == need && prefix != 0u) {
        exact = true;
        break;
      }
    }
    if (exact) {
      thr = prefix - 1u;  // key > prefix - 1: every key >= the bin's lowest value
      need_eq = 0;
    } else {
      thr = prefix;
      need_eq = need;
    }
  }
  // ordered compaction
  uint32_t gt = 0u, eq = 0u;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const bool in = j0 + e < n;
    gt += uint32_t(in && key[e] > thr);
    eq += uint32_t(in && key[e] == thr);
  }
  const uint32_t ex = tb_exclusive_scan<THREADS>(gt | (eq << 16), wtot, &total);
  if (kk > 0) {
    int eq_rank = int(ex >> 16);
    int pos = int(ex & 0xffffu) + min(eq_rank, need_eq);
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const bool in = j0 + e < n;
      const bool tie = in && key[e] == thr;
      const bool take = (in && key[e] > thr) || (tie && eq_rank < need_eq);
      eq_rank += int(tie);
      if (take && pos < kMaxSel) sel[pos] = j0 + e;
      pos += int(take);
    }
  }
  __syncthreads();
  const int32_t* trow = p.table + int64_t(row) * p.table_stride;
  // Map logical -> physical; pad with INT_MAX to a power of two >= 4 for the sorts.
  int pow2 = 4;
  while (pow2 < kk) pow2 <<= 1;
  for (int i = t; i < pow2; i += THREADS)
    sel[i] = i < kk ? trow[max(0, min(sel[i], static_cast<int>(p.table_stride) - 1))] : 0x7fffffff;
  __syncthreads();
  if (p.order == 0 && kk > 1) {
    bool desc = false;
    for (int i = t; i + 1 < kk; i += THREADS) desc |= sel[i] > sel[i + 1];
    if (__syncthreads_or(desc)) {
      if (kk <= 4 * THREADS) {
        // Rank sort: thread t places entries t + THREADS u at their rank, read with broadcast LDS
        // loads; lexicographic (id, index) keys make every rank distinct.
        const int per = (kk + THREADS - 1) / THREADS;
        int64_t mine[4];
        int rank[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = t + THREADS * u;
          mine[u] = (int64_t(i < kk ? sel[i] : 0x7fffffff) << 32) | i;
          rank[u] = 0;
        }
        for (int j = 0; j < kk; j += 4) {
          const int4 w4 = *reinterpret_cast<const int4*>(sel + j);
          const int64_t w[4] = {(int64_t(w4.x) << 32) | j, (int64_t(w4.y) << 32) | (j + 1),
                                (int64_t(w4.z) << 32) | (j + 2), (int64_t(w4.w) << 32) | (j + 3)};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            if (u < per) {
#pragma unroll
              for (int e = 0; e < 4; ++e) rank[u] += int(w[e] < mine[u]);
            }
          }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (t + THREADS * u < kk) sel[rank[u]] = int32_t(mine[u] >> 32);
        __syncthreads();
      } else {
        for (int size = 2; size <= pow2; size <<= 1) {
          for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = t; i < pow2; i += THREADS) {
              const int partner = i ^ stride;
              if (partner > i) {
                const bool up = (i & size) == 0;
                const int32_t a = sel[i], b = sel[partner];
                if ((a > b) == up) {
                  sel[i] = b;
                  sel[partner] = a;
                }
              }
            }
            __syncthreads();
          }
        }
      }
    }
  }
  int32_t* out = p.selected + int64_t(s) * p.sel_stride;
  for (int i = t; i < p.sel_width; i += THREADS) out[i] = i < kk ? sel[i] : 0;
  if (t == 0 && p.valid != nullptr) p.valid[s] = k;
}

}  // namespace
}  // namespace aspire

extern "C" int aspire_select_first_last_scores(const void* dump, int64_t kv_stride, int32_t n_heads,
                                               int32_t bsz, int32_t max_seq_length, const float* lse,
                                               int32_t lse_rows, const int32_t* qo_indptr,
                                               const int32_t* num_pages, const int32_t* row_ids,
                                               int32_t rows, int32_t page_size,
                                               float sm_scale_log2e, float* scores,
                                               int64_t score_stride, int32_t slots, void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(rows >= 0 && n_heads > 0 && bsz >= 0 && max_seq_length >= 0, "bad sizes");
  ASPIRE_CHECK_ARG(page_size > 0 && page_size <= 16, "page_size must be in [1, 16]");
  if (rows == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(dump && lse && qo_indptr && num_pages && scores, "null pointer");
  ASPIRE_CHECK_ARG(kv_stride >= max_seq_length, "kv_stride smaller than max_seq_length");
  ASPIRE_CHECK_ARG(slots == 1 || slots == 2, "slots must be 1 or 2");
  (void)bsz;
  const int pages = (max_seq_length + page_size - 1) / page_size;
  if (pages == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(score_stride >= pages, "score_stride smaller than the page count");
  ScoreParams p;
  p.dump = static_cast<const _Float16*>(dump);
  p.kv_stride = kv_stride;
  p.n_heads = n_heads;
  p.max_seq = max_seq_length;
  p.lse = lse;
  p.lse_rows = lse_rows;
  p.qo_indptr = qo_indptr;
  p.num_pages = num_pages;
  p.row_ids = row_ids;
  p.page_size = page_size;
  p.c = sm_scale_log2e;
  p.scores = scores;
  p.score_stride = score_stride;
  p.slots = slots;
  p.pages = pages;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool vec = page_size == 16 && kv_stride % 8 == 0 && max_seq_length % 8 == 0 &&
                   (reinterpret_cast<uintptr_t>(dump) & 15) == 0;
  if (vec) {
    const dim3 grid(rows, (pages + kScPages - 1) / kScPages);
    const dim3 block(2 * kScPages);
    if (slots == 2)
      hipLaunchKernelGGL(first_last_scores_p16_kernel<2>, grid, block, 0, st, p);
    else
      hipLaunchKernelGGL(first_last_scores_p16_kernel<1>, grid, block, 0, st, p);
  } else {
    hipLaunchKernelGGL(first_last_scores_kernel, dim3(rows, (pages + 15) / 16), dim3(256), 0, st, p);
  }
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}

extern "C" int aspire_select_topk(const float* scores, int64_t score_stride, const int32_t* num_pages,
                                  const int32_t* row_ids, int32_t segments, int32_t segs_per_row,
                                  int32_t L, int32_t count_mode, int32_t subset, int32_t min_pages,
                                  float pct, const int32_t* block_table, int64_t table_stride,
                                  int32_t order, int32_t* selected, int64_t sel_stride,
                                  int32_t sel_width, int32_t* valid, void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(segments >= 0 && segs_per_row > 0, "bad segment counts");
  if (segments == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(scores && num_pages && block_table && selected, "null pointer");
  ASPIRE_CHECK_ARG(count_mode >= 0 && count_mode <= 2, "count_mode must be 0, 1 or 2");
  ASPIRE_CHECK_ARG(order == 0 || order == 1, "order must be 0 (physical) or 1 (logical)");
  ASPIRE_CHECK_ARG(subset <= kMaxSel && (count_mode != 1 || min_pages <= kMaxSel),
                   "selection budget larger than 2048 pages");
  ASPIRE_CHECK_ARG(score_stride > 0 && score_stride <= 12288,
                   "score_stride (max pages) must be in [1, 12288]");
  ASPIRE_CHECK_ARG(table_stride > 0 && sel_width >= 0, "bad table stride or selection width");
  TopkParams p;
  p.scores = scores;
  p.score_stride = score_stride;
  p.num_pages = num_pages;
  p.row_ids = row_ids;
  p.segs_per_row = segs_per_row;
  p.L = L;
  p.count_mode = count_mode;
  p.subset = subset;
  p.min_pages = min_pages;
  p.pct = pct;
  p.table = block_table;
  p.table_stride = table_stride;
  p.order = order;
  p.selected = selected;
  p.sel_stride = sel_stride;
  p.sel_width = sel_width;
  p.valid = valid;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (score_stride <= 256 * 8)
    hipLaunchKernelGGL((topk_block_kernel<256, 8>), dim3(segments), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((topk_block_kernel<1024, 12>), dim3(segments), dim3(1024), 0, st, p);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}
