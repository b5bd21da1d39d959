// (a3) Page scoring and top-k page selection.
//
// first_last_scores: grid (rows, pages / 16); one thread per token, 16 lanes
// per page. It applies the reference selector's element-wise chain in the same
// precision (fp16 product, fp32 subtraction, nan_to_num, exp2, max over heads,
// sum over the two query slots) and reduces each page's 16 tokens with xor
// shuffles, reading only pages below the row's page count.
//
// topk: one workgroup per row / (row, kv head) segment. Scores become
// order-preserving uint32 keys in LDS; a 4-pass 8-bit radix select finds the
// k-th largest key, a block scan keeps every larger key plus the lowest-index
// ties, emitting logical pages in ascending order; a bitonic sort orders them
// by physical page id when the reference's order is requested.
#include <algorithm>

#include "common.h"

namespace aspire {
namespace {

constexpr float kFltMax = 3.4028234663852886e38f;
constexpr int kTopkThreads = 256;
constexpr int kMaxSel = 2048;

__global__ __launch_bounds__(256) void first_last_scores_kernel(
    const _Float16* dump, int64_t kv_stride, int n_heads, int max_seq, const float* lse,
    int lse_rows, const int32_t* qo_indptr, const int32_t* num_pages, const int32_t* row_ids,
    int page_size, float c, float* scores, int64_t score_stride, int slots, int pages) {
  const int rl = blockIdx.x;
  const int row = row_ids ? row_ids[rl] : rl;
  const int np = num_pages[row];
  const int j = blockIdx.y * 16 + (threadIdx.x >> 4);
  if (j >= np || j >= pages) return;  // all 16 lanes of a page leave together
  const int t = j * page_size + (threadIdx.x & 15);
  const int max_q = max(lse_rows - 1, 0);
  const int q_first = min(max(qo_indptr[row], 0), max_q);
  const int q_last = min(max(qo_indptr[row + 1] - 1, 0), max_q);
  float tok = 0.f;
  if (t < max_seq && (threadIdx.x & 15) < page_size) {
    for (int slot = 0; slot < slots; ++slot) {
      const int qrow = (slot == 0 && slots == 2) ? q_first : q_last;
      float mx = 0.f;  // exp2 values are >= 0
      for (int h = 0; h < n_heads; ++h) {
        const float lg =
            static_cast<float>(dump[(int64_t(row * n_heads + h) * slots + slot) * kv_stride + t]);
        const _Float16 prod = static_cast<_Float16>(lg * c);
        float n = static_cast<float>(prod) - lse[int64_t(qrow) * n_heads + h];
        if (n != n)
          n = -__builtin_huge_valf();
        else if (n == __builtin_huge_valf())
          n = kFltMax;
        else if (n == -__builtin_huge_valf())
          n = -kFltMax;
        mx = fmaxf(mx, exp2f(n));
      }
      tok += mx;
    }
  }
  float sum = tok;
  sum += __shfl_xor(sum, 1, 64);
  sum += __shfl_xor(sum, 2, 64);
  sum += __shfl_xor(sum, 4, 64);
  sum += __shfl_xor(sum, 8, 64);
  if ((threadIdx.x & 15) == 0) {
    const float bias = -static_cast<float>(j) * 1e-7f;
    scores[int64_t(rl) * score_stride + j] = sum + bias;
  }
}

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive block scan of one int per thread (kTopkThreads threads).
__device__ int block_exclusive_scan(int v, int* tmp, int& total) {
  const int tid = threadIdx.x;
  tmp[tid] = v;
  __syncthreads();
  for (int off = 1; off < kTopkThreads; off <<= 1) {
    const int add = tid >= off ? tmp[tid - off] : 0;
    __syncthreads();
    tmp[tid] += add;
    __syncthreads();
  }
  total = tmp[kTopkThreads - 1];
  const int incl = tmp[tid];
  __syncthreads();
  return incl - v;
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

__global__ __launch_bounds__(kTopkThreads) void topk_kernel(TopkParams p) {
  extern __shared__ uint32_t keys[];
  __shared__ uint32_t hist[256];
  __shared__ int scan_tmp[kTopkThreads];
  __shared__ int32_t sel[kMaxSel];
  __shared__ uint32_t s_prefix, s_mask;
  __shared__ int s_remaining;
  const int s = blockIdx.x;
  const int tid = threadIdx.x;
  const int rl = s / p.segs_per_row;
  const int row = p.row_ids ? p.row_ids[rl] : rl;
  const int n = min(max(p.num_pages[row], 0), static_cast<int>(p.score_stride));
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
  k = max(k, 0);
  const int kk = min(min(k, kMaxSel), p.sel_width);
  const float* sc = p.scores + int64_t(s) * p.score_stride;
  const int forced_from = n - p.L;
  for (int j = tid; j < n; j += kTopkThreads)
    keys[j] = j >= forced_from ? order_key(__builtin_huge_valf()) : order_key(sc[j]);
  if (tid == 0) {
    s_prefix = 0;
    s_mask = 0;
    s_remaining = kk;
  }
  __syncthreads();
  if (kk > 0) {
    for (int shift = 24; shift >= 0; shift -= 8) {
      hist[tid] = 0;
      __syncthreads();
      const uint32_t prefix = s_prefix, mask = s_mask;
      for (int j = tid; j < n; j += kTopkThreads) {
        const uint32_t key = keys[j];
        if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        int remaining = s_remaining;
        int cum = 0;
        for (int d = 255; d >= 0; --d) {
          const int hcount = static_cast<int>(hist[d]);
          if (cum + hcount >= remaining) {
            s_prefix = prefix | (uint32_t(d) << shift);
            s_remaining = remaining - cum;
            break;
          }
          cum += hcount;
        }
        s_mask = mask | (255u << shift);
      }
      __syncthreads();
    }
  }
  const uint32_t thr = s_prefix;
  const int need_eq = s_remaining;
  // Ordered compaction over contiguous per-thread chunks.
  const int chunk = (n + kTopkThreads - 1) / kTopkThreads;
  const int j0 = min(tid * chunk, n), j1 = min(j0 + chunk, n);
  int total = 0;
  int eq_local = 0;
  if (kk > 0)
    for (int j = j0; j < j1; ++j) eq_local += keys[j] == thr;
  const int eq_base = block_exclusive_scan(eq_local, scan_tmp, total);
  int take_local = 0;
  if (kk > 0) {
    int eq_seen = eq_base;
    for (int j = j0; j < j1; ++j) {
      const uint32_t key = keys[j];
      if (key > thr) {
        ++take_local;
      } else if (key == thr) {
        if (eq_seen < need_eq) ++take_local;
        ++eq_seen;
      }
    }
  }
  const int out_base = block_exclusive_scan(take_local, scan_tmp, total);
  if (kk > 0) {
    int eq_seen = eq_base;
    int o = out_base;
    for (int j = j0; j < j1; ++j) {
      const uint32_t key = keys[j];
      bool take = key > thr;
      if (key == thr) {
        take = eq_seen < need_eq;
        ++eq_seen;
      }
      if (take && o < kMaxSel) sel[o++] = j;
    }
  }
  __syncthreads();
  const int32_t* trow = p.table + int64_t(row) * p.table_stride;
  // Map logical -> physical; pad to a power of two for the sort.
  int pow2 = 1;
  while (pow2 < kk) pow2 <<= 1;
  for (int i = tid; i < pow2; i += kTopkThreads)
    sel[i] = i < kk ? trow[min(sel[i], static_cast<int>(p.table_stride) - 1)] : 0x7fffffff;
  __syncthreads();
  if (p.order == 0 && kk > 1) {
    for (int size = 2; size <= pow2; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < pow2; i += kTopkThreads) {
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
  int32_t* out = p.selected + int64_t(s) * p.sel_stride;
  for (int i = tid; i < p.sel_width; i += kTopkThreads) out[i] = i < kk ? sel[i] : 0;
  if (tid == 0 && p.valid != nullptr) p.valid[s] = k;
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
  const dim3 grid(rows, (pages + 15) / 16);
  hipLaunchKernelGGL(first_last_scores_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const _Float16*>(dump), kv_stride, n_heads, max_seq_length, lse,
                     lse_rows, qo_indptr, num_pages, row_ids, page_size, sm_scale_log2e, scores,
                     score_stride, slots, pages);
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
  const size_t lds = size_t(score_stride) * 4;
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
  hipLaunchKernelGGL(topk_kernel, dim3(segments), dim3(kTopkThreads), lds,
                     static_cast<hipStream_t>(stream), p);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}
