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
//     (head, slot) and thread, 128 pages per 256-thread workgroup;
//   * other page sizes (1..16): 16 lanes per page, one token per lane.
//
// topk: one wave per row / (row, kv head) segment. Scores become
// order-preserving uint32 keys (in registers up to 2048 pages, else in LDS);
// up to 32 steps of a bitwise search, each counting keys >= a candidate, find
// the k-th largest key (or stop once exactly k keys are >= the candidate); an ordered compaction keeps every larger key plus the
// lowest-index ties (mbcnt ranks), emitting logical pages in ascending order. When the reference's
// order is requested they are sorted by physical page id: skipped when the
// ids are already ascending, a rank sort up to 256 pages, bitonic beyond.
#include <algorithm>

#include "common.h"

namespace aspire {
namespace {

constexpr int kTopkThreads = 64;
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

__device__ __forceinline__ int slot_qrow(const ScoreParams& p, int row, int slot, int slots) {
  const int max_q = max(p.lse_rows - 1, 0);
  const int first = min(max(p.qo_indptr[row], 0), max_q);
  const int last = min(max(p.qo_indptr[row + 1] - 1, 0), max_q);
  return (slot == 0 && slots == 2) ? first : last;
}

// Page size 16: thread pair (2i, 2i+1) covers page blockIdx.y * 128 + i.
template <int SLOTS>
__global__ __launch_bounds__(256) void first_last_scores_p16_kernel(ScoreParams p) {
  const int rl = blockIdx.x;
  const int row = p.row_ids ? p.row_ids[rl] : rl;
  const int np = p.num_pages[row];
  const int j = blockIdx.y * 128 + (threadIdx.x >> 1);
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

__device__ __forceinline__ int popc64(uint64_t m) { return __builtin_popcountll(m); }

// Number of set bits of m in lanes below this one.
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
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

// Keys of one segment, lane l holding keys 256 i + 4 l + e (e < 4) of step i.
// KREG > 0: the keys live in KREG registers per lane (n_pad <= 64 * KREG);
// KREG == 0: they stay in LDS and every pass reads them back.
template <int KREG>
struct SegmentKeys {
  uint32_t reg[KREG > 0 ? KREG : 1];
  const uint32_t* lds;
  int n_pad;

  __device__ __forceinline__ uint4 quad(int i) const {
    if constexpr (KREG > 0) {
      return uint4{reg[4 * i], reg[4 * i + 1], reg[4 * i + 2], reg[4 * i + 3]};
    } else {
      return *reinterpret_cast<const uint4*>(lds + 256 * i + 4 * threadIdx.x);
    }
  }
  __device__ __forceinline__ int steps() const { return n_pad >> 8; }

  // Wave-wide count of keys >= cand (padding keys are 0 and cand >= 1),
  // counted per lane in VALU and summed once (a ballot + scalar popcount per
  // key stalls on every vector-to-scalar dependency).
  __device__ __forceinline__ int count_ge(uint32_t cand) const {
    int cnt = 0;
    if constexpr (KREG > 0) {
      // All KREG registers hold keys (0 past n): no per-step guard, no branch.
#pragma unroll
      for (int i = 0; i < KREG / 4; ++i) {
        const uint4 q = quad(i);
        cnt += int(q.x >= cand) + int(q.y >= cand) + int(q.z >= cand) + int(q.w >= cand);
      }
    } else {
      for (int i = 0; i < steps(); ++i) {
        const uint4 q = quad(i);
        cnt += int(q.x >= cand) + int(q.y >= cand) + int(q.z >= cand) + int(q.w >= cand);
      }
    }
    return wave_sum_int(cnt);
  }
};

template <int KREG>
__global__ __launch_bounds__(kTopkThreads) void topk_kernel(TopkParams p) {
  extern __shared__ __align__(16) uint32_t keys[];
  __shared__ __align__(16) int32_t sel[kMaxSel];
  const int s = blockIdx.x;
  const int lane = threadIdx.x;
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
  const uint32_t inf_key = order_key(__builtin_huge_valf());
  SegmentKeys<KREG> K;
  K.n_pad = (n + 255) & ~255;
  K.lds = keys;
  // Loads use a clamped index, so they are unconditional and all in flight at
  // once (a guarded load becomes a branch that waits for each load in turn).
  const int last = max(n - 1, 0);
  auto key_of = [&](int j, float v) {
    uint32_t key = order_key(v);  // selects, not branches: the loads stay unconditional
    key = j >= forced_from ? inf_key : key;
    return j >= n ? 0u : key;
  };
  if constexpr (KREG > 0) {
    // Padding keys are 0, below every candidate of the search.
    float v[KREG];
#pragma unroll
    for (int i = 0; i < KREG / 4; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * i + e] = sc[min(256 * i + 4 * lane + e, last)];
    }
#pragma unroll
    for (int i = 0; i < KREG / 4; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) K.reg[4 * i + e] = key_of(256 * i + 4 * lane + e, v[4 * i + e]);
    }
  } else {
    // Eight independent loads in flight per lane before the LDS writes.
    for (int j0 = 0; j0 < K.n_pad; j0 += 8 * kTopkThreads) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = sc[min(j0 + u * kTopkThreads + lane, last)];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + u * kTopkThreads + lane;
        if (j < K.n_pad) keys[j] = key_of(j, v[u]);
      }
    }
    __syncthreads();
  }
  // thr = the kk-th largest key: the largest value with count(key >= thr) >= kk.
  uint32_t thr = 0;
  int need_eq = n;  // kk == n: every key is taken
  if (kk > 0 && kk < n) {
    bool exact = false;
    for (int b = 31; b >= 0; --b) {
      const uint32_t cand = thr | (1u << b);
      const int c = K.count_ge(cand);
      if (c >= kk) thr = cand;
      if (c == kk) {  // exactly the keys >= cand are selected: stop early
        exact = true;
        break;
      }
    }
    if (exact) {
      thr -= 1u;  // take key > cand - 1, i.e. key >= cand (cand >= 1); no ties needed
      need_eq = 0;
    } else {
      const int gt = thr == 0xffffffffu ? 0 : K.count_ge(thr + 1u);
      need_eq = kk - gt;
    }
  }
  // Ordered compaction: every key above thr, plus the lowest-index ties.
  int base = 0, eq_base = 0;
  auto compact_step = [&](int i) {
    const int jl = 256 * i + lane * 4;
    const uint4 k4 = K.quad(i);
    const uint32_t kv[4] = {k4.x, k4.y, k4.z, k4.w};
    bool eq[4], gt[4];
    uint64_t eqm[4];
    int eq_below = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool in = jl + e < n;
      eq[e] = in && kv[e] == thr;
      gt[e] = in && kv[e] > thr;
      eqm[e] = __builtin_amdgcn_ballot_w64(eq[e]);
      eq_below += lanes_below(eqm[e]);
    }
    bool take[4];
    uint64_t tm[4];
    int take_below = 0;
    int rank = eq_base + eq_below;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      take[e] = gt[e] || (eq[e] && rank < need_eq);
      rank += eq[e];
      tm[e] = __builtin_amdgcn_ballot_w64(take[e]);
      take_below += lanes_below(tm[e]);
    }
    int pos = base + take_below;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (take[e] && pos < kMaxSel) sel[pos] = jl + e;
      pos += take[e];
      base += popc64(tm[e]);
      eq_base += popc64(eqm[e]);
    }
  };
  if (kk > 0) {
    if constexpr (KREG > 0) {
#pragma unroll
      for (int i = 0; i < KREG / 4; ++i)  // constant register indices
        if (i < K.steps() && base < kk) compact_step(i);
    } else {
      for (int i = 0; i < K.steps() && base < kk; ++i) compact_step(i);
    }
  }
  __syncthreads();
  const int32_t* trow = p.table + int64_t(row) * p.table_stride;
  // Map logical -> physical; pad with INT_MAX to a power of two >= 4 for the sorts.
  int pow2 = 4;
  while (pow2 < kk) pow2 <<= 1;
  for (int i = lane; i < pow2; i += kTopkThreads)
    sel[i] = i < kk ? trow[max(0, min(sel[i], static_cast<int>(p.table_stride) - 1))] : 0x7fffffff;
  __syncthreads();
  if (p.order == 0 && kk > 1) {
    // Already ascending (the reference's arange block table): nothing to do.
    bool desc = false;
    for (int i = lane; i + 1 < kk; i += kTopkThreads) desc |= sel[i] > sel[i + 1];
    if (__builtin_amdgcn_ballot_w64(desc) != 0) {
      if (kk <= 4 * kTopkThreads) {
        // Rank sort: lane l places entries l + 64u at their rank, read with
        // broadcast LDS loads (ties keep index order; equal ids are identical).
        // Lexicographic (id, index) keys make every rank distinct; entries
        // [kk, pad4) hold INT_MAX with indices >= kk, so they rank above all.
        const int per = (kk + kTopkThreads - 1) / kTopkThreads;
        int64_t mine[4];
        int rank[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = lane + 64 * u;
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
          if (lane + 64 * u < kk) sel[rank[u]] = int32_t(mine[u] >> 32);
        __syncthreads();
      } else {
        for (int size = 2; size <= pow2; size <<= 1) {
          for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = lane; i < pow2; i += kTopkThreads) {
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
  for (int i = lane; i < p.sel_width; i += kTopkThreads) out[i] = i < kk ? sel[i] : 0;
  if (lane == 0 && p.valid != nullptr) p.valid[s] = k;
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
    const dim3 grid(rows, (pages + 127) / 128);
    if (slots == 2)
      hipLaunchKernelGGL(first_last_scores_p16_kernel<2>, grid, dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL(first_last_scores_p16_kernel<1>, grid, dim3(256), 0, st, p);
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
  if (score_stride <= 64 * 32) {  // keys in 32 registers per lane
    hipLaunchKernelGGL(topk_kernel<32>, dim3(segments), dim3(kTopkThreads), 0, st, p);
  } else {
    const size_t lds = size_t((score_stride + 255) & ~int64_t(255)) * 4;
    hipLaunchKernelGGL(topk_kernel<0>, dim3(segments), dim3(kTopkThreads), lds, st, p);
  }
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}
