// (f4) Token sampling and speculative verification for gfx950.
//
// * topk_candidates_kernel: the top_k logits of a row and their ids, descending, ties to the
//   lower id. One 1024-thread workgroup per row, 16-byte loads; rows of up to 155,648 logits
//   are read once and kept in registers as keys. Radix select on 16-bit order-preserving keys
//   of the bf16 logits: the high byte of the k-th key (for register-held rows from counts at
//   the top bins below the row's maximum, else from a histogram), then a histogram of the low
//   byte among that bin, give the k-th key exactly (each boundary from suffix sums in one
//   wave); every key at or above it is collected (for register-held rows from the keys of the
//   boundary bin and above, copied once into per-thread LDS regions; else by a pass over the
//   row) and a bitonic sort (in one wave's registers up to 64 candidates, else in LDS) orders
//   them (ties by id), so the first top_k are the answer.
//   When the boundary key repeats so often that the candidates overflow LDS, an ordered pass
//   ranks its ties by id instead. Histograms use 256 LDS sub-histograms (wave, lane % 16) of
//   16-bit counters, so lanes with equal keys rarely serialise on one counter.
// * logits_pipe_kernel: temperature, softmax and top-p renormalisation of one row in LDS.
// * sample_kernel / chain_kernel / verify_kernel: inverse-CDF draws with the uniforms given
//   (a contiguous chunk per thread, chunk sums scanned in thread order, so the prefix sums
//   are the same on every run), the chain speculative-sampling rule, and the reference's
//   top-k verification fused around it (local vocabulary of top_k + 1 built on the fly).
// One workgroup of 256 threads per row or request; these are per-token kernels (one decode
// step samples at most a few hundred rows), latency- rather than bandwidth-bound.
#include <cfloat>

#include "common.h"

namespace aspire {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxTopK = 1024;
constexpr int kMaxPipeWidth = 4096;

// Order-preserving 16-bit key of a bf16 value; -0 and +0 share a key (they compare equal, so
// they tie and fall back to the id order).
__device__ __forceinline__ uint32_t bf16_key(uint16_t b) {
  if (b == 0x8000u) b = 0;
  return (b & 0x8000u) ? (~uint32_t(b) & 0xffffu) : (uint32_t(b) | 0x8000u);
}

// The keys of two packed bf16 values at once (16-bit packed integer operations): negative
// values flip every bit, others set the sign bit, and -0 (whose flipped bits give 0x7fff, a key
// no other value has) moves up to +0's key 0x8000.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short i16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2_keys(uint32_t w) {
  const u16x2 b = __builtin_bit_cast(u16x2, w);
  const u16x2 sgn = __builtin_bit_cast(u16x2, __builtin_bit_cast(i16x2, b) >> 15);
  const u16x2 k = b ^ (sgn | (u16x2){0x8000, 0x8000});
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(k, (k + (u16x2){1, 1}) & (u16x2){0x8000, 0x8000}));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ int wave_min_int(int v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = min(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ int wave_max_int(int v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = max(v, __shfl_xor(v, m, 64));
  return v;
}

// Block-wide reductions (256 threads); every thread gets the result.
__device__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) s += red[w];
  return s;
}
__device__ float block_max(float v, float* red) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = -FLT_MAX;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) s = fmaxf(s, red[w]);
  return s;
}
__device__ int block_min_int(int v, int* red) {
  v = wave_min_int(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int s = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) s = min(s, red[w]);
  return s;
}
__device__ int block_max_int(int v, int* red) {
  v = wave_max_int(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int s = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) s = max(s, red[w]);
  return s;
}

// Shared scratch of the draw: the per-thread chunk sums, scanned in thread order by one
// thread (256 additions: the same association on every run).
struct DrawLds {
  float part[kThreads];
  float excl[kThreads];
  float total;
  int ired[kWaves];
  float fred[kWaves];
};

// Inverse-CDF draw over w(0..n-1) (weights >= 0, any scale): the first index whose inclusive
// prefix sum exceeds u * sum(w); the last positive index if rounding leaves none; 0 if all are 0.
// Thread t owns indices [t * chunk, (t + 1) * chunk). Every thread must call it.
template <typename W>
__device__ int block_draw(const W& w, int n, float u, DrawLds& s) {
  const int t = threadIdx.x;
  if (n <= 64) {
    // At most 64 weights: wave 0 alone, one weight per lane, the prefix sums added in index
    // order (as below: one index per thread, chunk sums scanned in thread order), the first hit
    // and the last positive index by ballots; the result reaches the other waves through LDS.
    if (t < 64) {
      const float x = t < n ? w(t) : 0.f;
      float acc = 0.f, incl = 0.f;
      for (int j = 0; j < n; ++j) {
        acc += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j));
        incl = t == j ? acc : incl;
      }
      const float target = u * acc;
      const uint64_t hits = __ballot(t < n && incl > target);
      const uint64_t pos = __ballot(t < n && x > 0.f);
      const int res = hits ? __builtin_ctzll(hits) : (pos ? 63 - __builtin_clzll(pos) : 0);
      if (t == 0) s.ired[0] = res;
    }
    __syncthreads();
    const int res = s.ired[0];
    __syncthreads();  // (a later call may rewrite it)
    return res;
  }
  const int chunk = (n + kThreads - 1) / kThreads;
  const int i0 = min(t * chunk, n), i1 = min(i0 + chunk, n);
  float sum = 0.f;
  int last_pos = -1;
  for (int i = i0; i < i1; ++i) {
    const float x = w(i);
    sum += x;
    if (x > 0.f) last_pos = i;
  }
  s.part[t] = sum;
  __syncthreads();
  if (t == 0) {
    float acc = 0.f;
    for (int j = 0; j < kThreads; ++j) {
      s.excl[j] = acc;
      acc += s.part[j];
    }
    s.total = acc;
  }
  __syncthreads();
  const float target = u * s.total;
  int hit = INT_MAX;
  if (i0 < i1 && s.excl[t] + s.part[t] > target) {
    // The chunk's own running sum, from 0 in the order of part[t]: at the chunk's end
    // excl + local equals excl + part (and the next chunk's excl) exactly, so a chunk whose
    // check passes hits inside itself, and a weight of 0 never raises excl + local to a hit.
    const float excl = s.excl[t];
    float local = 0.f;
    for (int i = i0; i < i1; ++i) {
      local += w(i);
      if (excl + local > target) {
        hit = i;
        break;
      }
    }
  }
  hit = block_min_int(hit, s.ired);
  if (hit != INT_MAX) return hit;
  const int lp = block_max_int(last_pos, s.ired);
  return lp >= 0 ? lp : 0;
}

// ------------------------------------------------------------------ top-k candidates
struct TopKParams {
  const uint16_t* logits;
  int64_t stride;
  int32_t vocab, k;
  int64_t vocab_start;
  uint16_t* values;  // [rows, k] bf16
  int64_t* ids;      // [rows, k]
};

constexpr int kTkThreads = 1024;                     // one workgroup of 16 waves per row
constexpr int kTkSubHists = (kTkThreads / 64) * 16;   // sub-histograms: (wave, lane % 16)
constexpr int kTkHistStride = 129;  // 128 dwords of two 16-bit counters, +1 so sub-histograms start on other banks
constexpr int kTkCandCap = 2048;    // candidates sorted in LDS
constexpr int kTkResident = 19;     // 16-byte vectors per thread held in registers (rows up to 155,648 logits)
constexpr int kTkMaxVocab = 16000000;  // keeps every 16-bit sub-histogram counter below 65,536
constexpr int kTkRegion = 16;           // per-thread candidate entries of a register-held row
static_assert(kTkRegion * kTkThreads * 8 <= kTkSubHists * kTkHistStride * 4, "regions fit the histograms' LDS");

template <bool kVec>
__global__ __launch_bounds__(kTkThreads) void topk_candidates_kernel(TopKParams p) {
  __shared__ uint32_t hist[kTkSubHists][kTkHistStride];
  __shared__ uint32_t bins[256];
  __shared__ uint32_t bin_part[4][256];
  __shared__ uint64_t cand[kTkCandCap];
  __shared__ int32_t sel[6];  // threshold key, count above, ties needed, candidates written, ties present,
                              // a region overflowed
  __shared__ int32_t tie_scan[kTkThreads];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int sub = (t >> 6) * 16 + (lane & 15);
  // bins 2j and 2j + 1 share dword j of a sub-histogram as its low and high 16 bits
  auto hadd = [&](uint32_t bin) { atomicAdd(&hist[sub][bin >> 1], (bin & 1) ? 0x10000u : 1u); };
  const uint16_t* row = p.logits + int64_t(blockIdx.x) * p.stride;
  const int V = p.vocab;
  const int kk = min(p.k, V);

  // Rows of up to kTkResident vectors per thread are read once: their keys stay in
  // registers (two 16-bit keys per dword) for all passes.
  uint32_t kr[kTkResident][4];
  const bool resident = kVec && (V >> 3) <= kTkResident * kTkThreads;
  if (resident) {
    const int nv = V >> 3;
    const uint4* rv = reinterpret_cast<const uint4*>(row);
#pragma unroll
    for (int j = 0; j < kTkResident; ++j) {
      const int v = t + j * kTkThreads;
      // slots past the row hold raw 0xffff (a negative NaN) in both halves, whose key is 0:
      // below every threshold of the search, never its maximum
      const uint4 w = v < nv ? rv[v] : make_uint4(~0u, ~0u, ~0u, ~0u);
      kr[j][0] = bf16x2_keys(w.x);
      kr[j][1] = bf16x2_keys(w.y);
      kr[j][2] = bf16x2_keys(w.z);
      kr[j][3] = bf16x2_keys(w.w);
    }
  }
  // f(i, key) over the row: from registers, else 16-byte loads (8 logits, four in flight per
  // thread) when rows are 16-byte aligned, else element loads
  auto for_each = [&](auto&& f) {
    const int nv = kVec ? V >> 3 : 0;
    if (resident) {
#pragma unroll
      for (int j = 0; j < kTkResident; ++j) {
        const int v = t + j * kTkThreads;
        if (v < nv) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            f(8 * v + 2 * e, kr[j][e] & 0xffffu);
            f(8 * v + 2 * e + 1, kr[j][e] >> 16);
          }
        }
      }
    } else if (kVec) {
      constexpr int kInFlight = 4;
      const uint4* rv = reinterpret_cast<const uint4*>(row);
      for (int v0 = t; v0 < nv; v0 += kInFlight * kTkThreads) {
        uint4 wv[kInFlight];
#pragma unroll
        for (int j = 0; j < kInFlight; ++j) {
          const int v = v0 + j * kTkThreads;
          if (v < nv) wv[j] = rv[v];
        }
#pragma unroll
        for (int j = 0; j < kInFlight; ++j) {
          const int v = v0 + j * kTkThreads;
          if (v < nv) {
            const uint32_t u[4] = {bf16x2_keys(wv[j].x), bf16x2_keys(wv[j].y), bf16x2_keys(wv[j].z),
                                   bf16x2_keys(wv[j].w)};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              f(8 * v + 2 * e, u[e] & 0xffffu);
              f(8 * v + 2 * e + 1, u[e] >> 16);
            }
          }
        }
      }
    }
    for (int i = (nv << 3) + t; i < V; i += kTkThreads) f(i, bf16_key(row[i]));
  };
  auto clear_hist = [&]() {
    for (int i = t; i < kTkSubHists * kTkHistStride; i += kTkThreads) (&hist[0][0])[i] = 0;
  };
  // bins[b] = sum over sub-histograms (each quarter of the threads sums a quarter of them)
  auto sum_hist = [&]() {
    {
      const int b = t & 255, q = t >> 8;
      uint32_t c = 0;
      for (int h = q * (kTkSubHists / 4); h < (q + 1) * (kTkSubHists / 4); ++h) c += hist[h][b >> 1];
      bin_part[q][b] = (b & 1) ? (c >> 16) : (c & 0xffffu);
    }
    __syncthreads();
    if (t < 256) bins[t] = bin_part[0][t] + bin_part[1][t] + bin_part[2][t] + bin_part[3][t];
  };
  // The boundary bin below `base` keys counted above the histogram: the largest b with
  // base + sum(bins[b..255]) >= kk (or 0), from suffix sums of 4 bins per lane of wave 0 and
  // one ballot; the lane holding it stores (b, keys above b[, keys in b]).
  auto boundary = [&](uint32_t base, int* out_bin, int* out_above, int* out_count) {
    const uint32_t c0 = bins[4 * lane], c1 = bins[4 * lane + 1], c2 = bins[4 * lane + 2], c3 = bins[4 * lane + 3];
    const uint32_t own = c0 + c1 + c2 + c3;
    uint32_t suf = own;  // sum over lanes >= lane
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t o = __shfl_down(suf, off);
      if (lane + off < 64) suf += o;
    }
    const uint32_t s3 = base + suf - own + c3, s2 = s3 + c2, s1 = s2 + c1, s0 = s1 + c0;
    const uint32_t need = uint32_t(kk);
    const int mine = s3 >= need ? 3 : s2 >= need ? 2 : s1 >= need ? 1 : s0 >= need ? 0 : -1;
    const uint64_t m = __ballot(mine >= 0);
    const int hl = m ? 63 - __builtin_clzll(m) : 0;
    if (lane == hl) {
      const int j = mine >= 0 ? mine : 0;
      const uint32_t sj = j == 3 ? s3 : j == 2 ? s2 : j == 1 ? s1 : s0;
      const uint32_t cj = j == 3 ? c3 : j == 2 ? c2 : j == 1 ? c1 : c0;
      *out_bin = 4 * lane + j;
      *out_above = int(sj - cj);
      if (out_count) *out_count = int(cj);
    }
  };

  // Pass 1: the boundary bin (high byte) of the k-th key and the keys above it. Rows held in
  // registers first try the top of the key range: the row's largest key (packed 16-bit max)
  // gives its high byte h, and counts of the keys at or above h, h - 1, h - 2 (packed
  // saturating subtract, min and add: about 1.5 instructions per key, no atomics) find the
  // boundary when it is one of those bins, as it nearly always is for logits. Otherwise, and
  // for streamed rows, the high-byte histogram.
  __shared__ uint32_t red[kTkThreads / 64];
  auto block_reduce = [&](uint32_t v, bool is_max) -> uint32_t {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const uint32_t o = __shfl_xor(v, m);
      v = is_max ? max(v, o) : v + o;
    }
    if (lane == 0) red[t >> 6] = v;
    __syncthreads();
    uint32_t acc = 0;
#pragma unroll
    for (int w = 0; w < kTkThreads / 64; ++w) acc = is_max ? max(acc, red[w]) : acc + red[w];
    __syncthreads();
    return acc;
  };
  bool found = false;
  if (resident) {
    const int nv = V >> 3;
    // (register slots past the row hold key 0: below every threshold, never the maximum)
    u16x2 mx2 = {0, 0};
#pragma unroll
    for (int j = 0; j < kTkResident; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(u16x2, kr[j][e]));
    uint32_t kmax = max(uint32_t(mx2.x), uint32_t(mx2.y));
    for (int i = (nv << 3) + t; i < V; i += kTkThreads) kmax = max(kmax, bf16_key(row[i]));
    kmax = block_reduce(kmax, true);
    int b = int(kmax >> 8);
    uint32_t above = 0;  // keys in bins above b
    for (int it = 0; it < 3 && b >= 1; ++it, --b) {
      const unsigned short tm1 = static_cast<unsigned short>((b << 8) - 1);
      const u16x2 thr2 = {tm1, tm1}, one2 = {1, 1};
      u16x2 acc2 = {0, 0};  // at most 76 keys per half
#pragma unroll
      for (int j = 0; j < kTkResident; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc2 += __builtin_elementwise_min(
              __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2, kr[j][e]), thr2), one2);
      uint32_t cnt = uint32_t(acc2.x) + uint32_t(acc2.y);
      for (int i = (nv << 3) + t; i < V; i += kTkThreads) cnt += bf16_key(row[i]) >= uint32_t(b << 8) ? 1u : 0u;
      cnt = block_reduce(cnt, false);
      if (cnt >= uint32_t(kk)) {
        found = true;
        if (t == 0) {
          sel[0] = b;
          sel[1] = int(above);
          bins[b] = cnt - above;  // the only bin read before the next histogram
        }
        break;
      }
      above = cnt;
    }
  }
  if (!found) {
    clear_hist();
    __syncthreads();
    for_each([&](int, uint32_t key) { hadd(key >> 8); });
    __syncthreads();
    sum_hist();
    __syncthreads();
    if (t < 64) boundary(0u, &sel[0], &sel[1], nullptr);
  }
  if (t == 64) sel[5] = 0;
  __syncthreads();
  const uint32_t hb = uint32_t(sel[0]);
  // Rows held in registers: one sweep copies every key of the boundary bin and above, with its
  // id, into the thread's own region of the histograms' LDS (kTkRegion entries; ids are strided
  // over threads, so a region holds about 1/1024 of them), and the low byte and the candidates
  // come from those entries instead of two more passes over the row. A region that overflows
  // sends the row down the passes below.
  uint64_t* const region = reinterpret_cast<uint64_t*>(&hist[0][0]) + t * kTkRegion;
  bool compact = resident && sel[1] + int(bins[hb]) <= kTkRegion * kTkThreads;
  int n_mine = 0;
  if (compact) {
    const uint32_t lo_key = hb << 8;
    for_each([&](int i, uint32_t key) {
      if (key >= lo_key) {
        if (n_mine < kTkRegion) region[n_mine] = (uint64_t(key) << 32) | uint64_t(0xffffffffu - uint32_t(i));
        ++n_mine;
      }
    });
    if (n_mine > kTkRegion) sel[5] = 1;
    __syncthreads();
    compact = sel[5] == 0;
  }
  if (compact) {
    // low byte among the boundary bin's entries (a few per thread: one histogram)
    if (t < 256) bins[t] = 0;
    __syncthreads();
    for (int j = 0; j < n_mine; ++j) {
      const uint32_t key = uint32_t(region[j] >> 32);
      if ((key >> 8) == hb) atomicAdd(&bins[key & 255], 1u);
    }
    __syncthreads();
  } else {
    // pass 2: low byte among keys in the boundary bin
    clear_hist();
    __syncthreads();
    for_each([&](int, uint32_t key) {
      if ((key >> 8) == hb) hadd(key & 255);
    });
    __syncthreads();
    sum_hist();
    __syncthreads();
  }
  if (t < 64) {
    const uint32_t base = uint32_t(sel[1]);
    __builtin_amdgcn_wave_barrier();
    boundary(base, &sel[0], &sel[1], &sel[4]);  // low byte, keys above it, keys equal to it
  }
  __syncthreads();
  if (t == 0) {
    sel[0] = int((hb << 8) | uint32_t(sel[0]));  // the k-th largest key
    sel[2] = kk - sel[1];                       // ties to take, lowest ids first
    sel[3] = 0;
  }
  __syncthreads();
  const uint32_t kth = uint32_t(sel[0]);
  const int ties = sel[2];
  // sort key: larger key first, then the lower id
  auto push = [&](int i, uint32_t key) {
    const int slot = atomicAdd(&sel[3], 1);
    cand[slot] = (uint64_t(key) << 32) | uint64_t(0xffffffffu - uint32_t(i));
  };
  int n_sort;
  if (sel[1] + sel[4] <= kTkCandCap) {
    // every key >= the k-th (from the regions, else pass 3); sorting puts the lowest-id ties first
    if (compact) {
      for (int j = 0; j < n_mine; ++j) {
        const uint64_t e = region[j];
        if (uint32_t(e >> 32) >= kth) cand[atomicAdd(&sel[3], 1)] = e;
      }
    } else {
      for_each([&](int i, uint32_t key) {
        if (key >= kth) push(i, key);
      });
    }
    n_sort = sel[1] + sel[4];
  } else {
    // many equal keys at the boundary: rank the ties in id order (a contiguous chunk per
    // thread, chunk counts scanned in thread order) and take only the first ones
    const int chunk = (V + kTkThreads - 1) / kTkThreads;
    const int i0 = min(t * chunk, V), i1 = min(i0 + chunk, V);
    int my_ties = 0;
    for (int i = i0; i < i1; ++i) my_ties += bf16_key(row[i]) == kth;
    tie_scan[t] = my_ties;
    __syncthreads();
    if (t == 0) {
      int acc = 0;
      for (int j = 0; j < kTkThreads; ++j) {
        const int c = tie_scan[j];
        tie_scan[j] = acc;
        acc += c;
      }
    }
    __syncthreads();
    int tie_rank = tie_scan[t];
    for (int i = i0; i < i1; ++i) {
      const uint32_t key = bf16_key(row[i]);
      bool take = key > kth;
      if (key == kth) take = tie_rank++ < ties;
      if (take) push(i, key);
    }
    n_sort = kk;
  }
  __syncthreads();
  int n2 = 1;
  while (n2 < n_sort) n2 <<= 1;
  for (int i = n_sort + t; i < n2; i += kTkThreads) cand[i] = 0;
  __syncthreads();
  if (n2 <= 64) {
    // bitonic sort of at most 64 candidates in one wave's registers, descending
    if (t < 64) {
      uint64_t x = lane < n2 ? cand[lane] : 0ull;
      for (int size = 2; size <= 64; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
          const uint32_t lo = __shfl_xor(uint32_t(x), stride), hi = __shfl_xor(uint32_t(x >> 32), stride);
          const uint64_t y = (uint64_t(hi) << 32) | lo;
          const bool keep_max = ((lane & size) == 0) == ((lane & stride) == 0);
          x = keep_max ? (x > y ? x : y) : (x < y ? x : y);
        }
      }
      if (lane < n2) cand[lane] = x;
    }
    __syncthreads();
  } else
  // bitonic sort in LDS, descending
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = t; i < n2; i += kTkThreads) {
        const int j = i ^ stride;
        if (j > i) {
          const bool desc = (i & size) == 0;
          const uint64_t a = cand[i], b = cand[j];
          if (desc ? a < b : a > b) {
            cand[i] = b;
            cand[j] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  uint16_t* vout = p.values + int64_t(blockIdx.x) * p.k;
  int64_t* iout = p.ids + int64_t(blockIdx.x) * p.k;
  for (int j = t; j < p.k; j += kTkThreads) {
    const uint32_t id = 0xffffffffu - uint32_t(cand[j] & 0xffffffffu);
    if (j < kk && id < uint32_t(V)) {  // (ids come from the row: the bound is a guard)
      vout[j] = row[id];  // the logit's own bits (a -0 stays -0)
      iout[j] = int64_t(id) + p.vocab_start;
    } else {
      vout[j] = 0xff80u;  // -inf, id 0: the reference's padding of a narrow shard
      iout[j] = 0;
    }
  }
}

// ------------------------------------------------------------------ logits pipe
struct PipeParams {
  const void* values;
  int32_t values_f32;
  int64_t stride;
  int32_t width;
  float inv_temperature;  // 1 when no temperature
  float top_p;            // >= 1: no top-p
  float* probs;
  int64_t out_stride;
};

__global__ __launch_bounds__(kThreads) void logits_pipe_kernel(PipeParams p) {
  __shared__ float prob[kMaxPipeWidth];
  __shared__ uint32_t srt[kMaxPipeWidth];
  __shared__ float red[kWaves];
  __shared__ float part[kThreads];
  __shared__ float cut_value;
  const int t = threadIdx.x;
  const int n = p.width;
  const int64_t r = blockIdx.x;
  if (n <= 64) {
    // At most 64 candidates (the top-k lists): one wave, one candidate per lane, everything in
    // registers with the same arithmetic in the same order as below (the other waves' shares
    // of the block reductions are the identities); no workgroup barrier.
    if (t >= 64) return;
    float x = -FLT_MAX, e = 0.f;
    if (t < n) {
      x = p.values_f32 ? static_cast<const float*>(p.values)[r * p.stride + t]
                       : __uint_as_float(uint32_t(static_cast<const uint16_t*>(p.values)[r * p.stride + t]) << 16);
      x *= p.inv_temperature;
    }
    const float wmx = fmaxf(-FLT_MAX, wave_max(x));
    if (t < n) e = wmx == -INFINITY ? 0.f : expf(x - wmx);
    const float wsum = wave_sum(e);
    const float winv = wsum > 0.f ? 1.f / wsum : 0.f;
    const float pr = e * winv;
    float* wout = p.probs + r * p.out_stride;
    if (!(p.top_p < 1.f)) {
      if (t < n) wout[t] = pr;
      return;
    }
    // descending bitonic sort of the probabilities' bits (non-negative floats order like
    // integers); lanes past n hold 0
    uint32_t v = t < n ? __float_as_uint(pr) : 0u;
    for (int size = 2; size <= 64; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        const uint32_t o = __shfl_xor(v, stride, 64);
        const bool keep_max = ((t & size) == 0) == ((t & stride) == 0);
        v = keep_max ? max(v, o) : min(v, o);
      }
    }
    // prefix sums in element order; the cut is the value where the prefix first reaches top_p
    // (the last value when none does)
    float acc = 0.f;
    uint32_t cut = uint32_t(__builtin_amdgcn_readlane(int(v), n - 1));
    for (int j = 0; j < n; ++j) {
      const float vj = __uint_as_float(uint32_t(__builtin_amdgcn_readlane(int(v), j)));
      const float prev = acc;
      acc += vj;
      if (acc >= p.top_p && prev < p.top_p) {
        cut = __float_as_uint(vj);
        break;
      }
    }
    const float thresh = __uint_as_float(cut);
    const float wkept = wave_sum(t < n && pr >= thresh ? pr : 0.f);
    const float wrk = wkept > 0.f ? 1.f / wkept : 0.f;
    if (t < n) wout[t] = pr >= thresh ? pr * wrk : 0.f;
    return;
  }
  float mx = -FLT_MAX;
  for (int i = t; i < n; i += kThreads) {
    float x = p.values_f32 ? static_cast<const float*>(p.values)[r * p.stride + i]
                           : __uint_as_float(uint32_t(static_cast<const uint16_t*>(p.values)[r * p.stride + i]) << 16);
    x *= p.inv_temperature;
    prob[i] = x;
    mx = fmaxf(mx, x);
  }
  mx = block_max(mx, red);
  float sum = 0.f;
  for (int i = t; i < n; i += kThreads) {
    const float e = mx == -INFINITY ? 0.f : expf(prob[i] - mx);
    prob[i] = e;
    sum += e;
  }
  sum = block_sum(sum, red);
  const float inv = sum > 0.f ? 1.f / sum : 0.f;
  for (int i = t; i < n; i += kThreads) prob[i] *= inv;
  __syncthreads();
  float* out = p.probs + r * p.out_stride;
  if (!(p.top_p < 1.f)) {
    for (int i = t; i < n; i += kThreads) out[i] = prob[i];
    return;
  }
  // sort the probabilities (non-negative: float bits order like integers), descending
  int n2 = 1;
  while (n2 < n) n2 <<= 1;
  for (int i = t; i < n2; i += kThreads) srt[i] = i < n ? __float_as_uint(prob[i]) : 0u;
  __syncthreads();
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = t; i < n2; i += kThreads) {
        const int j = i ^ stride;
        if (j > i) {
          const bool desc = (i & size) == 0;
          const uint32_t a = srt[i], b = srt[j];
          if (desc ? a < b : a > b) {
            srt[i] = b;
            srt[j] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  // prefix sums of the sorted values: a contiguous chunk per thread, chunk sums in thread order
  const int chunk = (n + kThreads - 1) / kThreads;
  const int i0 = min(t * chunk, n), i1 = min(i0 + chunk, n);
  float s = 0.f;
  for (int i = i0; i < i1; ++i) s += __uint_as_float(srt[i]);
  part[t] = s;
  __syncthreads();
  if (t == 0) {
    float acc = 0.f;
    for (int j = 0; j < kThreads; ++j) {
      const float c = part[j];
      part[j] = acc;
      acc += c;
    }
    cut_value = __uint_as_float(srt[n - 1]);  // no prefix reaches top_p: keep everything
  }
  __syncthreads();
  // The smallest prefix reaching top_p ends in exactly one thread's chunk: the prefix at i is
  // excl + local, local the chunk's own running sum from 0 in the order of its part, so at the
  // chunk's end it equals the next chunk's excl exactly and the prefixes never step back.
  {
    const float excl = part[t];
    float local = 0.f;
    float prev = excl;
    for (int i = i0; i < i1; ++i) {
      local += __uint_as_float(srt[i]);
      const float cur = excl + local;
      if (cur >= p.top_p && prev < p.top_p) cut_value = __uint_as_float(srt[i]);
      prev = cur;
    }
  }
  __syncthreads();
  const float thresh = cut_value;
  float kept = 0.f;
  for (int i = t; i < n; i += kThreads) kept += prob[i] >= thresh ? prob[i] : 0.f;
  kept = block_sum(kept, red);
  const float rk = kept > 0.f ? 1.f / kept : 0.f;
  for (int i = t; i < n; i += kThreads) out[i] = prob[i] >= thresh ? prob[i] * rk : 0.f;
}

// ------------------------------------------------------------------ draws
__global__ __launch_bounds__(kThreads) void sample_kernel(const float* probs, int64_t stride, int32_t vocab,
                                                          const float* uniforms, int32_t* out) {
  __shared__ DrawLds s;
  const float* row = probs + int64_t(blockIdx.x) * stride;
  const int idx = block_draw([&](int i) { return row[i]; }, vocab, uniforms[blockIdx.x], s);
  if (threadIdx.x == 0) out[blockIdx.x] = idx;
}

struct ChainParams {
  const float* draft_probs;      // [R, D, V]
  const int32_t* draft_ids;      // [R, D]
  const float* target_probs;     // [R, D + 1, V]
  const float* uniforms;         // [R, D + 1]
  int32_t num_spec, vocab;
  int32_t* output;               // [R, D + 1]
  int32_t* accepted;             // [R] or null
  int32_t* emitted;              // [R]
};

__global__ __launch_bounds__(kThreads) void chain_kernel(ChainParams p) {
  __shared__ DrawLds s;
  __shared__ int stop;
  const int64_t r = blockIdx.x;
  const int D = p.num_spec, V = p.vocab;
  const float* q = p.draft_probs + r * D * V;
  const float* pt = p.target_probs + r * (D + 1) * V;
  const float* u = p.uniforms + r * (D + 1);
  const int32_t* x = p.draft_ids + r * D;
  if (threadIdx.x == 0) {
    int j = D, acc = 0;
    for (int i = 0; i < D; ++i) {
      const int xi = min(max(x[i], 0), V - 1);
      const bool ok = u[i] * q[int64_t(i) * V + xi] < pt[int64_t(i) * V + xi];
      acc += ok;
      if (!ok && j == D) j = i;
    }
    stop = j;
    if (p.accepted) p.accepted[r] = acc;
    p.emitted[r] = j;
  }
  __syncthreads();
  const int j = stop;
  const float* pj = pt + int64_t(j) * V;
  const float* qj = q + int64_t(min(j, D - 1)) * V;
  float wsum = 0.f;
  for (int i = threadIdx.x; i < V; i += kThreads) wsum += j < D ? fmaxf(pj[i] - qj[i], 0.f) : pj[i];
  wsum = block_sum(wsum, s.fred);
  const bool residual = j < D && wsum > 0.f;
  const int tok = block_draw([&](int i) { return residual ? fmaxf(pj[i] - qj[i], 0.f) : pj[i]; }, V, u[D], s);
  int32_t* out = p.output + r * (D + 1);
  for (int i = threadIdx.x; i <= D; i += kThreads) out[i] = i < j ? x[i] : (i == j ? tok : -1);
}

// The reference's top-k verification (aspire/engine/sampling.py:46-98) in one launch: the
// chain rule over a local vocabulary of top_k + 1 entries built on the fly. Local entry
// v < K of position i is the target's candidate v; entry K stands for "a token outside the
// target's top-k". Draft probabilities map onto the target's candidates by id (ids are unique
// within a row, so each entry takes at most one term).
struct VerifyParams {
  const float* draft_probs;    // [R, D, K]
  const int64_t* draft_ids;    // [R, D, K]
  const int32_t* draft_tokens; // [R, D]
  const int32_t* draft_counts; // [R]
  const float* target_probs;   // [R, D + 1, K]
  const int64_t* target_ids;   // [R, D + 1, K]
  const float* uniforms;       // [R, D + 1]
  int32_t num_spec, top_k;
  int64_t* output;             // [R, D + 1]
  int32_t* emitted;            // [R]
};

__global__ __launch_bounds__(kThreads) void verify_kernel(VerifyParams p) {
  __shared__ DrawLds s;
  __shared__ int local_tok[64];
  __shared__ float qx[64];
  __shared__ float px[64];
  __shared__ float wres[kMaxTopK + 1];
  __shared__ float pj_l[kMaxTopK + 1];
  __shared__ int64_t qid[kMaxTopK];  // position j's draft ids, sorted by (id, index)
  __shared__ int32_t qidx[kMaxTopK];
  __shared__ int stop;
  const int64_t r = blockIdx.x;
  const int D = p.num_spec, K = p.top_k;
  const int n = p.draft_counts[r];
  const float* dp = p.draft_probs + r * D * K;
  const int64_t* di = p.draft_ids + r * D * K;
  const float* tp = p.target_probs + r * (D + 1) * K;
  const int64_t* ti = p.target_ids + r * (D + 1) * K;
  const float* u = p.uniforms + r * (D + 1);
  // wave i handles position i: local token and its local draft probability
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int i = wave; i < D; i += kWaves) {
    const int64_t tok = p.draft_tokens[r * D + i];
    int first = INT_MAX;
    for (int v = lane; v < K; v += 64)
      if (ti[int64_t(i) * K + v] == tok) first = min(first, v);
    first = wave_min_int(first);
    const bool valid = i < n;
    const int lt = (valid && first != INT_MAX) ? first : K;
    // draft probability of the local token's id (the target's candidate, or the draft token)
    const int64_t want = lt < K ? ti[int64_t(i) * K + lt] : tok;
    float qsum = 0.f;
    for (int m = lane; m < K; m += 64) qsum += di[int64_t(i) * K + m] == want ? dp[int64_t(i) * K + m] : 0.f;
    qsum = wave_sum(qsum);
    if (lane == 0) {
      local_tok[i] = lt;
      qx[i] = valid ? qsum : 1.f;
      // the target probability of the local token, requested here for every position at once
      px[i] = (lt < K && i <= n) ? tp[int64_t(i) * K + lt] : 0.f;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int j = D;
    for (int i = 0; i < D; ++i) {
      const float pv = px[i];
      if (!(u[i] * qx[i] < pv)) {
        j = i;
        break;
      }
    }
    stop = j;
  }
  __syncthreads();
  const int j = stop;
  // local distributions at position j: target P (masked past the draft count), draft Q
  const bool pj_ok = j <= n;
  auto P = [&](int v) { return (v < K && pj_ok) ? tp[int64_t(j) * K + v] : 0.f; };
  // Q(v): the draft probability of the target's candidate v, the sum of dp[j, m] over the
  // draft entries m with that id, in ascending m. The draft's (id, m) pairs of position j are
  // sorted once in LDS (bitonic, padding sorts last), so each candidate finds its first pair by
  // binary search and adds its pairs in m order: O(K log K) per request instead of a scan of
  // all K draft ids per candidate.
  const bool need_q = j < D && j < n;  // block-uniform
  if (need_q) {
    int n2 = 1;
    while (n2 < K) n2 <<= 1;
    for (int m = threadIdx.x; m < n2; m += kThreads) {
      qid[m] = m < K ? di[int64_t(j) * K + m] : INT64_MAX;
      qidx[m] = m;
    }
    __syncthreads();
    for (int size = 2; size <= n2; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int a = threadIdx.x; a < n2; a += kThreads) {
          const int b = a ^ stride;
          if (b > a) {
            const bool up = (a & size) == 0;
            const int64_t ia = qid[a], ib = qid[b];
            const int32_t ma = qidx[a], mb = qidx[b];
            const bool a_after = ia > ib || (ia == ib && ma > mb);
            if (a_after == up) {
              qid[a] = ib;
              qid[b] = ia;
              qidx[a] = mb;
              qidx[b] = ma;
            }
          }
        }
        __syncthreads();
      }
    }
  }
  auto Q = [&](int v) -> float {
    if (v >= K || !need_q) return 0.f;  // entry K only ever lowers max(P - Q, 0), which is 0 there
    const int64_t id = ti[int64_t(j) * K + v];
    int lo = 0, hi = K;  // first sorted pair with id >= the candidate's
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (qid[mid] < id) lo = mid + 1;
      else hi = mid;
    }
    float q = 0.f;
    for (int i = lo; i < K && qid[i] == id; ++i) q += dp[int64_t(j) * K + qidx[i]];
    return q;
  };
  // P and the residual max(P - Q, 0) at position j, each computed once into LDS
  float wsum = 0.f;
  for (int v = threadIdx.x; v <= K; v += kThreads) {
    const float pv = P(v);
    pj_l[v] = pv;
    if (j < D) {
      const float w = fmaxf(pv - Q(v), 0.f);
      wres[v] = w;
      wsum += w;
    }
  }
  wsum = block_sum(wsum, s.fred);
  const bool residual = j < D && wsum > 0.f;
  const int lt = block_draw([&](int v) { return residual ? wres[v] : pj_l[v]; }, K + 1, u[D], s);
  const int emitted = min(j, n);
  int64_t* out = p.output + r * (D + 1);
  for (int i = threadIdx.x; i <= D; i += kThreads) {
    const int l = i < j ? local_tok[i] : (i == j ? lt : -1);
    out[i] = (l >= 0 && l < K && i <= emitted) ? ti[int64_t(i) * K + l] : -1;
  }
  if (threadIdx.x == 0) p.emitted[r] = emitted;
}

}  // namespace
}  // namespace aspire

extern "C" int aspire_topk_candidates(const void* logits, int64_t stride, int32_t rows, int32_t vocab, int32_t top_k,
                                      int64_t vocab_start, void* values, int64_t* ids, void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(rows >= 0 && vocab >= 1 && top_k >= 1 && top_k <= kMaxTopK, "need vocab >= 1, 1 <= top_k <= 1024");
  ASPIRE_CHECK_ARG(vocab <= kTkMaxVocab && stride >= vocab, "need vocab <= 16,000,000 and stride >= vocab");
  if (rows == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(logits && values && ids, "null pointer");
  TopKParams p{static_cast<const uint16_t*>(logits), stride, vocab, top_k, vocab_start,
               static_cast<uint16_t*>(values), ids};
  const bool vec = (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && stride % 8 == 0;
  if (vec)
    hipLaunchKernelGGL(topk_candidates_kernel<true>, dim3(rows), dim3(kTkThreads), 0, static_cast<hipStream_t>(stream), p);
  else
    hipLaunchKernelGGL(topk_candidates_kernel<false>, dim3(rows), dim3(kTkThreads), 0, static_cast<hipStream_t>(stream), p);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}

extern "C" int aspire_logits_pipe(const void* values, int32_t values_dtype, int64_t stride, int32_t rows, int32_t width,
                                  float temperature, float top_p, float* probs, int64_t out_stride, void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(rows >= 0 && width >= 1 && width <= kMaxPipeWidth, "width must be in [1, 4096]");
  ASPIRE_CHECK_ARG(values_dtype == 0 || values_dtype == 1, "values_dtype must be 0 (bf16) or 1 (fp32)");
  ASPIRE_CHECK_ARG(stride >= width && out_stride >= width, "bad row strides");
  if (rows == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(values && probs, "null pointer");
  PipeParams p{values, values_dtype, stride, width, temperature > 0.f ? 1.f / temperature : 1.f,
               (top_p > 0.f && top_p < 1.f) ? top_p : 2.f, probs, out_stride};
  hipLaunchKernelGGL(logits_pipe_kernel, dim3(rows), dim3(kThreads), 0, static_cast<hipStream_t>(stream), p);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}

extern "C" int aspire_sampling_from_probs(const float* probs, int64_t stride, int32_t rows, int32_t vocab,
                                          const float* uniforms, int32_t* out, void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(rows >= 0 && vocab >= 1 && stride >= vocab, "bad vocab / row stride");
  if (rows == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(probs && uniforms && out, "null pointer");
  hipLaunchKernelGGL(sample_kernel, dim3(rows), dim3(kThreads), 0, static_cast<hipStream_t>(stream), probs, stride,
                     vocab, uniforms, out);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}

extern "C" int aspire_chain_speculative_sampling(const float* draft_probs, const int32_t* draft_token_ids,
                                                 const float* target_probs, int32_t rows, int32_t num_spec,
                                                 int32_t vocab, const float* uniforms, int32_t* output_token_ids,
                                                 int32_t* accepted_num, int32_t* emitted_num, void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(rows >= 0 && num_spec >= 1 && vocab >= 1, "need num_spec >= 1 and vocab >= 1");
  if (rows == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(draft_probs && draft_token_ids && target_probs && uniforms && output_token_ids && emitted_num,
                   "null pointer");
  ChainParams p{draft_probs, draft_token_ids, target_probs, uniforms, num_spec, vocab, output_token_ids, accepted_num,
                emitted_num};
  hipLaunchKernelGGL(chain_kernel, dim3(rows), dim3(kThreads), 0, static_cast<hipStream_t>(stream), p);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}

extern "C" int aspire_verify_topk_speculation(const float* draft_probs, const int64_t* draft_ids,
                                              const int32_t* draft_tokens, const int32_t* draft_counts,
                                              const float* target_probs, const int64_t* target_ids,
                                              const float* uniforms, int32_t requests, int32_t max_draft,
                                              int32_t top_k, int64_t* output, int32_t* emitted, void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(requests >= 0 && max_draft >= 1 && max_draft <= 64 && top_k >= 1 && top_k <= kMaxTopK,
                   "need 1 <= max_draft <= 64 and 1 <= top_k <= 1024");
  if (requests == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(draft_probs && draft_ids && draft_tokens && draft_counts && target_probs && target_ids &&
                       uniforms && output && emitted,
                   "null pointer");
  VerifyParams p{draft_probs, draft_ids, draft_tokens, draft_counts, target_probs, target_ids, uniforms,
                 max_draft, top_k, output, emitted};
  hipLaunchKernelGGL(verify_kernel, dim3(requests), dim3(kThreads), 0, static_cast<hipStream_t>(stream), p);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}
