// Shared host/device helpers for libaspire_hip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/aspire_hip.h"

namespace aspire {

// ---------------------------------------------------------------- errors --
void set_error(const char* fmt, ...);
const char* last_error();

inline int fail(int code, const char* msg) {
  set_error("%s", msg);
  return code;
}

#define ASPIRE_CHECK_ARG(cond, msg)                         \
  do {                                                      \
    if (!(cond)) {                                          \
      ::aspire::set_error("%s: %s", __func__, msg);         \
      return ASPIRE_ERR_INVALID;                            \
    }                                                       \
  } while (0)

#define ASPIRE_CHECK_HIP(expr)                                                   \
  do {                                                                           \
    hipError_t _e = (expr);                                                      \
    if (_e != hipSuccess) {                                                      \
      ::aspire::set_error("%s: %s failed: %s", __func__, #expr, hipGetErrorString(_e)); \
      return ASPIRE_ERR_HIP;                                                     \
    }                                                                            \
  } while (0)

#define ASPIRE_CHECK_LAUNCH()                                                    \
  do {                                                                           \
    hipError_t _e = hipGetLastError();                                           \
    if (_e != hipSuccess) {                                                      \
      ::aspire::set_error("%s: kernel launch failed: %s", __func__, hipGetErrorString(_e)); \
      return ASPIRE_ERR_HIP;                                                     \
    }                                                                            \
  } while (0)

// ------------------------------------------------------------ constants --
constexpr int kHeadDim = 128;
constexpr int kPage = 16;
constexpr int kMaxRowTiles = 3;  // q_len * group <= 48
#ifndef ASPIRE_ATTN_WAVES_PER_BLOCK
#define ASPIRE_ATTN_WAVES_PER_BLOCK 4
#endif
// Waves per attention workgroup. The planner gives each group of num_kv_heads
// consecutive waves the same pages (one wave per kv head); with 4 waves per
// workgroup a group of 8 kv heads spans two workgroups dispatched together
// (8-wave workgroups measured no faster and constrain occupancy).
constexpr int kAttnWavesPerBlock = ASPIRE_ATTN_WAVES_PER_BLOCK;

// Work item of the attention plan (8 x int32, read with scalar loads).
struct WorkItem {
  int32_t q_start;      // first token of the row in q / out
  int32_t q_len;        // tokens of the row (| kItemDirect)
  int32_t kv_len;       // tokens in the row's (or segment's) page list
  int32_t list_base;    // kv_indices offset where the list starts
  int32_t page_begin;   // page range [page_begin, page_end) of this piece
  int32_t page_end;
  int32_t bg;           // (row << 8) | kv_head
  int32_t partial_row;  // first fp32 partial row, or -1 for a final write
};

// Set in WorkItem::q_len (above the token count) for items of a head-aligned
// plan whose kv heads read different page lists: those items load their own
// head's rows instead of staging shared pages through LDS.
constexpr int32_t kItemDirect = 1 << 16;

// Rows [row_begin, row_begin + row_count) of a split (row, kv head) segment whose pieces
// are merged (8 x int32). A segment with more pieces than one round of the merge kernel's
// loads (kMergeChunk) is cut into row ranges of at most kMergeRows / s rows, s = 2 or 4, so
// that s lane groups can share each row's pieces within the kernel's task budget.
struct MergeItem {
  int32_t q_start;
  int32_t q_len;
  int32_t bg;
  int32_t first_partial_row;
  int32_t num_pieces;
  int32_t rows;         // q_len * group; partials of piece i start at first + i*rows
  int32_t row_begin;
  int32_t row_count;
};
constexpr int kMergeRows = 16 * kMaxRowTiles;  // rows of one merge item at most
constexpr int kMergeChunk = 8;                 // pieces per round of a lane's merge loads

// Piece groups per row for a merge item of `pieces` pieces and `row_count` rows (1, 2 or 4).
__host__ __device__ inline int merge_piece_groups(int pieces, int row_count) {
  int s = 1;
  if (pieces > kMergeChunk && 2 * row_count <= kMergeRows) s = 2;
  if (pieces > 2 * kMergeChunk && 4 * row_count <= kMergeRows) s = 4;
  return s;
}

// Fixed offsets (int32 units) of the plan in the int workspace.
struct PlanOffsets {
  int64_t header;        // [0]=items c0, [1]=c1, [2]=c2, [3]=num_merge, [4]=kv heads per slot
  int64_t indptr[3];     // num_waves + 1 entries each
  int64_t items[3];      // max_items WorkItems each
  int64_t merge;         // max_merge MergeItems
  int64_t total;         // int32 count
};

inline PlanOffsets plan_offsets(const aspire_plan_layout& L) {
  PlanOffsets o;
  o.header = 0;
  int64_t cur = 32;
  for (int c = 0; c < 3; ++c) {
    o.indptr[c] = cur;
    cur += L.num_waves + 1;
  }
  cur = (cur + 7) & ~int64_t(7);
  for (int c = 0; c < 3; ++c) {
    o.items[c] = cur;
    cur += int64_t(L.max_items) * 8;
  }
  o.merge = cur;
  cur += int64_t(L.max_merge) * 8;
  o.total = cur;
  return o;
}

// ------------------------------------------------------- device helpers --
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;

__device__ __forceinline__ f32x4 mfma_16x16x32_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_16x16x16_bf16(i16x4 a, i16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// fp32 -> bf16 with round-to-nearest-even (finite inputs).
__device__ __forceinline__ uint32_t bf16_rne_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
// Two fp32 values rounded to nearest-even bf16 in one instruction
// (v_cvt_pk_bf16_f32); equal to bf16_rne_bits on every finite input.
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}
// fp32 values that are exactly representable in bf16: keep the upper halves.
__device__ __forceinline__ uint32_t pack_bf16x2_exact(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

__device__ __forceinline__ int wave_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Cross-row reductions of a 64-lane wave without LDS. permlane32_swap(v, v)
// returns (v[l % 32], v[l % 32 + 32]) and permlane16_swap(v, v) returns the
// values of rows (2k, 2k + 1) of 16 lanes for both rows of that pair, so
// combining the pair equals combining v with v[l ^ 32] (v[l ^ 16]).
__device__ __forceinline__ float max_xor32(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float max_xor16(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float add_xor32(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float add_xor16(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
// Sum of an int over the 64 lanes, all in VALU: DPP quad permutes (xor 1,
// xor 2), row_half_mirror and row_mirror (they pair quad q with 1 - q and
// half h with 1 - h once those are uniform), then the permlane swaps.
__device__ __forceinline__ int wave_sum_int(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
  const auto p16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = int(p16[0]) + int(p16[1]);
  const auto p32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  v = int(p32[0]) + int(p32[1]);
  return __builtin_amdgcn_readfirstlane(v);
}
// Sum of a float over the 64 lanes (same DPP / permlane steps as wave_sum_int).
__device__ __forceinline__ float wave_sum_f(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  return add_xor32(add_xor16(v));
}

// Paged append position of token tok (FlashInfer get_seq_lens +
// get_batch_indices_positions, restated): the last row b with
// append_indptr[b] <= tok owns it; with seq_len the row's cached tokens after
// the append, the token sits at ps = tok + seq_len - append_indptr[b + 1].
// Writes the page-list entry (kv_indptr[b] + ps / page) and the slot; false
// when the reference skips the token (no row, negative position, empty row,
// or past the row's length).
// Last i in [0, n) with a[i] <= x for a non-decreasing a, or -1; wave-uniform. Every lane of
// the wave must call it with the same arguments: lanes load 64 consecutive entries per round
// trip and one ballot finds the boundary (a binary search would chain ~log2(n) dependent loads).
__device__ __forceinline__ int wave_last_le(const int32_t* a, int n, int x) {
  const int lane = threadIdx.x & 63;
  int found = -1;
  for (int base = 0; base < n; base += 64) {
    const int i = base + lane;
    const uint64_t m = __ballot(i < n && a[i] <= x);  // a prefix of the chunk's lanes
    if (m) found = base + 63 - __builtin_clzll(m);
    if (m != ~uint64_t(0)) break;  // an entry above x, or the array's end, is in this chunk
  }
  return __builtin_amdgcn_readfirstlane(found);
}

// Called by every lane of the wave (wave_last_le).
__device__ __forceinline__ bool append_locate(const int32_t* append_indptr, int num_seq, const int32_t* kv_indptr,
                                              const int32_t* last_page_len, int page_size, int tok, int& entry,
                                              int& slot) {
  // last b in [0, num_seq) with append_indptr[b] <= tok (indptr is
  // non-decreasing, so an empty row never shadows the row that owns tok)
  const int b = wave_last_le(append_indptr, num_seq, tok);
  if (b < 0) return false;
  const int end = append_indptr[b + 1];
  if (tok >= end) return false;  // covered by no row: default position -1
  const int start_page = kv_indptr[b];
  const int page_count = kv_indptr[b + 1] - start_page;
  const int last = last_page_len[b];
  const int seq_len = max(page_count - 1, 0) * page_size + last;
  const int ps = tok + seq_len - end;
  if (ps < 0 || page_count == 0) return false;
  if (ps >= (page_count - 1) * page_size + last) return false;
  entry = start_page + ps / page_size;
  slot = ps % page_size;
  return true;
}

// v[l ^ 1] and v[l ^ 2] through DPP quad permutes ([1,0,3,2] and [2,3,0,1]).
__device__ __forceinline__ float dpp_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_xor2(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
}

}  // namespace aspire
