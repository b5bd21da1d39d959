// (a4, a5, a6) Mixed draft/verify paged attention for gfx950.
//
// One wave processes one (row, kv head) segment piece at a time: all
// q_len * group query rows of the GQA group against a contiguous range of
// the segment's 16-token pages. Per page and lane (r = lane % 16 selects a
// key / query row, grp = lane / 16 a group of 8-dim slices):
//   * K and V reach the lane as 4 x 128 bits of key r: dims 32c + 8grp
//     (c = 0..3), either staged through LDS by the workgroup (head-aligned
//     plans: 1 KiB contiguous row loads, see run_item) or loaded directly
//     (16 rows x 64 B per instruction);
//   * S^T = K . Q^T with 4 v_mfma_f32_16x16x32_bf16 (A = K rows straight from
//     registers, B = the row's Q slice; the MFMA sums over k in any order both
//     operands agree on, so the lane slices need no shuffle). Lane holds
//     S^T[key 4*grp + i][row r], which is already the B operand layout of the
//     P.V product;
//   * V is transposed in registers by an exact MFMA against the identity
//     (8 x v_mfma_f32_16x16x16_bf16): lane then holds V[keys 4*grp..+3][dim]
//     as the A operand of O^T = V^T . P^T, and the O^T accumulator of lane l
//     covers row r and its own 32 output dims;
//   * online softmax in fp32 with exp2 and a base-2 LSE; the row max is
//     reduced across the 4 lane groups with permlane swaps (no LDS).
// A row tile is 16 query rows; NT tiles share the K/V registers
// (q_len * group <= 16 * NT). One persistent launch runs every class.
#include <mutex>
#include <type_traits>

#include "common.h"

namespace aspire {
namespace {

struct AttnParams {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* cache;
  int64_t c_sp, c_skv, c_st, c_sh;
  const int32_t* kv_indices;
  uint16_t* out;
  int64_t o_st, o_sh;
  float* lse;
  const int32_t* plan;
  int64_t indptr_off[3], items_off[3];
  int class_mask;
  int32_t num_waves;
  float* part_o;
  float* part_lse;
  int32_t hq, hkv, group;
  float scale_log2;
  int32_t causal;
  void* dump;
  int32_t dump_kind, dump_f32, dump_vec;
  int64_t dump_stride;
  int32_t dump_heads;
  const int32_t* dump_flags;
  float* page_scores;
  int64_t ps_stride;
  int32_t staged_ok;  // cache layout allows workgroup-staged K/V (see run_item)
};

struct MergeParams {
  const int32_t* plan;
  int64_t merge_off;
  const float* part_o;
  const float* part_lse;
  uint16_t* out;
  int64_t o_st, o_sh;
  float* lse;
  int32_t hq, group;
  int32_t max_merge;  // merge items the plan region holds
};

constexpr float kNegInf = -__builtin_huge_valf();

#ifndef ASPIRE_DIM_MAP
#define ASPIRE_DIM_MAP 1
#endif
// The 1-tile class streams K/V with non-temporal loads (measured slightly
// faster for it, and slower for the 2- and 3-tile classes).
#ifndef ASPIRE_NT1_NTLOADS
#define ASPIRE_NT1_NTLOADS 1
#endif
#ifndef ASPIRE_TILE_LANES
#define ASPIRE_TILE_LANES 2
#endif
// Registers: at most two waves per SIMD (256 VGPRs), or one per tile lane when there are more.
#ifndef ASPIRE_ATTN_WAVES_PER_EU
#define ASPIRE_ATTN_WAVES_PER_EU (ASPIRE_TILE_LANES > 2 ? ASPIRE_TILE_LANES : 2)
#endif
#ifndef ASPIRE_STAGED
#define ASPIRE_STAGED 1
#endif
// Row-tile classes (1..3) whose items use the staged path. The 3-tile class
// keeps direct loads: its query fragments and accumulators leave no registers
// for the staging buffer (it spills, and measured slower).
#ifndef ASPIRE_STAGED_MAX_NT
#define ASPIRE_STAGED_MAX_NT 2
#endif

// Items of at most 4 query rows (one token's GQA group of 4, a draft row) on VALU
// v_dot2 / DPP reductions instead of MFMA. Off by default: see the A/B of the two
// paths in the counter profiles of the attention kernel.
#ifndef ASPIRE_DRAFT_VALU
#define ASPIRE_DRAFT_VALU 0
#endif
constexpr int kValuRows = 4;

// Online softmax of the MFMA rows with a slack of ASPIRE_ATTN_SLACK log2 units (0: the exact
// running max on every page). With a slack, a row's max moves only when a key exceeds it by
// more than the slack (exponentials stay below 2^slack), and a page's exponentials are first
// taken with the current offsets: the row maxima (two cross-lane exchanges), the rescale and a
// second pass of exponentials run only on an item's first page (which holds a visible key of
// every row that has one in the item) and on pages where some lane's sum of its exponentials
// of a row exceeds 2^slack (a wave-uniform branch). Measured on MI355X: 3-tile items 5% faster,
// config 1 and config 4 0.5-1.4%.
#ifndef ASPIRE_ATTN_SLACK
#define ASPIRE_ATTN_SLACK 8
#endif
#if ASPIRE_ATTN_SLACK
constexpr float kAttnSumLimit = float(1 << ASPIRE_ATTN_SLACK);  // 2^slack
#endif

// Split-KV partial rows: plain stores, or non-temporal ones in the kernel instance the host
// launches for short plans (aspire_attention_args.partial_nt: at most 64 page-heads per wave).
// Measured on MI355X at config 4 f = 1.0 (32 page-heads per wave): 44.5 against 45.0 us;
// long launches measured 0.2% slower with non-temporal partials, so they keep plain stores.
template <bool kNt>
__device__ __forceinline__ void store_partial4(float* dst, float a, float b, float c, float d) {
  if constexpr (kNt) {
    f32x4 v;
    v[0] = a;
    v[1] = b;
    v[2] = c;
    v[3] = d;
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(dst));
  } else {
    *reinterpret_cast<float4*>(dst) = make_float4(a, b, c, d);
  }
}

// Tile lanes. A workgroup holds kAttnWavesPerBlock kv heads (the plan's waves) x kTileLanes
// waves: the tile lanes of a head share that head's item list, and lane tl computes the
// 16-row tiles [tl * k, min((tl + 1) * k, tiles)) of an item of `tiles` tiles, with
// k = ceil(tiles / kTileLanes). At 3 lanes no wave carries more than one tile: a 33-48-row
// item's three tiles run on three waves of one SIMD, whose MFMA -> softmax -> MFMA chains
// interleave, instead of one wave's chain three tiles long. Every wave of a workgroup helps
// stage the slot's pages; waves with no tile of an item only stage. Wave w of a workgroup
// is tile lane w / kAttnWavesPerBlock of head lane w % kAttnWavesPerBlock.
constexpr int kTileLanes = ASPIRE_TILE_LANES;
static_assert(kTileLanes >= 1 && kTileLanes <= kMaxRowTiles, "1 to 3 tile lanes");
constexpr int kWgWaves = kAttnWavesPerBlock * kTileLanes;

// Workgroup-staged K/V (head-aligned plans): LDS per workgroup, two buffers x {K, V} x 16
// key rows x 1 KiB (the rows' 4 heads), in uint4. A page's 32 row-halves (16 K rows, 16 V
// rows) are loaded by the workgroup's waves in blocks of kStagePerWave.
constexpr int kStageRowChunks = 64;                      // 16-byte chunks per 1 KiB row-half
constexpr int kStageKv = 16 * kStageRowChunks;           // one of K / V
constexpr int kStageBuf = 2 * kStageKv;                  // one buffer
constexpr int kStageChunks = 2 * kStageBuf;              // 64 KiB
constexpr int kStageRowHalves = 32;
// Row-tile classes of at least ASPIRE_SPLIT_MIN_TILES tiles are split over the tile lanes;
// smaller items are computed by tile lane 0 alone (the other lanes only take the barriers).
#ifndef ASPIRE_SPLIT_MIN_TILES
#define ASPIRE_SPLIT_MIN_TILES 3
#endif
// Tile lanes whose waves load the staged pages of a split item (lane 0 alone stages the others).
#ifndef ASPIRE_SPLIT_STAGE_LANES
#define ASPIRE_SPLIT_STAGE_LANES 1
#endif
static_assert(kAttnWavesPerBlock == 4, "staged K/V assumes 4 kv heads per workgroup");
// Per-head-lane page scores of the key-mean epilogue (64 pages, fp32), after the stage buffers.
constexpr int kScoreChunks = kAttnWavesPerBlock * 64 / 4;
// One 1 KiB row that the staging slots past the page's 32 row-halves write (their loads use
// the out-of-range offset and return zeros): every wave issues the same straight-line loads
// and stores, since loads under a per-slot branch made the compiler wait for every load in
// flight (vmcnt(0)) before each of them.
constexpr int kDummyChunks = kStageRowChunks;
constexpr int kLdsChunks = kStageChunks + kScoreChunks + kDummyChunks;
// V^T of staged items: transpose reads from LDS (ds_read_b64_tr_b16) for waves that compute
// at least this many tiles of an item, and for every wave of a split item; the others read V
// rows and transpose them with the identity MFMA (measured faster for 1-tile items at one
// computing wave per SIMD).
#ifndef ASPIRE_VT_READ_MIN_NT
#define ASPIRE_VT_READ_MIN_NT 2
#endif

// LDS row swizzle: 16-byte chunk c of key row r is stored at chunk c ^ swz(r); swz swaps
// the two 2-bit halves of r. Whole-row writes (one row, 64 consecutive chunks) are
// conflict-free; the 16-row column reads of the MFMA operand layout (rows 0..15, chunk
// 4c + grp) and the transpose reads of V^T (rows 4grp + 0..3) measure pairwise bank
// conflicts on gfx950 (8 and 4 cycles per read where 4 and 2 are possible). Placements that
// remove them (c ^ r for column reads; c ^ swz(r) with the 8-byte halves swapped on rows
// with bit 2 set for transpose reads) measured no faster here: this kernel is HBM-bound.
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | (r >> 2); }

// LDS-only release/acquire around the workgroup barrier: waits for this
// wave's LDS writes (lgkmcnt) but not for its K/V loads in flight.
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Element offset of the 8-dim slice c (0..3) a lane of group grp owns. Any
// assignment works as long as K, V, Q and the output agree (the MFMA sums over
// k in whatever order both operands use); with 32*c + 8*grp the four lanes of
// one key row read 64 contiguous bytes per load instruction.
__device__ __forceinline__ int dim_off(int grp, int c) {
  return ASPIRE_DIM_MAP ? 32 * c + 8 * grp : 32 * grp + 8 * c;
}

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

__device__ __forceinline__ uint4 load16(const uint16_t* ptr) { return *reinterpret_cast<const uint4*>(ptr); }

// K / V loads go through buffer resources: a per-page scalar descriptor (base =
// the page's K or V rows of this kv head) and one per-lane 32-bit byte offset
// that stays fixed for the whole item; slice c adds an immediate 64*c. A lane
// whose key is past kv_len uses an offset beyond the descriptor's range, which
// the hardware answers with zeros (no branch, no out-of-range access).
constexpr uint32_t kBufferConfig = 0x00020000u;  // gfx9 raw buffer dword 3
constexpr int kOutOfRange = 0x7ffffff0;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const uint16_t* base, int32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0, bytes, kBufferConfig);
}

// NTL sets the non-temporal policy bit (aux 2): streamed K/V is read once.
template <bool NTL>
__device__ __forceinline__ void load_rows(__amdgpu_buffer_rsrc_t rsrc, int voff, uint4 (&dst)[4]) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff + 64 * c, 0, NTL ? 2 : 0);
    dst[c] = make_uint4(v.x, v.y, v.z, v.w);
  }
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) {
  return __builtin_bit_cast(bf16x8, u);
}

__device__ __forceinline__ i16x4 as_i16x4(uint32_t a, uint32_t b) {
  uint2 u = make_uint2(a, b);
  return __builtin_bit_cast(i16x4, u);
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2v;

// acc + a.lo * b.lo + a.hi * b.hi for two packed bf16 pairs, fp32 accumulation.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, a), __builtin_bit_cast(bf16x2v, b), acc,
                                         false);
}
// Max / sum over the 16 lanes of each 16-lane row (DPP quad permutes, then row_half_mirror and
// row_mirror, which pair quads and halves once those are uniform); every lane gets the result.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  return v;
}

__device__ __forceinline__ void store_dump(const AttnParams& p, int64_t idx, float v) {
  if (p.dump_f32) {
    static_cast<float*>(p.dump)[idx] = v;
  } else {
    _Float16 h = static_cast<_Float16>(v);
    static_cast<_Float16*>(p.dump)[idx] = h;
  }
}

// The workgroup's staging of one head-aligned slot's pages (see run_item) by its first SW
// waves: wave q < SW loads row-halves j = q * PER + i (K rows for j < 16, V rows j - 16
// after), each one whole 1 KiB row of the slot's 4 heads, one 128-bit non-temporal load per
// lane, and stores them to LDS chunk c ^ swz(row) of its row. kActive (q < SW) is a template
// argument: the two roles are separate straight-line loops, since a runtime role test made
// the compiler's wait analysis at the loop head treat the query loads as possibly pending and
// wait for the stage loads in flight (vmcnt) before the first MFMA of every page.
template <int SW, bool kActive>
struct Stager {
  static constexpr int PER = (kStageRowHalves + SW - 1) / SW;
  const uint16_t* head0;  // the slot's first kv head in page 0 (p.cache + g0 * c_sh)
  int64_t c_sp;
  int span;               // bytes of a page's K and V rows of 4 heads (buffer range)
  int offs[PER];
  int rows_at[PER];       // LDS chunk of the lane's piece of the row-half, or -1 past the page
  int lane;
  uint4 st[PER];

  __device__ __forceinline__ Stager(const AttnParams& p, int g0, int q, int lane_) : lane(lane_) {
    head0 = p.cache + int64_t(g0) * p.c_sh;
    c_sp = p.c_sp;
    const int row_b = int(p.c_st) * 2;
    span = int(p.c_skv) * 2 + 15 * row_b + 4 * kHeadDim * 2;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int j = q * PER + i;
      const int kv = j >> 4, row = j & 15;
      const bool real = j < kStageRowHalves;
      offs[i] = real ? kv * int(p.c_skv) * 2 + row * row_b + lane * 16 : kOutOfRange;
      rows_at[i] = real ? kv * kStageKv + row * kStageRowChunks + (lane ^ swz(row)) : -1;
    }
  }
  // Every active wave issues the same straight-line loads and stores: slots past the
  // page's 32 row-halves load zeros (out-of-range offset) and store them to the dummy LDS
  // row. (Loads under a per-slot branch made the compiler wait for every load in flight,
  // vmcnt(0), before each of them.)
  __device__ __forceinline__ void load(int64_t phys, bool ok) {
    if constexpr (!kActive) return;
    const __amdgpu_buffer_rsrc_t rs = page_rsrc(head0 + phys * c_sp, span);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? offs[i] : kOutOfRange, 0, 2);
      st[i] = make_uint4(v.x, v.y, v.z, v.w);
    }
  }
  __device__ __forceinline__ void store(uint4* stage_lds, int buf) const {
    if constexpr (!kActive) return;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int at = rows_at[i] >= 0 ? buf * kStageBuf + rows_at[i] : kStageChunks + kScoreChunks + lane;
      stage_lds[at] = st[i];
    }
  }
};

// One (row, kv head) piece: this wave computes NT of its tiles, from tile tile0 (rows
// 16 * tile0 ...). compute = false: a wave with no tile of the item, which only takes its
// part in staging the pages (staged items) or has nothing to do (direct items).
template <int NT, int SW, bool kStage, bool kSplitItem = false, bool kValu = false, bool kNt = false>
__device__ __forceinline__ void run_item(const AttnParams& p, const WorkItem& it, int lane,
                                         i16x4 ident, bool staged, uint4* stage_lds, int tile0, bool compute) {
  static_assert(!kValu || NT == 1, "the VALU path serves 1-tile items");
  constexpr bool kNtl = NT == 1 && ASPIRE_NT1_NTLOADS;
  const int r = lane & 15;
  const int grp = lane >> 4;
  const int G = p.group;
  const int b = it.bg >> 8;
  const int g = it.bg & 255;
  const int rows = it.q_len * G;
  const int kv_len = it.kv_len;
  const bool stage_path = NT <= ASPIRE_STAGED_MAX_NT && staged;
  if (!compute && !stage_path) return;

  // Query fragments and per-row causal limits.
  bf16x8 qf[NT][4];
  int limit[NT];
  int row_qi[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int row = (tile0 + t) * 16 + r;
    if (compute && row < rows) {
      const int qi = row / G;
      const int hh = row - qi * G;
      const uint16_t* src = p.q + int64_t(it.q_start + qi) * p.q_st + int64_t(g * G + hh) * p.q_sh;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        qf[t][c] = as_bf16x8(*reinterpret_cast<const uint4*>(src + dim_off(grp, c)));
      limit[t] = p.causal ? min(kv_len - it.q_len + qi, kv_len - 1) : kv_len - 1;
      row_qi[t] = qi;
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) qf[t][c] = as_bf16x8(make_uint4(0, 0, 0, 0));
      limit[t] = -1;
      row_qi[t] = -1;
    }
  }

  // VALU rows: every lane holds each row's q for its own 32 dims (4 chunks of 8); S is
  // summed over the 4 dim groups with permlane swaps and maximised over the 16 keys with
  // DPP; P.V accumulates in each lane for its key slot r and is summed over the 16 key
  // lanes once, after the last page (the online-softmax rescale is uniform over keys).
  uint4 qv[kValuRows][4];
  int vlim[kValuRows];
  float vm[kValuRows], vl[kValuRows];
  float4 vacc[kValuRows][4][2];
  if constexpr (kValu) {
#pragma unroll
    for (int j = 0; j < kValuRows; ++j) {
      const int qi = j / G;
      if (j < rows) {
        const uint16_t* src =
            p.q + int64_t(it.q_start + qi) * p.q_st + int64_t(g * G + (j - qi * G)) * p.q_sh;
#pragma unroll
        for (int c = 0; c < 4; ++c) qv[j][c] = load16(src + dim_off(grp, c));
        vlim[j] = p.causal ? min(kv_len - it.q_len + qi, kv_len - 1) : kv_len - 1;
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) qv[j][c] = make_uint4(0, 0, 0, 0);
        vlim[j] = -1;
      }
      vm[j] = kNegInf;
      vl[j] = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) vacc[j][c][0] = vacc[j][c][1] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }

  float m[NT], l[NT], m_use[NT];
  f32x4 acc[NT][8];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    m[t] = kNegInf;
    m_use[t] = 0.f;
    l[t] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // smallest causal limit of the item's rows (its first query token)
  const int min_limit = p.causal ? min(kv_len - it.q_len, kv_len - 1) : kv_len - 1;
  const bool do_dump = p.dump_kind != 0 && (p.dump_flags == nullptr || p.dump_flags[b] != 0);
  // (q_len 1 rows of at most 16 query rows: one tile, computed by tile lane 0)
  const bool do_score = NT == 1 && compute && tile0 == 0 && p.page_scores != nullptr && it.q_len == 1 && rows <= 16;
  // key-mean epilogue: this lane's 4-key partial sums of the last 4 pages (sc0 newest) and
  // the wave's 64-page score block in LDS
  float sc0 = 0.f, sc1 = 0.f, sc2 = 0.f, sc3 = 0.f;
  float score_buf = 0.f;  // the VALU draft path's 64-page block (lane = page slot)
  float* const score_lds = reinterpret_cast<float*>(stage_lds + kStageChunks) +
                           ((threadIdx.x >> 6) % kAttnWavesPerBlock) * 64;
  const int dump_slots = p.dump_kind == 2 ? 2 : 1;
  // Dump entry of each tile's row: the lane's element offset of key 0, or -1 for rows that
  // write nothing (kind 1: a row's last query; kind 2: its first and last).
  int64_t dump_at[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    dump_at[t] = -1;
    const int qi = row_qi[t];
    if (do_dump && qi >= 0) {
      const int slot = p.dump_kind == 2 ? (qi == 0 ? 0 : (qi == it.q_len - 1 ? 1 : -1)) : (qi == it.q_len - 1 ? 0 : -1);
      if (slot >= 0) {
        const int head = g * G + ((tile0 + t) * 16 + r - qi * G);
        dump_at[t] = (int64_t(b * p.dump_heads + head) * dump_slots + slot) * p.dump_stride;
      }
    }
  }

  // Page ids are read with scalar loads (constant address space): they are
  // wave-uniform, and scalar loads are tracked by lgkmcnt, so waiting for an id
  // never drains the outstanding K/V vector loads. The id of page pg+2 is
  // requested one iteration before use; the index is clamped into the item.
  const int pb = it.page_begin;
  const int pe = it.page_end;
  typedef const __attribute__((address_space(4))) int32_t* const_ids_t;
  const const_ids_t ids = (const_ids_t)(p.kv_indices + it.list_base);
  auto page_id = [&](int pg) -> int64_t { return int64_t(ids[min(pg, pe - 1)]); };

  // Buffer-load addressing for this item: lane byte offset within one kv
  // head's rows of a page, and the byte extent of those rows.
  const int lane_off = (r * int(p.c_st) + 8 * grp) * 2;
  const int rows_bytes = (15 * int(p.c_st) + kHeadDim) * 2;
  auto load_k = [&](int64_t phys, bool ok, uint4(&dst)[4]) {
    load_rows<kNtl>(page_rsrc(p.cache + phys * p.c_sp + int64_t(g) * p.c_sh, rows_bytes), ok ? lane_off : kOutOfRange,
              dst);
  };
  auto load_v = [&](int64_t phys, bool ok, uint4(&dst)[4]) {
    load_rows<kNtl>(page_rsrc(p.cache + phys * p.c_sp + p.c_skv + int64_t(g) * p.c_sh, rows_bytes),
              ok ? lane_off : kOutOfRange, dst);
  };

  // Per-page compute. after_qk runs once QK^T has consumed K, after_pv once
  // P.V has consumed V (the half-page pipeline issues the next loads there).
  // vsrc: the page's V rows as loaded (uint4[4], lane r = key r, transposed
  // here) or its V^T fragments ready for the PV MFMA (i16x4[8], one per
  // 16-dim slice j, read transposed from LDS).
  auto page_body = [&](int pg, const uint4 (&kr)[4], const auto& vsrc, auto&& after_qk, auto&& after_pv) {
    if constexpr (kValu) {
      float sv[kValuRows];
#pragma unroll
      for (int j = 0; j < kValuRows; ++j) {
        float a = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          a = dot2_bf16(kr[c].x, qv[j][c].x, a);
          a = dot2_bf16(kr[c].y, qv[j][c].y, a);
          a = dot2_bf16(kr[c].z, qv[j][c].z, a);
          a = dot2_bf16(kr[c].w, qv[j][c].w, a);
        }
        sv[j] = a;
      }
      after_qk();
      // the 4 dim groups' partial dot products: every lane now holds q_j . k_r in full
#pragma unroll
      for (int j = 0; j < kValuRows; ++j) sv[j] = add_xor32(add_xor16(sv[j]));
      const int key = pg * 16 + r;
      if (do_dump && grp < rows) {
        const int qi = grp / G;
        int slot = -1;
        if (p.dump_kind == 2)
          slot = qi == 0 ? 0 : (qi == it.q_len - 1 ? 1 : -1);
        else if (qi == it.q_len - 1)
          slot = 0;
        if (slot >= 0 && key < kv_len) {
          const int head = g * G + (grp - qi * G);
          const float v = grp == 0 ? sv[0] : grp == 1 ? sv[1] : grp == 2 ? sv[2] : sv[3];
          store_dump(p, (int64_t(b * p.dump_heads + head) * dump_slots + slot) * p.dump_stride + key, v);
        }
      }
      if (do_score) {
        // key-mean score of this page: max over the group's heads of sum_{valid keys} q.k / count
        const int cnt = min(16, kv_len - pg * 16);
        float val = kNegInf;
#pragma unroll
        for (int j = 0; j < kValuRows; ++j) {
          if (j < rows) {
            const float rs = row16_sum(key < kv_len ? sv[j] : 0.f);
            val = fmaxf(val, cnt == 16 ? rs * 0.0625f : rs / float(cnt));
          }
        }
        const int slot = (pg - pb) & 63;
        score_buf = lane == slot ? val : score_buf;
        if (slot == 63 || pg == pe - 1) {
          if (lane <= slot) p.page_scores[int64_t(b * p.hkv + g) * p.ps_stride + (pg - slot) + lane] = score_buf;
        }
      }
      float pr[kValuRows], alpha[kValuRows];
      bool moved = false;
#pragma unroll
      for (int j = 0; j < kValuRows; ++j) {
        const float x = key <= vlim[j] ? sv[j] * p.scale_log2 : kNegInf;
        const float m_new = fmaxf(vm[j], row16_max(x));
        float a = 1.f, e = 0.f;
        if (m_new != kNegInf) {
          a = __builtin_amdgcn_exp2f(vm[j] - m_new);
          e = __builtin_amdgcn_exp2f(x - m_new);
        }
        vl[j] = vl[j] * a + e;  // this lane's key slot only; summed over the 16 keys at the end
        vm[j] = m_new;
        alpha[j] = a;
        pr[j] = e;
        moved |= a != 1.f;
      }
      if (__builtin_amdgcn_ballot_w64(moved) != 0) {
#pragma unroll
        for (int j = 0; j < kValuRows; ++j)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            vacc[j][c][0] *= alpha[j];
            vacc[j][c][1] *= alpha[j];
          }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint4 v = vsrc[c];
        const float4 lo = make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                                      __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
        const float4 hi = make_float4(__uint_as_float(v.z << 16), __uint_as_float(v.z & 0xffff0000u),
                                      __uint_as_float(v.w << 16), __uint_as_float(v.w & 0xffff0000u));
#pragma unroll
        for (int j = 0; j < kValuRows; ++j) {
          vacc[j][c][0] += pr[j] * lo;
          vacc[j][c][1] += pr[j] * hi;
        }
      }
      after_pv();
    } else {
      const int base_pos = pg * 16 + grp * 4;

      f32x4 s[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c) s[t] = mfma_16x16x32_bf16(as_bf16x8(kr[c]), qf[t][c], s[t]);
      }
      after_qk();

      i16x4 pf[NT];
#if !ASPIRE_ATTN_SLACK
      float alpha[NT];
#else
      // a row's first page of the item sets its max (its keys are visible there if anywhere)
      bool over = pg == pb;
      float xs[NT][4], pv[NT][4], ps[NT];
#endif
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (do_dump && dump_at[t] >= 0) {
          // the lane's 4 consecutive keys of its row: one 8-byte (fp16) or 16-byte (fp32)
          // store when all 4 are valid and the entry is aligned, else one store per key
          const int64_t at = dump_at[t] + base_pos;
          if (p.dump_vec && base_pos + 4 <= kv_len) {
            if (p.dump_f32) {
              *reinterpret_cast<float4*>(static_cast<float*>(p.dump) + at) = make_float4(s[t][0], s[t][1], s[t][2], s[t][3]);
            } else {
              typedef __attribute__((ext_vector_type(4))) _Float16 half4;
              half4 h;
#pragma unroll
              for (int i = 0; i < 4; ++i) h[i] = static_cast<_Float16>(s[t][i]);
              *reinterpret_cast<half4*>(static_cast<_Float16*>(p.dump) + at) = h;
            }
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (base_pos + i < kv_len) store_dump(p, at + i, s[t][i]);
          }
        }
        if (NT == 1 && do_score && t == 0) {
          // Key-mean score of a page: max over the group's heads of sum_{valid keys} q.k / count.
          // Each lane adds its 4 keys; the cross-lane sums run once per 4 pages: two
          // half-wave and one 16-lane exchange turn the 4 pages' partials into page
          // pg - 3 + grp's totals in lane group grp, then the heads' max (lanes r < G) and
          // one LDS write per group. A partial batch at the piece's end rewrites the slots of
          // pages already written (same values) or slots no store reads.
          float rs = (s[t][0] + s[t][1]) + (s[t][2] + s[t][3]);
          if (pg * 16 + 16 > kv_len) {
            rs = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) rs += (base_pos + i < kv_len) ? s[t][i] : 0.f;
          }
          sc3 = sc2;
          sc2 = sc1;
          sc1 = sc0;
          sc0 = rs;
          const int slot = (pg - pb) & 63;
          if ((slot & 3) == 3 || pg == pe - 1) {
            const auto h0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(sc3), __float_as_uint(sc1), false, false);
            const auto h1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(sc2), __float_as_uint(sc0), false, false);
            const float a0 = __uint_as_float(h0[0]) + __uint_as_float(h0[1]);  // pages pg-3 (low half), pg-1 (high)
            const float a1 = __uint_as_float(h1[0]) + __uint_as_float(h1[1]);  // pages pg-2 (low half), pg (high)
            const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(a0), __float_as_uint(a1), false, false);
            const float tot = __uint_as_float(q[0]) + __uint_as_float(q[1]);   // page pg - 3 + grp
            const int page = pg - 3 + grp;
            const int cnt = min(16, kv_len - page * 16);
            float val = (r < G) ? (cnt >= 16 ? tot * 0.0625f : tot / float(max(cnt, 1))) : kNegInf;
            // max over the group's heads (lanes r < G of each 16-lane group)
            if (G > 1) val = fmaxf(val, dpp_xor1(val));
            if (G > 2) val = fmaxf(val, dpp_xor2(val));
            if (G > 4) val = fmaxf(val, shfl_xor_f(val, 4));
            if (G > 8) val = fmaxf(val, shfl_xor_f(val, 8));
            if (r == 0) score_lds[(page - pb) & 63] = val;
            // One coalesced store per 64 pages (a store per page would share vmcnt
            // with the K/V loads in flight).
            if (slot == 63 || pg == pe - 1) {
              const float v = score_lds[lane];  // a wave's LDS accesses complete in order
              if (lane <= slot) p.page_scores[int64_t(b * p.hkv + g) * p.ps_stride + (pg - slot) + lane] = v;
            }
          }
        }

#if ASPIRE_ATTN_SLACK
        // raw scores, masked; exponentials with the current offset (scale folded into the fma)
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = s[t][i];
        if (pg * 16 + 15 > min_limit) {
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] = (base_pos + i <= limit[t]) ? x[i] : kNegInf;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) xs[t][i] = x[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) pv[t][i] = __builtin_amdgcn_exp2f(fmaf(x[i], p.scale_log2, -m_use[t]));
        ps[t] = (pv[t][0] + pv[t][1]) + (pv[t][2] + pv[t][3]);
        over |= ps[t] > kAttnSumLimit;
#else
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = s[t][i] * p.scale_log2;
        // only pages that reach a row's causal limit or kv_len need the mask
        // (rows past the tile keep their unmasked, finite, unused values)
        if (pg * 16 + 15 > min_limit) {
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] = (base_pos + i <= limit[t]) ? x[i] : kNegInf;
        }
        float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
        mx = max_xor32(max_xor16(mx));
        const float m_new = fmaxf(m[t], mx);
        float a = 1.f;
        float pv[4] = {0.f, 0.f, 0.f, 0.f};
        if (m_new != kNegInf) {
          a = __builtin_amdgcn_exp2f(m[t] - m_new);
#pragma unroll
          for (int i = 0; i < 4; ++i) pv[i] = __builtin_amdgcn_exp2f(x[i] - m_new);
        }
        l[t] = l[t] * a + ((pv[0] + pv[1]) + (pv[2] + pv[3]));
        m[t] = m_new;
        alpha[t] = a;
        pf[t] = as_i16x4(pack_bf16x2_rne(pv[0], pv[1]), pack_bf16x2_rne(pv[2], pv[3]));
#endif
      }
#if ASPIRE_ATTN_SLACK
      if (__builtin_amdgcn_ballot_w64(over) != 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          float mx = fmaxf(fmaxf(xs[t][0], xs[t][1]), fmaxf(xs[t][2], xs[t][3]));
          mx = max_xor32(max_xor16(mx)) * p.scale_log2;
          const float m_new = mx > m[t] + float(ASPIRE_ATTN_SLACK) ? mx : m[t];
          const float mu = m_new == kNegInf ? 0.f : m_new;
          // a row with no key before (m = -inf) has zero sums: alpha 0 keeps them zero
          const float a = __builtin_amdgcn_exp2f(m[t] - mu);
          m[t] = m_new;
          m_use[t] = mu;
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[t][j] *= a;
          l[t] *= a;
#pragma unroll
          for (int i = 0; i < 4; ++i) pv[t][i] = __builtin_amdgcn_exp2f(fmaf(xs[t][i], p.scale_log2, -mu));
          ps[t] = (pv[t][0] + pv[t][1]) + (pv[t][2] + pv[t][3]);
        }
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        l[t] += ps[t];
        pf[t] = as_i16x4(pack_bf16x2_rne(pv[t][0], pv[t][1]), pack_bf16x2_rne(pv[t][2], pv[t][3]));
      }
#else

      // Rescale the accumulators only when some row's running max moved: once
      // the max settles (most pages), alpha is exactly 1 for every row and the
      // multiplies are skipped (a wave-uniform branch; results are unchanged).
      bool moved = false;
#pragma unroll
      for (int t = 0; t < NT; ++t) moved |= alpha[t] != 1.f;
      if (__builtin_amdgcn_ballot_w64(moved) != 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[t][j] *= alpha[t];
      }
#endif

      // O^T += V^T P^T, one 16-dim slice at a time. Rows from registers are
      // transposed with an exact identity MFMA (the values are bf16 already).
      constexpr bool kVt = std::is_same_v<std::remove_cv_t<std::remove_reference_t<decltype(vsrc)>>, i16x4[8]>;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        i16x4 vt;
        if constexpr (kVt) {
          vt = vsrc[j];
        } else {
          const uint4 src = vsrc[j >> 1];
          const i16x4 va = (j & 1) ? as_i16x4(src.z, src.w) : as_i16x4(src.x, src.y);
          const f32x4 d = mfma_16x16x16_bf16(va, ident, f32x4{0.f, 0.f, 0.f, 0.f});
          vt = as_i16x4(pack_bf16x2_exact(d[0], d[1]), pack_bf16x2_exact(d[2], d[3]));
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t][j] = mfma_16x16x16_bf16(vt, pf[t], acc[t][j]);
      }
      after_pv();
    }
  };

  if constexpr (NT <= ASPIRE_STAGED_MAX_NT) {
    if (staged) {
      // Workgroup-staged K/V. The workgroup's head lanes hold kv heads g0..g0+3
      // of one head-aligned slot: the same pages, and together 1 KiB of
      // contiguous cache per key row (the rows' 4 heads). Every wave of the
      // workgroup loads a block of the page's 32 row-halves (K or V rows) as
      // whole 1 KiB rows, one 128-bit non-temporal load per lane and row, and
      // stores them to LDS; after a barrier every computing wave reads its own
      // head's rows from LDS in the MFMA operand layout. Contiguous 1 KiB loads
      // stream measurably faster from HBM than 16 rows x 64 B per instruction.
      // LDS chunk c of key row r sits at c ^ swz(r) (see swz). Two LDS buffers:
      // page pg is read from one while page pg + 1 is stored to the other and
      // page pg + 2 is in flight. Every wave of the workgroup takes the same
      // barriers: waves with no tile of the item stage and wait only.
      if (pb < pe) {
        const int gl = g & 3;
        Stager<SW, kStage> stg(p, g & ~3, wave_uniform(threadIdx.x >> 6), lane);
        auto read_rows = [&](int buf, int kv, uint4(&dst)[4]) {
          const uint4* base = stage_lds + buf * kStageBuf + kv * kStageKv + r * kStageRowChunks;
#pragma unroll
          for (int c = 0; c < 4; ++c) dst[c] = base[(gl * 16 + c * 4 + grp) ^ swz(r)];
        };
        // V^T fragments straight from the staged rows with the LDS transpose
        // read: of the 16 lanes of group grp, lane r addresses key row
        // 4*grp + r/4 at dims 32*(j/2) + 8*(r%4) + 4*(j%2) (4 consecutive
        // bf16), and the read hands lane r element r%4 of the lanes r/4 + 4e,
        // e = 0..3: keys 4*grp + e of dim 32*(j/2) + 8*(r/4) + 4*(j%2) + r%4,
        // the A operand of the PV MFMA in the slice order of the epilogue.
        const int vt_row = 4 * grp + (r >> 2);
        auto read_vt = [&](int buf, i16x4(&vt)[8]) {
          const char* base = reinterpret_cast<const char*>(stage_lds + buf * kStageBuf + kStageKv +
                                                           vt_row * kStageRowChunks);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int chunk = (gl * 16 + 4 * (j >> 1) + (r & 3)) ^ swz(vt_row);
            vt[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4*)(base + chunk * 16 + 8 * (j & 1)));
          }
        };
        stg.load(page_id(pb), true);
        stg.store(stage_lds, 0);
        stg.load(page_id(pb + 1), pb + 1 < pe);
        stage_barrier();
        int64_t id_ahead = page_id(pb + 2);
        int pg = pb;
        if (!compute) {
          do {
            stg.store(stage_lds, ((pg - pb) & 1) ^ 1);
            const int64_t nphys = id_ahead;
            id_ahead = page_id(pg + 3);
            stg.load(nphys, pg + 2 < pe);
            stage_barrier();
          } while (++pg < pe);
          return;
        }
        do {
          const int buf = (pg - pb) & 1;
          uint4 kr[4];
          // V^T by transpose reads for waves of ASPIRE_VT_READ_MIN_NT tiles or more; the
          // others read V rows (conflict-free 128-bit reads) and transpose them with the
          // identity MFMA, which measured faster for 1-tile items at one wave per SIMD
          constexpr bool kVtRead = NT >= ASPIRE_VT_READ_MIN_NT || kSplitItem;
          using VSrc = std::conditional_t<kVtRead, i16x4[8], uint4[4]>;
          VSrc vs;
          read_rows(buf, 0, kr);
          page_body(
              pg, kr, vs,
              [&] {
                // keys past kv_len (only on a segment's last page) may hold stale
                // values: zero them so 0 * stale cannot reach the sums
                const bool tail = pg * 16 + 16 > kv_len;
                if constexpr (kVtRead) {
                  read_vt(buf, vs);
                  if (tail) {
                    const int k0 = pg * 16 + 4 * grp;
                    const uint32_t m0 = (k0 < kv_len ? 0xffffu : 0u) | (k0 + 1 < kv_len ? 0xffff0000u : 0u);
                    const uint32_t m1 = (k0 + 2 < kv_len ? 0xffffu : 0u) | (k0 + 3 < kv_len ? 0xffff0000u : 0u);
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                      const uint2 w = __builtin_bit_cast(uint2, vs[j]);
                      vs[j] = as_i16x4(w.x & m0, w.y & m1);
                    }
                  }
                } else {
                  read_rows(buf, 1, vs);
                  // a per-lane select here measured faster than the tail-only mask
                  const bool v_ok = pg * 16 + r < kv_len;
#pragma unroll
                  for (int c = 0; c < 4; ++c) vs[c] = v_ok ? vs[c] : make_uint4(0, 0, 0, 0);
                }
              },
              [&] {
                stg.store(stage_lds, buf ^ 1);
                const int64_t nphys = id_ahead;
                id_ahead = page_id(pg + 3);
                stg.load(nphys, pg + 2 < pe);
                stage_barrier();
              });
        } while (++pg < pe);
      }
    }
  }

  if (!compute) return;  // (a staged piece with no pages)

  // One K/V register buffer pipelined at half-page granularity: the next
  // page's K is requested as soon as this page's QK^T has consumed K, and its V
  // as soon as P.V has consumed each V slice (about one page in flight per
  // wave, 32 VGPRs; a second buffer measured no faster). Prologue and loop
  // share one block so the loop head sees a single, straight-line load order.
  // (Tile lanes of one direct item each load the pages they compute on.)
  if (!stage_path && pb < pe) {
    uint4 kr[4], vr[4];
    {
      const int64_t phys = page_id(pb);
      const bool ok = pb * 16 + r < kv_len;
      load_k(phys, ok, kr);
      __builtin_amdgcn_sched_barrier(0);
      load_v(phys, ok, vr);
    }
    int64_t id_ahead = page_id(pb + 1);
    int pg = pb;
    do {
      const bool has_next = pg + 1 < pe;
      const int64_t next_phys = id_ahead;
      id_ahead = page_id(pg + 2);
      // Issued unconditionally (straight-line code keeps the wait counts
      // exact); past the item's last page the out-of-range offset returns zeros.
      const bool next_ok = has_next && (pg + 1) * 16 + r < kv_len;
      page_body(pg, kr, vr, [&] { load_k(next_phys, next_ok, kr); }, [&] { load_v(next_phys, next_ok, vr); });
    } while (++pg < pe);
  }

  if constexpr (kValu) {
    // sum the per-key-slot partials over the 16 key lanes of each dim group; lane (r, grp)
    // then writes row r / 4's dims dim_off(grp, r % 4) .. + 8
    const int jr = r >> 2, cr = r & 3;
    float lt = 0.f, mt = kNegInf;
    float4 o0 = make_float4(0.f, 0.f, 0.f, 0.f), o1 = o0;
#pragma unroll
    for (int j = 0; j < kValuRows; ++j) {
      const float lj = row16_sum(vl[j]);
      if (j == jr) {
        lt = lj;
        mt = vm[j];
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float4 a0 = vacc[j][c][0], a1 = vacc[j][c][1];
        a0.x = row16_sum(a0.x); a0.y = row16_sum(a0.y); a0.z = row16_sum(a0.z); a0.w = row16_sum(a0.w);
        a1.x = row16_sum(a1.x); a1.y = row16_sum(a1.y); a1.z = row16_sum(a1.z); a1.w = row16_sum(a1.w);
        if (j == jr && c == cr) {
          o0 = a0;
          o1 = a1;
        }
      }
    }
    if (jr < rows) {
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      const float lse_v = lt > 0.f ? mt + __builtin_log2f(lt) : kNegInf;
      const int qi = jr / G;
      const int head = g * G + (jr - qi * G);
      if (it.partial_row < 0) {
        const int token = it.q_start + qi;
        uint16_t* dst = p.out + int64_t(token) * p.o_st + int64_t(head) * p.o_sh + dim_off(grp, cr);
        uint4 w;
        w.x = pack_bf16x2_rne(o0.x * inv, o0.y * inv);
        w.y = pack_bf16x2_rne(o0.z * inv, o0.w * inv);
        w.z = pack_bf16x2_rne(o1.x * inv, o1.y * inv);
        w.w = pack_bf16x2_rne(o1.z * inv, o1.w * inv);
        *reinterpret_cast<uint4*>(dst) = w;
        if (grp == 0 && cr == 0 && p.lse != nullptr) p.lse[int64_t(token) * p.hq + head] = lse_v;
      } else {
        const int64_t prow = int64_t(it.partial_row) + jr;
        float* dst = p.part_o + prow * kHeadDim + dim_off(grp, cr);
        store_partial4<kNt>(dst, o0.x * inv, o0.y * inv, o0.z * inv, o0.w * inv);
        store_partial4<kNt>(dst + 4, o1.x * inv, o1.y * inv, o1.z * inv, o1.w * inv);
        if (grp == 0 && cr == 0) p.part_lse[prow] = lse_v;
      }
    }
    return;
  }

  // Epilogue: normalise and write the final output or the fp32 partial.
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    float lt = l[t];
    lt += shfl_xor_f(lt, 16);
    lt += shfl_xor_f(lt, 32);
    const int row = (tile0 + t) * 16 + r;
    if (row >= rows) continue;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const float lse_v = lt > 0.f ? m[t] + __builtin_log2f(lt) : kNegInf;
    if (it.partial_row < 0) {
      const int qi = row / G;
      const int head = g * G + (row - qi * G);
      const int token = it.q_start + qi;
      uint16_t* dst = p.out + int64_t(token) * p.o_st + int64_t(head) * p.o_sh;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f32x4 a0 = acc[t][2 * c];
        const f32x4 a1 = acc[t][2 * c + 1];
        uint4 w;
        w.x = pack_bf16x2_rne(a0[0] * inv, a0[1] * inv);
        w.y = pack_bf16x2_rne(a0[2] * inv, a0[3] * inv);
        w.z = pack_bf16x2_rne(a1[0] * inv, a1[1] * inv);
        w.w = pack_bf16x2_rne(a1[2] * inv, a1[3] * inv);
        *reinterpret_cast<uint4*>(dst + dim_off(grp, c)) = w;
      }
      if (grp == 0 && p.lse != nullptr) p.lse[int64_t(token) * p.hq + head] = lse_v;
    } else {
      const int64_t prow = int64_t(it.partial_row) + row;
      float* dst = p.part_o + prow * kHeadDim;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const f32x4 a = acc[t][j];
        store_partial4<kNt>(dst + dim_off(grp, j >> 1) + 4 * (j & 1), a[0] * inv, a[1] * inv, a[2] * inv, a[3] * inv);
      }
      if (grp == 0) p.part_lse[prow] = lse_v;
    }
  }
}

// One item of a class for this wave: n of its tiles from tile0 (n = K or the short share R;
// 0: no tile), kStage: the wave loads a block of the staged pages.
template <int TILES, int K, int R, int SW, bool kStage, bool kSplit, bool kNt>
__device__ __forceinline__ void run_class_item(const AttnParams& p, const WorkItem& it, int lane, i16x4 ident,
                                               bool stg, uint4* stage_lds, int tile0, int n) {
  if constexpr (TILES == 1 && ASPIRE_DRAFT_VALU) {
    if (it.q_len * p.group <= kValuRows) {
      run_item<1, SW, kStage, false, true, kNt>(p, it, lane, ident, stg, stage_lds, tile0, n > 0);
      return;
    }
  }
  if (n == K) {
    run_item<K, SW, kStage, kSplit, false, kNt>(p, it, lane, ident, stg, stage_lds, tile0, true);
  } else if constexpr (R > 0) {
    if (n == R) run_item<R, SW, kStage, kSplit, false, kNt>(p, it, lane, ident, stg, stage_lds, tile0, true);
    else run_item<K, SW, kStage, kSplit, false, kNt>(p, it, lane, ident, stg, stage_lds, tile0, false);
  } else {
    run_item<K, SW, kStage, kSplit, false, kNt>(p, it, lane, ident, stg, stage_lds, tile0, false);
  }
}

// Items of one row-tile class (TILES 16-row tiles) for this wave, tile lane tl of its head.
template <int TILES, bool kNt>
__device__ __forceinline__ void run_class(const AttnParams& p, int c, int w0, int w1, int lane, i16x4 ident,
                                          bool staged, uint4* stage_lds, int tl) {
  constexpr bool kSplit = TILES >= ASPIRE_SPLIT_MIN_TILES;
  constexpr int LANES = kSplit ? kTileLanes : 1;             // lanes that compute this class
  constexpr int K = (TILES + LANES - 1) / LANES;             // tiles per computing lane
  constexpr int R = TILES % K;                               // the last computing lane's share, if short
  constexpr int SW = kAttnWavesPerBlock * (kSplit ? ASPIRE_SPLIT_STAGE_LANES : 1);  // staging waves
  const int tile0 = tl * K;
  const int n = tl < LANES ? min(K, TILES - tile0) : 0;
  const bool stager = wave_uniform(threadIdx.x >> 6) < SW;
  const WorkItem* items = reinterpret_cast<const WorkItem*>(p.plan + p.items_off[c]);
  for (int w = w0; w < w1; ++w) {
    WorkItem it;
    it.q_start = wave_uniform(items[w].q_start);
    const int q_len_flags = wave_uniform(items[w].q_len);
    it.q_len = q_len_flags & (kItemDirect - 1);
    it.kv_len = wave_uniform(items[w].kv_len);
    it.list_base = wave_uniform(items[w].list_base);
    it.page_begin = wave_uniform(items[w].page_begin);
    it.page_end = wave_uniform(items[w].page_end);
    it.bg = wave_uniform(items[w].bg);
    it.partial_row = wave_uniform(items[w].partial_row);
    // The flag is a property of the row, so the workgroup's waves (heads of one slot and
    // their tile lanes, walking the same rows) all take the same path, and so take the same
    // barriers; the class's tiles per lane (K) decide it for every lane alike.
    const bool stg = staged && !(q_len_flags & kItemDirect) && K <= ASPIRE_STAGED_MAX_NT;
    constexpr bool kSplitItems = kSplit && LANES > 1;
    if (stager) {
      run_class_item<TILES, K, R, SW, true, kSplitItems, kNt>(p, it, lane, ident, stg, stage_lds, tile0, n);
    } else {
      run_class_item<TILES, K, R, SW, false, kSplitItems, kNt>(p, it, lane, ident, stg, stage_lds, tile0, n);
    }
  }
}

// One persistent launch for all row-tile classes: each wave runs its class-1
// items, then class 2, then class 3 (the planner balances every class over
// the head waves), so the launch has one ramp and one tail. A workgroup is
// kAttnWavesPerBlock head waves of the plan x kTileLanes tile lanes; the
// default grid runs one head wave per SIMD (plus its tile lanes).
template <bool kNt>
__global__ __launch_bounds__(64 * kWgWaves)
__attribute__((amdgpu_waves_per_eu(ASPIRE_ATTN_WAVES_PER_EU))) void attention_kernel(AttnParams p) {
  const int lane = threadIdx.x & 63;
  const int wl = wave_uniform(threadIdx.x >> 6);
  const int tl = wl / kAttnWavesPerBlock;
  const int wave = wave_uniform(blockIdx.x * kAttnWavesPerBlock + wl % kAttnWavesPerBlock);
  if (wave >= p.num_waves) return;
  // Identity B operand: lane holds B[k = 4*grp + j][n = r] = (k == n).
  const int r = lane & 15, grp = lane >> 4;
  const uint32_t one = 0x3f80u;  // bf16 1.0
  uint32_t e0 = (4 * grp + 0 == r ? one : 0u) | ((4 * grp + 1 == r ? one : 0u) << 16);
  uint32_t e1 = (4 * grp + 2 == r ? one : 0u) | ((4 * grp + 3 == r ? one : 0u) << 16);
  const i16x4 ident = as_i16x4(e0, e1);
  // Head-aligned plans (header[4] = kv heads per slot, a multiple of 4) give
  // the head lanes of a workgroup the same pages: their items stage K/V
  // through LDS. The flag is uniform over the workgroup, so every wave takes
  // the same barriers.
  __shared__ uint4 stage_lds[kLdsChunks];
  const int hpu = wave_uniform(p.plan[4]);
  const bool staged = p.staged_ok && hpu > 0 && hpu % 4 == 0;
  // every class's item range for this wave, read in one round trip at the start (a wave
  // that finishes its class-1 items then finds empty classes 2 and 3 without waiting)
  int w0[3], w1[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const int32_t* indptr = p.plan + p.indptr_off[c];
    w0[c] = wave_uniform(indptr[wave]);
    w1[c] = wave_uniform(indptr[wave + 1]);
  }
  if (p.class_mask & 1) run_class<1, kNt>(p, 0, w0[0], w1[0], lane, ident, staged, stage_lds, tl);
  if (p.class_mask & 2) run_class<2, kNt>(p, 1, w0[1], w1[1], lane, ident, staged, stage_lds, tl);
  if (p.class_mask & 4) run_class<3, kNt>(p, 2, w0[2], w1[2], lane, ident, staged, stage_lds, tl);
}

// Merge of split segments. A task is (merge item, 4 units), one unit per 16-lane group: a
// unit is (row, piece group) of the item's row range, and lane l of a group combines dims
// 8 (l % 16) .. + 8 of its row over the pieces of its piece group, so a row's partials are
// read as 512 contiguous bytes per piece. Items with more pieces than one round of loads
// covers (kMergeChunk) come as row ranges of at most 24 or 12 rows whose rows split their
// pieces over s = 2 or 4 adjacent groups (pieces g, g + s, ...); the groups of a row then
// combine their (max, sum, o) states by cross-lane exchanges. A 36-row item of 69 pieces
// thus takes 36 waves with three rounds of loads each instead of 9 waves with nine. Tasks
// past an item's units end after reading its header.
constexpr int kMergeTaskUnits = 4;
constexpr int kMergeTasksPerItem = kMergeRows / kMergeTaskUnits;

__global__ __launch_bounds__(256) void merge_kernel(MergeParams p) {
  constexpr int kChunk = kMergeChunk;  // pieces whose loads are issued together
  const int lane = threadIdx.x & 63;
  const int wave = wave_uniform(blockIdx.x * 4 + (threadIdx.x >> 6));
  const int waves = gridDim.x * 4;
  const MergeItem* items = reinterpret_cast<const MergeItem*>(p.plan + p.merge_off);
  // The wave's first item is read together with the item count (one round trip instead
  // of two); its index stays inside the plan's merge region whatever the count is.
  const int mi_first = min(wave / kMergeTasksPerItem, p.max_merge - 1);
  const int first_rows = wave_uniform(items[mi_first].rows);
  const int first_row_count = wave_uniform(items[mi_first].row_count);
  const int first_pieces = wave_uniform(items[mi_first].num_pieces);
  const int first_row_begin = wave_uniform(items[mi_first].row_begin);
  const int first_partial = wave_uniform(items[mi_first].first_partial_row);
  const int first_bg = wave_uniform(items[mi_first].bg);
  const int first_q_start = wave_uniform(items[mi_first].q_start);
  const int num_merge = wave_uniform(p.plan[3]);
  const int gsub = lane >> 4, d8 = (lane & 15) * 8;
  for (int u = wave; u < num_merge * kMergeTasksPerItem; u += waves) {
    const int mi = u / kMergeTasksPerItem;
    const int v0 = (u - mi * kMergeTasksPerItem) * kMergeTaskUnits;
    const bool first_item = mi == mi_first;
    const int rows = first_item ? first_rows : wave_uniform(items[mi].rows);
    const int row_count = first_item ? first_row_count : wave_uniform(items[mi].row_count);
    const int pieces = first_item ? first_pieces : wave_uniform(items[mi].num_pieces);
    const int s = merge_piece_groups(pieces, row_count);  // piece groups per row
    if (v0 >= row_count * s) continue;
    const int v = v0 + gsub;
    // units past the item's rows repeat its last row
    const int row = (first_item ? first_row_begin : wave_uniform(items[mi].row_begin)) + min(v / s, row_count - 1);
    const int pg = v & (s - 1);
    const int my_pieces = (pieces - pg + s - 1) / s;
    const int64_t first =
        (first_item ? first_partial : wave_uniform(items[mi].first_partial_row)) + int64_t(row);
    // Running (max, sum, o) over chunks of the group's pieces; within a chunk every LSE and
    // partial load is issued before any is used (one memory round trip).
    float mx = kNegInf, sum = 0.f;
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < my_pieces; k0 += kChunk) {
      const int n = min(kChunk, my_pieces - k0);
      float lse[kChunk];
      float4 va[kChunk], vb[kChunk];
#pragma unroll
      for (int x = 0; x < kChunk; ++x) {
        const int64_t pr = first + int64_t(pg + (k0 + min(x, n - 1)) * s) * rows;
        lse[x] = x < n ? p.part_lse[pr] : kNegInf;
        const float4* src = reinterpret_cast<const float4*>(p.part_o + pr * kHeadDim + d8);
        va[x] = src[0];
        vb[x] = src[1];
      }
      float cmx = mx;
#pragma unroll
      for (int x = 0; x < kChunk; ++x) cmx = fmaxf(cmx, lse[x]);
      if (cmx == kNegInf) continue;
      const float scale = __builtin_amdgcn_exp2f(mx - cmx);  // 0 when mx = -inf
      sum *= scale;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] *= scale;
#pragma unroll
      for (int x = 0; x < kChunk; ++x) {
        const float w = __builtin_amdgcn_exp2f(lse[x] - cmx);  // 0 for padding / empty pieces
        sum += w;
        o[0] += w * va[x].x;
        o[1] += w * va[x].y;
        o[2] += w * va[x].z;
        o[3] += w * va[x].w;
        o[4] += w * vb[x].x;
        o[5] += w * vb[x].y;
        o[6] += w * vb[x].z;
        o[7] += w * vb[x].w;
      }
      mx = cmx;
    }
    // Piece groups of a row sit in adjacent 16-lane groups: fold them pairwise.
    for (int mask = 16; mask < 16 * s; mask <<= 1) {
      const float mo = __shfl_xor(mx, mask);
      const float so = __shfl_xor(sum, mask);
      float oo[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) oo[i] = __shfl_xor(o[i], mask);
      const float mn = fmaxf(mx, mo);
      if (mn != kNegInf) {
        const float a = __builtin_amdgcn_exp2f(mx - mn), b = __builtin_amdgcn_exp2f(mo - mn);
        sum = sum * a + so * b;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = o[i] * a + oo[i] * b;
        mx = mn;
      }
    }
    if (pg != 0 || v / s >= row_count) continue;
    const float inv = sum > 0.f ? 1.f / sum : 0.f;
    const int G = p.group;
    const int qi = row / G;
    const int g = (first_item ? first_bg : wave_uniform(items[mi].bg)) & 255;
    const int head = g * G + (row - qi * G);
    const int token = (first_item ? first_q_start : wave_uniform(items[mi].q_start)) + qi;
    uint4 w;
    w.x = pack_bf16x2_rne(o[0] * inv, o[1] * inv);
    w.y = pack_bf16x2_rne(o[2] * inv, o[3] * inv);
    w.z = pack_bf16x2_rne(o[4] * inv, o[5] * inv);
    w.w = pack_bf16x2_rne(o[6] * inv, o[7] * inv);
    *reinterpret_cast<uint4*>(p.out + int64_t(token) * p.o_st + int64_t(head) * p.o_sh + d8) = w;
    if ((lane & 15) == 0 && p.lse != nullptr)
      p.lse[int64_t(token) * p.hq + head] = sum > 0.f ? mx + __builtin_log2f(sum) : kNegInf;
  }
}

// Standalone state merge: one thread per (row, 4 dims).
__global__ __launch_bounds__(256) void merge_states_kernel(const float* v, const float* s, int n,
                                                           int64_t rows, void* v_out, int out_bf16,
                                                           float* s_out) {
  const int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (e >= rows * 32) return;
  const int64_t row = e >> 5;
  const int d4 = int(e & 31) * 4;
  float mx = kNegInf;
  for (int k = 0; k < n; ++k) mx = fmaxf(mx, s[int64_t(k) * rows + row]);
  float o[4] = {0.f, 0.f, 0.f, 0.f};
  float sum = 0.f;
  if (mx != kNegInf) {
    for (int k = 0; k < n; ++k) {
      const float w = __builtin_amdgcn_exp2f(s[int64_t(k) * rows + row] - mx);
      const float4 x = *reinterpret_cast<const float4*>(v + (int64_t(k) * rows + row) * kHeadDim + d4);
      sum += w;
      o[0] += w * x.x;
      o[1] += w * x.y;
      o[2] += w * x.z;
      o[3] += w * x.w;
    }
  }
  const float inv = sum > 0.f ? 1.f / sum : 0.f;
  if (out_bf16) {
    uint2 w2;
    w2.x = pack_bf16x2_rne(o[0] * inv, o[1] * inv);
    w2.y = pack_bf16x2_rne(o[2] * inv, o[3] * inv);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(v_out) + row * kHeadDim + d4) = w2;
  } else {
    *reinterpret_cast<float4*>(static_cast<float*>(v_out) + row * kHeadDim + d4) =
        make_float4(o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv);
  }
  if (d4 == 0 && s_out != nullptr) s_out[row] = sum > 0.f ? mx + __builtin_log2f(sum) : kNegInf;
}

inline bool al16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace
}  // namespace aspire

// Split-KV partials of aspire_attention_run_static: a file-scope device array
// of ASPIRE_STATIC_SCRATCH_BYTES that every GPU the library runs on holds until
// the process ends. In host code `scratch` names the host-side shadow, not
// device memory: its device address comes from hipGetSymbolAddress, once per
// device (static_scratch_ptr), and only that address reaches kernels.
static __device__ __align__(256) float scratch[ASPIRE_STATIC_SCRATCH_BYTES / sizeof(float)];

namespace aspire {
namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];  // per device, guarded by g_scratch_mu

// Device address of `scratch` on device dev (the current device).
int static_scratch_ptr(int dev, float** out) {
  ASPIRE_CHECK_ARG(dev >= 0 && dev < kMaxScratchDevices, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    ASPIRE_CHECK_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    ASPIRE_CHECK_ARG(ptr != nullptr, "hipGetSymbolAddress returned no address for the scratch array");
    g_scratch_ptr[dev] = ptr;
  }
  *out = static_cast<float*>(g_scratch_ptr[dev]);
  return ASPIRE_OK;
}

// Shared body of both entry points: the partials live at float_ws.
int attention_run_impl(const aspire_plan_layout* layout, const aspire_attention_args* a, float* float_ws,
                       void* stream) {
  ASPIRE_CHECK_ARG(a->head_dim == kHeadDim, "head_dim must be 128");
  ASPIRE_CHECK_ARG(a->page_size == kPage, "page_size must be 16");
  ASPIRE_CHECK_ARG(a->num_kv_heads > 0 && a->num_kv_heads < 256 &&
                       a->num_qo_heads % a->num_kv_heads == 0 &&
                       a->num_qo_heads / a->num_kv_heads <= 16 * kMaxRowTiles,
                   "bad head counts (num_qo_heads a multiple of num_kv_heads, group at most 48)");
  ASPIRE_CHECK_ARG(a->q && a->kv_cache && a->kv_indices && a->out && a->plan_dev && float_ws,
                   "null pointer");
  ASPIRE_CHECK_ARG(al16(a->q) && al16(a->kv_cache) && al16(a->out) && al16(float_ws),
                   "q, kv_cache, out and the float workspace must be 16-byte aligned");
  ASPIRE_CHECK_ARG(a->q_stride_t % 8 == 0 && a->q_stride_h % 8 == 0 && a->out_stride_t % 8 == 0 &&
                       a->out_stride_h % 8 == 0 && a->cache_stride_p % 8 == 0 &&
                       a->cache_stride_kv % 8 == 0 && a->cache_stride_t % 8 == 0 &&
                       a->cache_stride_h % 8 == 0,
                   "strides must be multiples of 8 elements");
  ASPIRE_CHECK_ARG(a->dump_kind >= 0 && a->dump_kind <= 2, "dump_kind must be 0, 1 or 2");
  ASPIRE_CHECK_ARG(a->cache_stride_t > 0 && (15 * a->cache_stride_t + kHeadDim) * 2 < (int64_t(1) << 30),
                   "cache token stride too large for 32-bit buffer offsets");
  ASPIRE_CHECK_ARG(a->dump_kind == 0 || (a->dump != nullptr && a->dump_kv_stride > 0 &&
                                         a->dump_num_heads > 0),
                   "dump buffer, stride and head count required");
  const PlanOffsets off = plan_offsets(*layout);
  AttnParams p;
  p.q = static_cast<const uint16_t*>(a->q);
  p.q_st = a->q_stride_t;
  p.q_sh = a->q_stride_h;
  p.cache = static_cast<const uint16_t*>(a->kv_cache);
  p.c_sp = a->cache_stride_p;
  p.c_skv = a->cache_stride_kv;
  p.c_st = a->cache_stride_t;
  p.c_sh = a->cache_stride_h;
  p.kv_indices = a->kv_indices;
  p.out = static_cast<uint16_t*>(a->out);
  p.o_st = a->out_stride_t;
  p.o_sh = a->out_stride_h;
  p.lse = a->lse;
  p.plan = static_cast<const int32_t*>(a->plan_dev);
  p.num_waves = layout->num_waves;
  p.part_o = float_ws;
  p.part_lse = float_ws + layout->partial_rows_cap * kHeadDim;
  p.hq = a->num_qo_heads;
  p.hkv = a->num_kv_heads;
  p.group = a->num_qo_heads / a->num_kv_heads;
  p.scale_log2 = a->sm_scale * 1.4426950408889634f;
  p.causal = a->causal;
  p.dump = a->dump;
  p.dump_kind = a->dump_kind;
  p.dump_f32 = a->dump_dtype == 1;
  p.dump_stride = a->dump_kv_stride;
  // 4 consecutive keys of a row form one aligned vector (8 or 16 bytes) when the row stride
  // is a multiple of 4 entries and the buffer is 16-byte aligned
  p.dump_vec = a->dump_kind != 0 && a->dump_kv_stride % 4 == 0 && al16(a->dump);
  p.dump_heads = a->dump_num_heads;
  p.dump_flags = a->dump_mode_flags;
  p.page_scores = a->page_scores;
  p.ps_stride = a->page_score_stride;
  // Staged K/V reads 4 adjacent heads as one 1 KiB row; byte offsets within a
  // page (both kv halves, 16 rows) must fit the 32-bit buffer offsets.
  p.staged_ok = ASPIRE_STAGED && a->cache_stride_h == kHeadDim &&
                (a->cache_stride_kv + 15 * a->cache_stride_t + 4 * kHeadDim) * 2 < (int64_t(1) << 30);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((layout->num_waves + kAttnWavesPerBlock - 1) / kAttnWavesPerBlock);
  const dim3 block(64 * kWgWaves);
  for (int c = 0; c < 3; ++c) {
    p.indptr_off[c] = off.indptr[c];
    p.items_off[c] = off.items[c];
  }
  p.class_mask = a->class_mask & 7;
  if (p.class_mask) {
    if (a->partial_nt)
      hipLaunchKernelGGL(attention_kernel<true>, grid, block, 0, s, p);
    else
      hipLaunchKernelGGL(attention_kernel<false>, grid, block, 0, s, p);
    ASPIRE_CHECK_LAUNCH();
  }
  if (a->launch_merge) {
    ASPIRE_CHECK_ARG(layout->max_merge > 0, "plan layout holds no merge items");
    MergeParams mp;
    mp.plan = p.plan;
    mp.merge_off = off.merge;
    mp.part_o = p.part_o;
    mp.part_lse = p.part_lse;
    mp.out = p.out;
    mp.o_st = p.o_st;
    mp.o_sh = p.o_sh;
    mp.lse = p.lse;
    mp.hq = p.hq;
    mp.group = p.group;
    mp.max_merge = layout->max_merge;
    // 8,192 waves: a config-3 layer's 512 items x 12 tasks get a wave each (with 4,096 the
    // merge took 7.2 us there, 6.2 us now); waves past the tasks exit after one load
    hipLaunchKernelGGL(merge_kernel, dim3(2048), dim3(256), 0, s, mp);
    ASPIRE_CHECK_LAUNCH();
  }
  return ASPIRE_OK;
}

}  // namespace
}  // namespace aspire

extern "C" int aspire_attention_run(const aspire_plan_layout* layout, const aspire_attention_args* a,
                                    void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(layout && a, "null argument");
  return attention_run_impl(layout, a, a->float_ws, stream);
}

extern "C" int aspire_attention_run_static(const aspire_plan_layout* layout, const aspire_attention_args* a,
                                           void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(layout && a, "null argument");
  ASPIRE_CHECK_ARG(a->float_ws == nullptr, "float_ws must be NULL: the partials live in the library's static array");
  // The plan's partial rows are bounded by the layout's capacity; the layout
  // must not describe more float workspace than the static array holds.
  if (layout->float_ws_bytes > int64_t(ASPIRE_STATIC_SCRATCH_BYTES) || layout->partial_rows_cap < 0 ||
      layout->partial_rows_cap * int64_t(kHeadDim + 1) * 4 > int64_t(ASPIRE_STATIC_SCRATCH_BYTES)) {
    set_error("aspire_attention_run_static: the layout's float workspace (%lld bytes, %lld partial rows) exceeds "
              "the static scratch of %lld bytes; build the layout with float_ws_bytes <= ASPIRE_STATIC_SCRATCH_BYTES",
              static_cast<long long>(layout->float_ws_bytes), static_cast<long long>(layout->partial_rows_cap),
              static_cast<long long>(ASPIRE_STATIC_SCRATCH_BYTES));
    return ASPIRE_ERR_CAPACITY;
  }
  // The scratch address is per device: the stream must run on the current device.
  int dev = -1;
  ASPIRE_CHECK_HIP(hipGetDevice(&dev));
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    ASPIRE_CHECK_HIP(hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev));
    ASPIRE_CHECK_ARG(sdev == dev, "the stream belongs to another device than the current one");
  }
  float* ws = nullptr;
  const int rc = static_scratch_ptr(dev, &ws);
  if (rc != ASPIRE_OK) return rc;
  return attention_run_impl(layout, a, ws, stream);
}

extern "C" int aspire_merge_states(const float* v, const float* s, int32_t num_states, int64_t rows,
                                   int32_t head_dim, void* v_out, int32_t out_dtype, float* s_out,
                                   void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(head_dim == kHeadDim, "head_dim must be 128");
  ASPIRE_CHECK_ARG(num_states >= 1 && rows >= 0, "bad sizes");
  if (rows == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(v && s && v_out, "null pointer");
  ASPIRE_CHECK_ARG(al16(v) && al16(v_out), "v and v_out must be 16-byte aligned");
  const int64_t threads = rows * 32;
  const int64_t blocks = (threads + 255) / 256;
  ASPIRE_CHECK_ARG(blocks < (int64_t(1) << 31), "too many rows");
  hipLaunchKernelGGL(merge_states_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), v, s, num_states, rows, v_out,
                     out_dtype == 1 ? 1 : 0, s_out);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}
