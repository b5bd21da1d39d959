// (f3) Chunked-prefill paged attention for gfx950.
//
// A workgroup of kPfWaves waves takes one query block of one (row, kv head): kPfWaves x 16 x
// kPfTiles query rows (block_tokens = that / G tokens, G = q heads per kv head), 16 x kPfTiles
// rows per wave. Default build: 4 waves of two 16-row tiles (128 rows), 168 VGPRs and 48 KiB
// of LDS, so three workgroups share a CU (three waves per SIMD); each K fragment and each V^T
// fragment read from LDS feeds both tiles' MFMAs, half the LDS reads per flop of one tile per
// wave. Every page of the block's keys is read from HBM once per workgroup: two pages at a
// time (K and V rows of this kv head, 16 KiB) go straight from HBM into one of kPfStages LDS
// stage buffers (buffer_load ... lds, kPfStages - 1 steps ahead), and each wave runs its tiles
// over those 32 keys:
//   * S^T = K . Q^T per page and tile with 4 v_mfma_f32_16x16x32_bf16 (K rows from LDS,
//     Q fragments in registers); lane (r, grp) holds S^T[key 4grp + i][row r];
//   * online softmax in fp32 over the 32 keys (exp2 with the scale folded into its argument,
//     base-2 LSE), causal masking only on steps that reach a row's limit; the running max
//     moves only when some key exceeds it by more than kPfSlack, and the exponentials are
//     taken with the current offsets first, so on most steps (no lane's sum of a row's
//     exponentials above 2^kPfSlack) no max is computed and the cross-lane max, the rescale
//     and a second pass of exponentials are skipped;
//   * O^T += V^T . P^T with 8 v_mfma_f32_16x16x32_bf16 per tile: each lane's 8 keys are
//     keys 4grp..4grp+3 of both pages (the order S^T left them in), V^T comes from LDS with
//     transpose reads (ds_read_b64_tr_b16) and is shared by the wave's tiles.
// The grid is 1-D with the kv head fastest: the last query blocks of every head (the most
// keys under a causal mask) start first, and with num_kv_heads a multiple of 8 the
// round-robin spread of workgroups over the 8 XCDs keeps each head's pages in one L2.
// Waves whose tokens end before a step skip its compute but keep staging.
#include "common.h"

namespace aspire {
namespace {

constexpr float kNegInfP = -__builtin_huge_valf();
#ifndef ASPIRE_PF_WAVES
#define ASPIRE_PF_WAVES 4
#endif
#ifndef ASPIRE_PF_TILES
#define ASPIRE_PF_TILES 2
#endif
#ifndef ASPIRE_PF_RESCALE_SLACK
#define ASPIRE_PF_RESCALE_SLACK 8
#endif
constexpr float kPfSlack = ASPIRE_PF_RESCALE_SLACK;
constexpr float kPfSumLimit = float(1 << ASPIRE_PF_RESCALE_SLACK);  // 2^kPfSlack
#ifndef ASPIRE_PF_STAGES
#define ASPIRE_PF_STAGES 3
#endif
constexpr int kPfStages = ASPIRE_PF_STAGES;  // LDS stage buffers (loads run kPfStages - 1 steps ahead)
static_assert(kPfStages >= 3 && kPfStages <= 8, "3 to 8 stage buffers");
constexpr int kPfWaves = ASPIRE_PF_WAVES;   // waves per workgroup
constexpr int kPfTiles = ASPIRE_PF_TILES;   // 16-row query tiles per wave
constexpr int kPfRows = 16 * kPfTiles;      // query rows per wave
constexpr int kPfBlockRows = kPfWaves * kPfRows;
constexpr int kPfThreads = 64 * kPfWaves;
#ifndef ASPIRE_PF_WAVES_PER_EU
#define ASPIRE_PF_WAVES_PER_EU 3
#endif
constexpr int kPfWavesPerEu = ASPIRE_PF_WAVES_PER_EU;  // register budget: waves per SIMD
constexpr int kPfRowChunks = 16;            // 16-byte chunks per 256-byte key row (one kv head)
constexpr int kPfHalf = 16 * kPfRowChunks;  // K or V rows of one page, in chunks
constexpr int kPfPage = 2 * kPfHalf;        // one page: K rows, then V rows
constexpr int kPfStage = 2 * kPfPage;       // one step: two pages
constexpr int kPfStepKeys = 2 * kPage;      // keys per step

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4p;
constexpr uint32_t kPfBufferConfig = 0x00020000u;  // gfx9 raw buffer dword 3
static_assert(kPfThreads % 64 == 0 && 1024 % kPfThreads == 0, "a step's chunks split evenly over the threads");

// A pointer the whole wave agrees on, kept in scalar registers (buffer descriptors need that).
template <typename T>
__device__ __forceinline__ T* uniform_ptr(const T* ptr) {
  const uint64_t v = reinterpret_cast<uint64_t>(ptr);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v)), hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
  return reinterpret_cast<T*>((uint64_t(hi) << 32) | lo);
}

__device__ __forceinline__ int pf_swz(int r) { return ((r & 3) << 2) | (r >> 2); }

__device__ __forceinline__ i16x4 pf_i16x4(uint32_t a, uint32_t b) {
  uint2 u = make_uint2(a, b);
  return __builtin_bit_cast(i16x4, u);
}

struct PrefillParams {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* cache;
  int64_t c_sp, c_skv, c_st, c_sh;
  const int32_t* kv_indices;
  const int32_t* kv_indptr;
  const int32_t* last_page_len;
  const int32_t* qo_indptr;
  const int32_t* block_indptr;
  int32_t num_rows, total_blocks, block_tokens;
  uint16_t* out;
  int64_t o_st, o_sh;
  float* lse;
  int32_t hq, group;
  float scale_log2;
  int32_t causal;
};

__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(kPfWavesPerEu))) void prefill_kernel(
    PrefillParams p) {
  __shared__ uint4 stg0[kPfStage];
  __shared__ uint4 stg1[kPfStage];
  __shared__ uint4 stg2[kPfStage];
  __shared__ uint4 stg3[kPfStage];
  __shared__ uint4 stg4[kPfStages > 4 ? kPfStage : 1];
  __shared__ uint4 stg5[kPfStages > 5 ? kPfStage : 1];
  __shared__ uint4 stg6[kPfStages > 6 ? kPfStage : 1];
  __shared__ uint4 stg7[kPfStages > 7 ? kPfStage : 1];
  uint4* const stages[8] = {stg0, stg1, stg2, stg3, stg4, stg5, stg6, stg7};
  const int lane = threadIdx.x & 63;
  const int wave = wave_uniform(threadIdx.x >> 6);
  __builtin_assume(wave >= 0 && wave < kPfWaves);
  const int r = lane & 15, grp = lane >> 4;
  const int G = p.group;

  // (query block, kv head) of this workgroup: kv head fastest, so consecutive workgroups
  // (spread over the XCDs round robin) keep one head per XCD when num_kv_heads is a
  // multiple of 8, and the last query blocks of every head start first
  const int hkv = p.hq / G;
  const int g = wave_uniform(int(blockIdx.x) % hkv);
  const int blk = wave_uniform(p.total_blocks - 1 - int(blockIdx.x) / hkv);
  int lo = 0, hi = p.num_rows - 1, b = 0;
  while (lo <= hi) {
    const int mid = (lo + hi) >> 1;
    if (p.block_indptr[mid] <= blk) {
      b = mid;
      lo = mid + 1;
    } else {
      hi = mid - 1;
    }
  }
  b = wave_uniform(b);
  const int qb = blk - p.block_indptr[b];
  const int q0 = p.qo_indptr[b];
  const int q_len = p.qo_indptr[b + 1] - q0;
  const int list0 = p.kv_indptr[b];
  const int np = p.kv_indptr[b + 1] - list0;
  const int kv_len = max(np - 1, 0) * kPage + p.last_page_len[b];
  const int tpw = kPfRows / G;  // tokens per wave
  const int tok0 = qb * p.block_tokens;
  const int ntok = min(p.block_tokens, q_len - tok0);
  const int wt0 = tok0 + wave * tpw;
  const int wn = max(0, min(tpw, q_len - wt0));
  const int rows = wn * G;
  // keys of the block (all waves stage them) and of this wave
  const int shift = kv_len - q_len;
  const int blk_last = p.causal ? min(shift + tok0 + ntok - 1, kv_len - 1) : kv_len - 1;
  const int blk_pages = blk_last >= 0 ? blk_last / kPage + 1 : 0;
  const int steps = wave_uniform((blk_pages + 1) / 2);
  const int vlim = wave_uniform(min(kv_len, blk_pages * kPage));
  const int w_last = wave_uniform(rows > 0 ? (p.causal ? min(shift + wt0 + wn - 1, kv_len - 1) : kv_len - 1) : -1);
  const int w_min_limit = wave_uniform(p.causal ? min(shift + wt0, kv_len - 1) : kv_len - 1);

  // Q fragments (B operand of S^T = K . Q^T) and causal limits of the wave's rows
  bf16x8 qf[kPfTiles][4];
  int limit[kPfTiles];
#pragma unroll
  for (int t = 0; t < kPfTiles; ++t) {
    const int row = t * 16 + r;
    if (row < rows) {
      const int ti = row / G;
      const int hh = row - ti * G;
      const uint16_t* src = p.q + int64_t(q0 + wt0 + ti) * p.q_st + int64_t(g * G + hh) * p.q_sh;
#pragma unroll
      for (int c = 0; c < 4; ++c) qf[t][c] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(src + 32 * c + 8 * grp));
      limit[t] = p.causal ? min(shift + wt0 + ti, kv_len - 1) : kv_len - 1;
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) qf[t][c] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
      limit[t] = -1;
    }
  }
  // Per row (lane r of each tile): the running max m (base-2, scaled), the offset its
  // exponentials use (0 while the row has no key yet), the accumulators O^T, and this lane's
  // part of the row sum (fp32, over the lane's keys; the 4 lane groups are added at the end).
  float m[kPfTiles], m_use[kPfTiles], l[kPfTiles];
  f32x4 acc[kPfTiles][8];
#pragma unroll
  for (int t = 0; t < kPfTiles; ++t) {
    m[t] = kNegInfP;
    m_use[t] = 0.f;
    l[t] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Staging. A step's 16 KiB are 16 slots of 1 KiB (one load of 64 lanes x 16 B each): slot L
  // holds rows 4 (L & 3) .. 4 (L & 3) + 3 of kind L >> 2 (K rows of page 2s, its V rows, K rows
  // of page 2s + 1, its V rows) and lands at chunks 64 L .. 64 L + 63 of the stage buffer. They
  // travel from HBM straight into LDS (buffer_load ... lds). Wave w issues slots w * kPer ..
  // w * kPer + kPer - 1, all of one kind, so it needs one page id and one scalar buffer
  // descriptor per step; each lane fetches the global chunk that belongs at its LDS position.
  // K rows are placed with chunk c of row r at c ^ r (conflict-free column reads), V rows at
  // c ^ swz(r) (the transpose reads). Rows from vlim on (stale slots past kv_len, pages the
  // block does not reach) lie past the descriptor's range, which ends after the page's last
  // valid row (row stride >= 256 bytes, so a 16-byte chunk is wholly inside or wholly outside):
  // such loads write zeros into LDS, and the waves issue the same instructions on every step.
  constexpr int kPer = kPfStage / kPfThreads;  // 1 KiB loads per wave and step
  static_assert(kPer >= 1 && kPer <= 4, "a wave's slots of a step share one kind");
  const int kind = wave_uniform((wave * kPer) >> 2);
  const int my_page = kind >> 1;  // 0: page 2s of step s, 1: page 2s + 1
  const bool is_v = (kind & 1) != 0;
  const int row_bytes = int(p.c_st) * 2;
  int voff[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int crow = 4 * ((wave * kPer + i) & 3) + (lane >> 4), cpos = lane & 15;
    voff[i] = crow * row_bytes + (cpos ^ (is_v ? pf_swz(crow) : crow)) * 16;
  }
  const char* const kind_base = uniform_ptr(
      reinterpret_cast<const char*>(p.cache + int64_t(g) * p.c_sh + (is_v ? p.c_skv : int64_t(0))));
  const uint32_t page_bytes = uint32_t(p.c_sp) * 2u;  // below 2^32 (checked on the host)
  typedef const __attribute__((address_space(4))) int32_t* const_ids_t;
  const const_ids_t ids = (const_ids_t)(p.kv_indices + list0);
  // this wave's page of step k (clamped to the row's last page; steps past the block load nothing)
  auto page_id = [&](int k) -> int { return ids[min(2 * k + my_page, max(np - 1, 0))]; };
  // the barrier's wait: this wave's loads of the next step have landed, those of the
  // kPfStages - 2 steps after it may still be in flight (s_waitcnt vmcnt(n) lgkmcnt(0), gfx9
  // encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4 left at 7, lgkmcnt 11:8)
  constexpr int kPfWaitN = (kPfStages - 2) * kPer;
  constexpr int kPfWait = (kPfWaitN & 15) | ((kPfWaitN >> 4) << 14) | 0x70;
  auto issue = [&](uint4* buf, int k, int id) {
    // byte range of the page: its rows below vlim
    const int rows_valid = min(max(vlim - (k * kPfStepKeys + my_page * kPage), 0), kPage);
    const int span = rows_valid > 0 ? (rows_valid - 1) * row_bytes + 256 : 0;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(kind_base + uint64_t(uint32_t(id)) * page_bytes), (short)0, span, kPfBufferConfig);
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void*)(buf + (wave * kPer + i) * 64), 16, voff[i], 0, 0, 0);
  };
  // LDS release / acquire around the barrier without a memory fence: the fence would also wait
  // for the step loads in flight (they write LDS). The explicit wait covers this wave's loads of
  // the next step (2 * kPer later ones may stay in flight) and its LDS reads of this step's
  // buffer, which the loads issued after the barrier overwrite; the empty asm statements keep
  // the compiler from moving LDS accesses across the barrier.
  auto step_barrier = [&]() {
    __builtin_amdgcn_s_waitcnt(kPfWait);  // vmcnt((kPfStages - 2) * kPer), lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  const int vt_row = 4 * grp + (r >> 2);
  // S^T of the wave's current step: lane (r, grp) holds keys key0 + 4grp + i (sa) and
  // key0 + 16 + 4grp + i (sb); P of the step in bf16 for P.V
  f32x4 sa[kPfTiles], sb[kPfTiles];
  bf16x8 pf[kPfTiles];
  // this lane's K chunks (column reads) and V^T transpose reads, as chunk indices into a stage
  // buffer, computed once
  int kidx[4], vidx[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    kidx[c] = r * kPfRowChunks + ((4 * c + grp) ^ r);
    vidx[c] = kPfHalf + vt_row * kPfRowChunks + ((4 * c + (r & 3)) ^ pf_swz(vt_row));
  }
  auto scores = [&](const uint4* kb) {
    uint4 kr[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) kr[c] = kb[kidx[c]];
#pragma unroll
    for (int tt = 0; tt < kPfTiles; ++tt) {
      sa[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) sa[tt] = mfma_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[c]), qf[tt][c], sa[tt]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) kr[c] = kb[kPfPage + kidx[c]];
#pragma unroll
    for (int tt = 0; tt < kPfTiles; ++tt) {
      sb[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) sb[tt] = mfma_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[c]), qf[tt][c], sb[tt]);
    }
  };
  // online softmax over the step's 32 keys; the scale is folded into exp2's argument. The
  // running max moves only when some key exceeds it by more than kPfSlack (log2 units), so
  // exponentials stay below 2^kPfSlack. They are computed with the current offsets first: a
  // step on which no lane's sum of its 8 exponentials of a row exceeds 2^kPfSlack (so none of
  // them does) keeps them, and only otherwise (and on the first step, which sets every row's
  // max: key 0 is visible to every row) are the row maxima taken across lanes, the offsets
  // moved, the accumulators rescaled and the exponentials recomputed (a wave-uniform branch).
  auto softmax = [&](int s) {
    const int key0 = s * kPfStepKeys;
    const int pos = key0 + grp * 4;
    const bool need_mask = key0 + kPfStepKeys - 1 > w_min_limit;
    float x[kPfTiles][8];
#pragma unroll
    for (int tt = 0; tt < kPfTiles; ++tt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[tt][i] = sa[tt][i];
        x[tt][4 + i] = sb[tt][i];
      }
      if (need_mask) {
        const int d = limit[tt] - pos;  // keys pos + i with i <= d are visible
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[tt][i] = i <= d ? x[tt][i] : kNegInfP;
          x[tt][4 + i] = kPage + i <= d ? x[tt][4 + i] : kNegInfP;
        }
      }
    }
    float pv[kPfTiles][8], ps[kPfTiles];
    auto exponentials = [&]() {
#pragma unroll
      for (int tt = 0; tt < kPfTiles; ++tt) {
#pragma unroll
        for (int i = 0; i < 8; ++i) pv[tt][i] = __builtin_amdgcn_exp2f(fmaf(x[tt][i], p.scale_log2, -m_use[tt]));
        ps[tt] = ((pv[tt][0] + pv[tt][1]) + (pv[tt][2] + pv[tt][3])) + ((pv[tt][4] + pv[tt][5]) + (pv[tt][6] + pv[tt][7]));
      }
    };
    exponentials();
    bool over = s == 0;
#pragma unroll
    for (int tt = 0; tt < kPfTiles; ++tt) over |= ps[tt] > kPfSumLimit;
    if (__builtin_amdgcn_ballot_w64(over) != 0) {
#pragma unroll
      for (int tt = 0; tt < kPfTiles; ++tt) {
        float mx = fmaxf(fmaxf(fmaxf(x[tt][0], x[tt][1]), fmaxf(x[tt][2], x[tt][3])),
                         fmaxf(fmaxf(x[tt][4], x[tt][5]), fmaxf(x[tt][6], x[tt][7])));
        mx = max_xor32(max_xor16(mx)) * p.scale_log2;
        const float m_new = mx > m[tt] + kPfSlack ? mx : m[tt];
        const float mu = m_new == kNegInfP ? 0.f : m_new;
        // a row with no key before (m = -inf) has zero sums: alpha 0 keeps them zero
        const float a = __builtin_amdgcn_exp2f(m[tt] - mu);
        m[tt] = m_new;
        m_use[tt] = mu;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[tt][j] *= a;
        l[tt] *= a;
      }
      exponentials();
    }
#pragma unroll
    for (int tt = 0; tt < kPfTiles; ++tt) {
      uint4 w;
      w.x = pack_bf16x2_rne(pv[tt][0], pv[tt][1]);
      w.y = pack_bf16x2_rne(pv[tt][2], pv[tt][3]);
      w.z = pack_bf16x2_rne(pv[tt][4], pv[tt][5]);
      w.w = pack_bf16x2_rne(pv[tt][6], pv[tt][7]);
      pf[tt] = __builtin_bit_cast(bf16x8, w);
      l[tt] += ps[tt];
    }
  };
  // O^T += V^T . P^T with 16x16x32 MFMAs over the step's 32 keys: lane (r, grp) carries keys
  // 4grp..4grp+3 of both pages, the order P^T's fragment uses; V^T by transpose reads. Keys
  // from vlim on were requested out of range, which writes zeros into LDS, so 0 * stale never
  // reaches the sums.
  auto pv_update = [&](const uint4* kb) {
    const char* va = reinterpret_cast<const char*>(kb);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int off = vidx[j >> 1] * 16 + 8 * (j & 1);
      const uint2 wa = __builtin_bit_cast(
          uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(va + off)));
      const uint2 wb = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                     (__attribute__((address_space(3))) i16x4*)(va + kPfPage * 16 + off)));
      const bf16x8 vt = __builtin_bit_cast(bf16x8, make_uint4(wa.x, wa.y, wb.x, wb.y));
#pragma unroll
      for (int tt = 0; tt < kPfTiles; ++tt) acc[tt][j] = mfma_16x16x32_bf16(vt, pf[tt], acc[tt][j]);
    }
  };
  auto compute = [&](const uint4* kb, int s) {
    scores(kb);
    softmax(s);
    pv_update(kb);
  };

  // Pipeline over kPfStages LDS stage buffers (step k in buffer k % kPfStages, separate LDS
  // objects so the compiler can tell a load into one from a read of another): at the start of
  // step s the loads of step s + kPfStages - 1 go into the buffer step s - 1 used (free since
  // that step's barrier); the barrier at the end of step s waits for step s + 1's loads. Page
  // ids are scalar loads one step ahead of their use. Every step issues the same loads (steps
  // past the block read nothing: every chunk is out of range), so the wait count is the same
  // on every iteration.
  if (steps > 0) {
#pragma unroll
    for (int k = 0; k < kPfStages - 1; ++k) issue(stages[k], k, page_id(k));
    int next_id = page_id(kPfStages - 1);
    __builtin_amdgcn_s_waitcnt(kPfWait);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    auto body = [&](int s, uint4* cur, uint4* fill) {
      const int id = next_id;
      next_id = page_id(s + kPfStages);
      issue(fill, s + kPfStages - 1, id);
      if (s < steps && s * kPfStepKeys <= w_last) compute(cur, s);
      step_barrier();
    };
    for (int s = 0; s < steps; s += kPfStages) {
#pragma unroll
      for (int u = 0; u < kPfStages; ++u) body(s + u, stages[u], stages[(u + kPfStages - 1) % kPfStages]);
    }
  }

  // epilogue: normalise, write bf16 rows and the base-2 LSE
#pragma unroll
  for (int tt = 0; tt < kPfTiles; ++tt) {
    float lt = l[tt];
    lt += shfl_xor_f(lt, 16);
    lt += shfl_xor_f(lt, 32);
    const int row = tt * 16 + r;
    if (row >= rows) continue;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const float lse_v = lt > 0.f ? m[tt] + __builtin_log2f(lt) : kNegInfP;
    const int ti = row / G;
    const int head = g * G + (row - ti * G);
    const int token = q0 + wt0 + ti;
    uint16_t* dst = p.out + int64_t(token) * p.o_st + int64_t(head) * p.o_sh;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const f32x4 a0 = acc[tt][2 * c];
      const f32x4 a1 = acc[tt][2 * c + 1];
      uint4 w;
      w.x = pack_bf16x2_rne(a0[0] * inv, a0[1] * inv);
      w.y = pack_bf16x2_rne(a0[2] * inv, a0[3] * inv);
      w.z = pack_bf16x2_rne(a1[0] * inv, a1[1] * inv);
      w.w = pack_bf16x2_rne(a1[2] * inv, a1[3] * inv);
      *reinterpret_cast<uint4*>(dst + 32 * c + 8 * grp) = w;
    }
    if (grp == 0 && p.lse != nullptr) p.lse[int64_t(token) * p.hq + head] = lse_v;
  }
}

inline bool pf_al16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace
}  // namespace aspire

extern "C" int aspire_prefill_block_tokens(int32_t num_qo_heads, int32_t num_kv_heads) {
  using namespace aspire;
  if (num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads != 0) return 0;
  const int G = num_qo_heads / num_kv_heads;
  if (G > kPfRows || kPfRows % G != 0) return 0;
  return kPfBlockRows / G;
}

extern "C" int aspire_prefill_run(const aspire_prefill_args* a, void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(a != nullptr, "null argument");
  ASPIRE_CHECK_ARG(a->head_dim == kHeadDim && a->page_size == kPage, "head_dim 128 and page_size 16 only");
  const int bt = aspire_prefill_block_tokens(a->num_qo_heads, a->num_kv_heads);
  ASPIRE_CHECK_ARG(bt > 0 && int64_t(a->total_blocks) * a->num_kv_heads < (int64_t(1) << 31),
                   "num_qo_heads must be a multiple of num_kv_heads with a group dividing a wave's query rows "
                   "(aspire_prefill_block_tokens > 0), and query blocks x kv heads below 2^31");
  ASPIRE_CHECK_ARG(a->block_tokens == bt, "block_tokens must be aspire_prefill_block_tokens(hq, hkv)");
  ASPIRE_CHECK_ARG(a->num_rows >= 0 && a->total_blocks >= 0, "bad sizes");
  ASPIRE_CHECK_ARG(a->cache_stride_t > 0 && a->cache_stride_t < (int64_t(1) << 26),
                   "cache_stride_t must be positive and below 2^26 elements (a page's rows span 32-bit offsets)");
  ASPIRE_CHECK_ARG(a->cache_stride_p > 0 && a->cache_stride_p < (int64_t(1) << 31),
                   "cache_stride_p must be positive and below 2^31 elements");
  // by the bit pattern (positive, finite, below 1e30), which no floating-point flag can fold
  const uint32_t scale_bits = __builtin_bit_cast(uint32_t, a->sm_scale);
  ASPIRE_CHECK_ARG(scale_bits > 0u && scale_bits < __builtin_bit_cast(uint32_t, 1e30f),
                   "sm_scale must be positive and finite");
  if (a->num_rows == 0 || a->total_blocks == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(a->q && a->kv_cache && a->kv_indices && a->kv_indptr && a->kv_last_page_len && a->qo_indptr &&
                       a->block_indptr && a->out,
                   "null pointer");
  ASPIRE_CHECK_ARG(pf_al16(a->q) && pf_al16(a->kv_cache) && pf_al16(a->out), "q, kv_cache and out must be 16-byte aligned");
  ASPIRE_CHECK_ARG(a->q_stride_t % 8 == 0 && a->q_stride_h % 8 == 0 && a->out_stride_t % 8 == 0 &&
                       a->out_stride_h % 8 == 0 && a->cache_stride_p % 8 == 0 && a->cache_stride_kv % 8 == 0 &&
                       a->cache_stride_t % 8 == 0 && a->cache_stride_h % 8 == 0,
                   "strides must be multiples of 8 elements");
  PrefillParams p;
  p.q = static_cast<const uint16_t*>(a->q);
  p.q_st = a->q_stride_t;
  p.q_sh = a->q_stride_h;
  p.cache = static_cast<const uint16_t*>(a->kv_cache);
  p.c_sp = a->cache_stride_p;
  p.c_skv = a->cache_stride_kv;
  p.c_st = a->cache_stride_t;
  p.c_sh = a->cache_stride_h;
  p.kv_indices = a->kv_indices;
  p.kv_indptr = a->kv_indptr;
  p.last_page_len = a->kv_last_page_len;
  p.qo_indptr = a->qo_indptr;
  p.block_indptr = a->block_indptr;
  p.num_rows = a->num_rows;
  p.total_blocks = a->total_blocks;
  p.block_tokens = bt;
  p.out = static_cast<uint16_t*>(a->out);
  p.o_st = a->out_stride_t;
  p.o_sh = a->out_stride_h;
  p.lse = a->lse;
  p.hq = a->num_qo_heads;
  p.group = a->num_qo_heads / a->num_kv_heads;
  p.scale_log2 = a->sm_scale * 1.4426950408889634f;
  p.causal = a->causal;
  hipLaunchKernelGGL(prefill_kernel, dim3(a->total_blocks * a->num_kv_heads), dim3(kPfThreads), 0,
                     static_cast<hipStream_t>(stream), p);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}
