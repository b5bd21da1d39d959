// (f2) QK RMSNorm + rotary permute + interleaved RoPE + paged KV append, one launch.
//
// Per layer the reference runs q_norm, k_norm, two permutes, mylib::rope and
// mylib::update_kv_padded (aspire/models/sparse_draft_transformer.py:149-171):
// six launches and four round trips of q / k through HBM. Here one wave
// handles one head of one token (lane i owns rotated pair i, i.e. dims 2i and
// 2i+1 after the permute): it normalises, rotates and writes q in place and
// k / v into the page pool at the token's append position.
//
//   * RMSNorm (transformer.py:505-516): fp32 sum of squares (wave sum),
//     x * (1 / sqrt(mean + eps)) rounded to bf16, times the bf16 weight,
//     rounded again;
//   * permute (transformer.py:360-364): output pair i takes input dims i and
//     i + D/2 (the norm weight follows the input dim);
//   * RoPE, FlashInfer's interleaved convention (mixed_transformer.py:159-198):
//     angle = fp32(position) * fp32 frequency (the host computes the D/2
//     frequencies once, including the Llama 3.1 smoothing), accurate sincosf,
//     (a, b) -> (a cos - b sin, b cos + a sin) in fp32, rounded to bf16;
//   * append: the row / slot rule of the plain append (append_locate).
#include <algorithm>
#include <cmath>

#include "common.h"

namespace aspire {
namespace {

constexpr int kPairs = kHeadDim / 2;

struct RopeParams {
  uint16_t* q;
  int64_t q_st, q_sh;
  uint16_t* k;
  int64_t k_st, k_sh;
  const uint16_t* v;
  int64_t v_st, v_sh;
  int32_t hq, hkv;
  const uint16_t* q_w;
  const uint16_t* k_w;
  float eps;
  int32_t permute;
  float freq[kPairs];
  const int32_t* indptr;
  const int32_t* offsets;
  int32_t num_rows;
  uint16_t* cache;
  int64_t c_sp, c_skv, c_st, c_sh;
  int32_t page_size;
  const int32_t* page_indices;
  const int32_t* page_indptr;
  const int32_t* last_page_len;
  int32_t num_seq;
  int32_t write_k;
};

__device__ __forceinline__ float bf16_to_f(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }
__device__ __forceinline__ uint16_t f_to_bf16(float f) { return static_cast<uint16_t>(bf16_rne_bits(f)); }

constexpr int kHeadsPerBlock = 4;  // one wave per head

// Grid (tokens, ceil((hq + hkv) / 4)): wave w of block (tok, hb) prepares
// head 4 * hb + w of token tok (q heads first, then k heads) and, when
// 4 * hb + w < hkv, copies that v head into the page.
__global__ __launch_bounds__(256) void qk_norm_rope_append_kernel(RopeParams p) {
  const int tok = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int h = blockIdx.y * kHeadsPerBlock + wave;
  // rope position: row b of indptr owns tok (last b with indptr[b] <= tok < indptr[b + 1])
  int pos = -1;
  {
    const int b = wave_last_le(p.indptr, p.num_rows, tok);
    if (b >= 0 && tok < p.indptr[b + 1]) pos = p.offsets[b] + tok - p.indptr[b];
  }
  pos = wave_uniform(pos);
  int entry = -1, slot = 0;
  const bool append = p.cache != nullptr &&
                      append_locate(p.indptr, p.num_seq, p.page_indptr, p.last_page_len, p.page_size, tok, entry, slot);
  uint16_t* page_k = nullptr;
  if (append) page_k = p.cache + int64_t(p.page_indices[entry]) * p.c_sp + int64_t(slot) * p.c_st;

  if (h < p.hq + p.hkv) {
    float c = 1.f, s = 0.f;
    if (pos >= 0) sincosf(static_cast<float>(pos) * p.freq[lane], &s, &c);
    const int in0 = p.permute ? lane : 2 * lane;
    const int in1 = p.permute ? lane + kPairs : 2 * lane + 1;
    const bool is_q = h < p.hq;
    uint16_t* row = is_q ? p.q + int64_t(tok) * p.q_st + int64_t(h) * p.q_sh
                         : p.k + int64_t(tok) * p.k_st + int64_t(h - p.hq) * p.k_sh;
    float x0 = bf16_to_f(row[in0]);
    float x1 = bf16_to_f(row[in1]);
    const uint16_t* w = is_q ? p.q_w : p.k_w;
    if (w != nullptr) {
      const float ms = wave_sum_f(x0 * x0 + x1 * x1) / float(kHeadDim);
      const float r = 1.f / sqrtf(ms + p.eps);
      x0 = bf16_to_f(f_to_bf16(bf16_to_f(f_to_bf16(x0 * r)) * bf16_to_f(w[in0])));
      x1 = bf16_to_f(f_to_bf16(bf16_to_f(f_to_bf16(x1 * r)) * bf16_to_f(w[in1])));
    }
    float y0 = x0, y1 = x1;
    if (pos >= 0) {
      y0 = x0 * c - x1 * s;
      y1 = x1 * c + x0 * s;
    }
    const uint32_t packed = uint32_t(f_to_bf16(y0)) | (uint32_t(f_to_bf16(y1)) << 16);
    // every lane has read its inputs before any lane stores (one wave per head)
    if (is_q || p.write_k) *reinterpret_cast<uint32_t*>(row + 2 * lane) = packed;
    if (!is_q && append)
      *reinterpret_cast<uint32_t*>(page_k + int64_t(h - p.hq) * p.c_sh + 2 * lane) = packed;
  }
  if (append && p.v != nullptr && h < p.hkv && lane < kHeadDim / 8) {
    uint16_t* page_v = page_k + p.c_skv;
    const uint16_t* src = p.v + int64_t(tok) * p.v_st;
    *reinterpret_cast<uint4*>(page_v + int64_t(h) * p.c_sh + lane * 8) =
        *reinterpret_cast<const uint4*>(src + int64_t(h) * p.v_sh + lane * 8);
  }
}

inline bool aligned(const void* ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0; }

}  // namespace
}  // namespace aspire

extern "C" int aspire_rope_frequencies(int32_t head_dim, float rope_theta, float rope_scale, int32_t llama31,
                                       float low_freq_factor, float high_freq_factor, float old_context_len,
                                       float* out) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(out && head_dim > 0 && head_dim % 2 == 0, "bad arguments");
  ASPIRE_CHECK_ARG(rope_theta > 0.f && rope_scale > 0.f, "rope_theta and rope_scale must be positive");
  const double two_pi = 6.283185307179586;
  for (int i = 0; i < head_dim / 2; ++i) {
    const double f = std::pow(double(rope_theta), -2.0 * i / head_dim);
    double g = f / rope_scale;
    if (llama31) {
      // Llama 3.1: unchanged above the high-frequency cut, divided by the scale
      // below the low-frequency cut, interpolated in between
      const double wavelen = two_pi / f;
      if (wavelen < double(old_context_len) / high_freq_factor) {
        g = f;
      } else if (wavelen <= double(old_context_len) / low_freq_factor) {
        const double sm = (old_context_len / wavelen - low_freq_factor) / (double(high_freq_factor) - low_freq_factor);
        g = (1.0 - sm) * f / rope_scale + sm * f;
      }
    }
    out[i] = static_cast<float>(g);
  }
  return ASPIRE_OK;
}

extern "C" int aspire_qk_norm_rope_append(const aspire_rope_args* a, void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(a != nullptr, "null arguments");
  ASPIRE_CHECK_ARG(a->head_dim == kHeadDim, "head_dim must be 128");
  ASPIRE_CHECK_ARG(a->total_tokens >= 0 && a->num_qo_heads >= 0 && a->num_kv_heads >= 0, "bad sizes");
  if (a->total_tokens == 0 || a->num_qo_heads + a->num_kv_heads == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG((a->num_qo_heads == 0 || a->q) && (a->num_kv_heads == 0 || a->k), "null q / k");
  ASPIRE_CHECK_ARG(a->num_rows >= 0 && (a->num_rows == 0 || (a->indptr && a->offsets)), "null indptr / offsets");
  ASPIRE_CHECK_ARG((a->q_norm_weight == nullptr) == (a->k_norm_weight == nullptr),
                   "q and k norm weights go together");
  ASPIRE_CHECK_ARG(aligned(a->q, 4) && aligned(a->k, 4) && a->q_stride_h % 2 == 0 && a->k_stride_h % 2 == 0 &&
                       a->q_stride_t % 2 == 0 && a->k_stride_t % 2 == 0,
                   "q / k rows must be 4-byte aligned");
  RopeParams p;
  p.q = static_cast<uint16_t*>(a->q);
  p.q_st = a->q_stride_t;
  p.q_sh = a->q_stride_h;
  p.k = static_cast<uint16_t*>(a->k);
  p.k_st = a->k_stride_t;
  p.k_sh = a->k_stride_h;
  p.v = static_cast<const uint16_t*>(a->v);
  p.v_st = a->v_stride_t;
  p.v_sh = a->v_stride_h;
  p.hq = a->num_qo_heads;
  p.hkv = a->num_kv_heads;
  p.q_w = static_cast<const uint16_t*>(a->q_norm_weight);
  p.k_w = static_cast<const uint16_t*>(a->k_norm_weight);
  p.eps = a->norm_eps;
  p.permute = a->permute && a->q_norm_weight != nullptr;
  const int rc = aspire_rope_frequencies(kHeadDim, a->rope_theta, a->rope_scale, a->llama31, a->low_freq_factor,
                                         a->high_freq_factor, a->old_context_len, p.freq);
  if (rc != ASPIRE_OK) return rc;
  p.indptr = a->indptr;
  p.offsets = a->offsets;
  p.num_rows = a->num_rows;
  p.cache = static_cast<uint16_t*>(a->kv_cache);
  p.c_sp = a->cache_stride_p;
  p.c_skv = a->cache_stride_kv;
  p.c_st = a->cache_stride_t;
  p.c_sh = a->cache_stride_h;
  p.page_size = a->page_size;
  p.page_indices = a->kv_page_indices;
  p.page_indptr = a->kv_page_indptr;
  p.last_page_len = a->kv_last_page_len;
  p.num_seq = a->num_seq;
  p.write_k = a->write_k;
  if (p.cache != nullptr) {
    ASPIRE_CHECK_ARG(a->num_seq > 0 && a->num_seq <= a->num_rows, "append rows must be a prefix of the rope rows");
    ASPIRE_CHECK_ARG(a->kv_page_indices && a->kv_page_indptr && a->kv_last_page_len, "null page table");
    ASPIRE_CHECK_ARG(a->page_size > 0, "page_size must be positive");
    ASPIRE_CHECK_ARG(aligned(a->kv_cache, 16) && a->cache_stride_p % 8 == 0 && a->cache_stride_kv % 8 == 0 &&
                         a->cache_stride_t % 8 == 0 && a->cache_stride_h % 8 == 0,
                     "cache must be 16-byte aligned with strides in multiples of 8 elements");
    ASPIRE_CHECK_ARG(a->v == nullptr || (aligned(a->v, 16) && a->v_stride_t % 8 == 0 && a->v_stride_h % 8 == 0),
                     "v rows must be 16-byte aligned");
  }
  const int head_blocks = (std::max(a->num_qo_heads + a->num_kv_heads, a->num_kv_heads) + kHeadsPerBlock - 1) /
                          kHeadsPerBlock;
  hipLaunchKernelGGL(qk_norm_rope_append_kernel, dim3(a->total_tokens, head_blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), p);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}
