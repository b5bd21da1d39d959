// (a1) Paged KV append: one workgroup per appended token scatters its K and V
// rows (all kv heads) into the page pool through the page table. The row /
// position computation of FlashInfer's get_seq_lens and
// get_batch_indices_positions_kernel is folded in (closed form, one binary
// search over append_indptr per token), so the reference's three launches
// become one. Pure byte copy: bit-exact by construction.
#include "common.h"

namespace aspire {
namespace {

struct AppendParams {
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sn, k_sh, v_sn, v_sh;
  const int32_t* append_indptr;
  const int32_t* kv_indices;
  const int32_t* kv_indptr;
  const int32_t* last_page_len;
  int32_t num_seq;
  uint16_t* cache;
  int64_t c_sp, c_skv, c_st, c_sh;
  int32_t num_heads;
  int32_t page_size;
};

template <bool kVec>
__global__ __launch_bounds__(256) void append_kernel(AppendParams p) {
  const int tok = blockIdx.x;
  int list_idx, slot;
  if (!append_locate(p.append_indptr, p.num_seq, p.kv_indptr, p.last_page_len, p.page_size, tok, list_idx, slot))
    return;
  const int64_t phys = p.kv_indices[list_idx];
  uint16_t* dst_k = p.cache + phys * p.c_sp + int64_t(slot) * p.c_st;
  uint16_t* dst_v = dst_k + p.c_skv;
  const uint16_t* src_k = p.k + int64_t(tok) * p.k_sn;
  const uint16_t* src_v = p.v + int64_t(tok) * p.v_sn;
  if (kVec) {
    // 16 x 16B chunks per head row, K and V.
    const int units = p.num_heads * 16;
    for (int u = threadIdx.x; u < 2 * units; u += blockDim.x) {
      const int which = u >= units;
      const int uu = which ? u - units : u;
      const int h = uu >> 4, c = (uu & 15) * 8;
      const uint16_t* src = which ? src_v + h * p.v_sh + c : src_k + h * p.k_sh + c;
      uint16_t* dst = (which ? dst_v : dst_k) + h * p.c_sh + c;
      *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
    }
  } else {
    const int units = p.num_heads * kHeadDim;
    for (int u = threadIdx.x; u < 2 * units; u += blockDim.x) {
      const int which = u >= units;
      const int uu = which ? u - units : u;
      const int h = uu / kHeadDim, d = uu % kHeadDim;
      const uint16_t* src = which ? src_v + h * p.v_sh + d : src_k + h * p.k_sh + d;
      uint16_t* dst = (which ? dst_v : dst_k) + h * p.c_sh + d;
      *dst = *src;
    }
  }
}

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace
}  // namespace aspire

extern "C" int aspire_paged_kv_append(const void* k, const void* v, int64_t k_stride_n,
                                      int64_t k_stride_h, int64_t v_stride_n, int64_t v_stride_h,
                                      const int32_t* append_indptr, const int32_t* kv_page_indices,
                                      const int32_t* kv_page_indptr,
                                      const int32_t* kv_last_page_len, int32_t num_seq,
                                      void* kv_cache, int64_t cache_stride_p,
                                      int64_t cache_stride_kv, int64_t cache_stride_t,
                                      int64_t cache_stride_h, int32_t total_tokens,
                                      int32_t num_heads, int32_t head_dim, int32_t page_size,
                                      void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(total_tokens >= 0 && num_seq >= 0 && num_heads > 0, "bad sizes");
  ASPIRE_CHECK_ARG(head_dim == kHeadDim, "head_dim must be 128");
  ASPIRE_CHECK_ARG(page_size > 0, "page_size must be positive");
  if (total_tokens == 0 || num_seq == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(k && v && kv_cache && append_indptr && kv_page_indices && kv_page_indptr &&
                       kv_last_page_len,
                   "null pointer");
  AppendParams p;
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.k_sn = k_stride_n;
  p.k_sh = k_stride_h;
  p.v_sn = v_stride_n;
  p.v_sh = v_stride_h;
  p.append_indptr = append_indptr;
  p.kv_indices = kv_page_indices;
  p.kv_indptr = kv_page_indptr;
  p.last_page_len = kv_last_page_len;
  p.num_seq = num_seq;
  p.cache = static_cast<uint16_t*>(kv_cache);
  p.c_sp = cache_stride_p;
  p.c_skv = cache_stride_kv;
  p.c_st = cache_stride_t;
  p.c_sh = cache_stride_h;
  p.num_heads = num_heads;
  p.page_size = page_size;
  const bool vec = aligned16(k) && aligned16(v) && aligned16(kv_cache) && (k_stride_n % 8 == 0) &&
                   (k_stride_h % 8 == 0) && (v_stride_n % 8 == 0) && (v_stride_h % 8 == 0) &&
                   (cache_stride_p % 8 == 0) && (cache_stride_kv % 8 == 0) &&
                   (cache_stride_t % 8 == 0) && (cache_stride_h % 8 == 0);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vec)
    hipLaunchKernelGGL(append_kernel<true>, dim3(total_tokens), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(append_kernel<false>, dim3(total_tokens), dim3(256), 0, s, p);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}
