// (a2) Mixed draft/verify page list: one workgroup per row computes its
// indptr prefix (a block reduction over the preceding rows' counts) and copies
// its page ids; one launch replaces the reference's cumsum + Triton copy.
#include "common.h"

namespace aspire {
namespace {

struct PageListParams {
  const void* mode_flags;
  int32_t mode_size;
  const int32_t* draft;
  int64_t draft_width, draft_total;
  const int32_t* verify;
  int64_t verify_width, verify_total;
  const int32_t* draft_n;
  const int32_t* verify_n;
  int32_t batch;
  int32_t* indices;
  int64_t capacity;
  int32_t* indptr;
  int32_t fill_to;
};

__device__ __forceinline__ bool is_draft_row(const PageListParams& p, int b) {
  if (p.mode_size == 1) return static_cast<const uint8_t*>(p.mode_flags)[b] == 0;
  if (p.mode_size == 8) return static_cast<const int64_t*>(p.mode_flags)[b] == 0;
  return static_cast<const int32_t*>(p.mode_flags)[b] == 0;
}

__device__ __forceinline__ int row_pages(const PageListParams& p, int b) {
  return is_draft_row(p, b) ? p.draft_n[b] : p.verify_n[b];
}

__global__ __launch_bounds__(256) void page_list_kernel(PageListParams p) {
  __shared__ long long partial[256];
  const int b = blockIdx.x;
  long long acc = 0;
  for (int c = threadIdx.x; c < b; c += blockDim.x) acc += row_pages(p, c);
  partial[threadIdx.x] = acc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) partial[threadIdx.x] += partial[threadIdx.x + s];
    __syncthreads();
  }
  const long long start = partial[0];
  const int n = row_pages(p, b);
  const long long end = start + n;
  if (threadIdx.x == 0) {
    if (b == 0) p.indptr[0] = 0;
    p.indptr[b + 1] = static_cast<int32_t>(end);
    if (b == p.batch - 1)
      for (int i = p.batch + 1; i < p.fill_to; ++i) p.indptr[i] = static_cast<int32_t>(end);
  }
  if (n <= 0) return;
  const bool draft = is_draft_row(p, b);
  const int32_t* src = draft ? p.draft : p.verify;
  const int64_t base = int64_t(b) * (draft ? p.draft_width : p.verify_width);
  const int64_t total = draft ? p.draft_total : p.verify_total;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int64_t si = base + i;
    const long long di = start + i;
    if (si < total && di < p.capacity) p.indices[di] = src[si];
  }
}

__global__ void page_list_empty_kernel(int32_t* indptr, int32_t fill_to) {
  for (int i = threadIdx.x; i < max(fill_to, 1); i += blockDim.x) indptr[i] = 0;
}

}  // namespace
}  // namespace aspire

extern "C" int aspire_build_mixed_page_list(const void* mode_flags, int32_t mode_flags_elem_size,
                                            const int32_t* draft_indices, int64_t draft_width,
                                            int64_t draft_rows, const int32_t* verify_indices,
                                            int64_t verify_width, int64_t verify_rows,
                                            const int32_t* draft_num_pages,
                                            const int32_t* verify_num_pages, int32_t batch,
                                            int32_t* paged_kv_indices, int64_t indices_capacity,
                                            int32_t* paged_kv_indptr, int32_t indptr_fill_to,
                                            void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(batch >= 0, "negative batch");
  ASPIRE_CHECK_ARG(paged_kv_indptr != nullptr, "null indptr");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (batch == 0) {
    hipLaunchKernelGGL(page_list_empty_kernel, dim3(1), dim3(64), 0, s, paged_kv_indptr,
                       indptr_fill_to);
    ASPIRE_CHECK_LAUNCH();
    return ASPIRE_OK;
  }
  ASPIRE_CHECK_ARG(mode_flags && draft_indices && verify_indices && draft_num_pages &&
                       verify_num_pages && paged_kv_indices,
                   "null pointer");
  ASPIRE_CHECK_ARG(mode_flags_elem_size == 1 || mode_flags_elem_size == 4 ||
                       mode_flags_elem_size == 8,
                   "mode_flags element size must be 1, 4 or 8");
  PageListParams p;
  p.mode_flags = mode_flags;
  p.mode_size = mode_flags_elem_size;
  p.draft = draft_indices;
  p.draft_width = draft_width;
  p.draft_total = draft_width * draft_rows;
  p.verify = verify_indices;
  p.verify_width = verify_width;
  p.verify_total = verify_width * verify_rows;
  p.draft_n = draft_num_pages;
  p.verify_n = verify_num_pages;
  p.batch = batch;
  p.indices = paged_kv_indices;
  p.capacity = indices_capacity;
  p.indptr = paged_kv_indptr;
  p.fill_to = indptr_fill_to;
  hipLaunchKernelGGL(page_list_kernel, dim3(batch), dim3(256), 0, s, p);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}
