// (a2) Mixed draft/verify page list: one workgroup per segment computes its
// indptr prefix (a block reduction over the preceding segments' counts) and
// copies its page ids; one launch replaces the reference's cumsum + Triton copy.
//
// A segment is a row (heads == 1, the reference's lists) or one (row, kv head)
// pair (heads == H_kv): draft segments then copy their own head's selection
// and verify segments the row's block table, once per head or, with `share`,
// once per row (every head of the row starts at the same entry).
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
  int32_t heads;  // segments per row
  int32_t share;  // verify rows: one list for all heads
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

// Entries segment s adds to the running offset. Segment s belongs to row
// s / heads; draft counts are per segment, verify counts per row. A shared
// verify row adds its list after its last head, so all its heads start at the
// row's first entry.
__device__ __forceinline__ int seg_advance(const PageListParams& p, int s) {
  const int b = s / p.heads;
  if (is_draft_row(p, b)) return p.draft_n[s];
  if (p.share && s - b * p.heads != p.heads - 1) return 0;
  return p.verify_n[b];
}

__global__ __launch_bounds__(256) void page_list_kernel(PageListParams p) {
  __shared__ long long partial[256];
  const int sg = blockIdx.x;
  const int b = sg / p.heads;
  const int segs = p.batch * p.heads;
  long long acc = 0;
  for (int c = threadIdx.x; c < sg; c += blockDim.x) acc += seg_advance(p, c);
  partial[threadIdx.x] = acc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) partial[threadIdx.x] += partial[threadIdx.x + s];
    __syncthreads();
  }
  const long long start = partial[0];
  const long long end = start + seg_advance(p, sg);
  // indptr[s] = first entry of segment s; indptr[segs] (and the fill) = total
  if (threadIdx.x == 0) {
    p.indptr[sg] = static_cast<int32_t>(start);
    if (sg == segs - 1)
      for (int i = segs; i < max(p.fill_to, segs + 1); ++i) p.indptr[i] = static_cast<int32_t>(end);
  }
  const bool draft = is_draft_row(p, b);
  const int n = draft ? p.draft_n[sg] : (p.share && sg != b * p.heads ? 0 : p.verify_n[b]);
  if (n <= 0) return;
  const int32_t* src = draft ? p.draft : p.verify;
  const int64_t base = draft ? int64_t(sg) * p.draft_width : int64_t(b) * p.verify_width;
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

namespace aspire {
namespace {

int launch_page_list(const void* mode_flags, int32_t mode_flags_elem_size, const int32_t* draft_indices,
                     int64_t draft_width, int64_t draft_rows, const int32_t* verify_indices, int64_t verify_width,
                     int64_t verify_rows, const int32_t* draft_num_pages, const int32_t* verify_num_pages,
                     int32_t batch, int32_t heads, int32_t share, int32_t* paged_kv_indices,
                     int64_t indices_capacity, int32_t* paged_kv_indptr, int32_t indptr_fill_to, void* stream) {
  ASPIRE_CHECK_ARG(batch >= 0, "negative batch");
  ASPIRE_CHECK_ARG(heads >= 1, "heads must be positive");
  ASPIRE_CHECK_ARG(paged_kv_indptr != nullptr, "null indptr");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (batch == 0) {
    hipLaunchKernelGGL(page_list_empty_kernel, dim3(1), dim3(64), 0, s, paged_kv_indptr, indptr_fill_to);
    ASPIRE_CHECK_LAUNCH();
    return ASPIRE_OK;
  }
  ASPIRE_CHECK_ARG(int64_t(batch) * heads < (int64_t(1) << 31), "too many segments");
  ASPIRE_CHECK_ARG(mode_flags && draft_indices && verify_indices && draft_num_pages && verify_num_pages &&
                       paged_kv_indices,
                   "null pointer");
  ASPIRE_CHECK_ARG(mode_flags_elem_size == 1 || mode_flags_elem_size == 4 || mode_flags_elem_size == 8,
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
  p.heads = heads;
  p.share = share != 0 && heads > 1;
  p.indices = paged_kv_indices;
  p.capacity = indices_capacity;
  p.indptr = paged_kv_indptr;
  p.fill_to = indptr_fill_to;
  hipLaunchKernelGGL(page_list_kernel, dim3(batch * heads), dim3(256), 0, s, p);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
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
  return aspire::launch_page_list(mode_flags, mode_flags_elem_size, draft_indices, draft_width, draft_rows,
                                  verify_indices, verify_width, verify_rows, draft_num_pages, verify_num_pages,
                                  batch, 1, 0, paged_kv_indices, indices_capacity, paged_kv_indptr,
                                  indptr_fill_to, stream);
}

extern "C" int aspire_build_head_page_lists(const void* mode_flags, int32_t mode_flags_elem_size,
                                            const int32_t* selected, int64_t selected_width,
                                            const int32_t* selected_counts, const int32_t* verify_indices,
                                            int64_t verify_width, int64_t verify_rows,
                                            const int32_t* verify_num_pages, int32_t batch, int32_t num_kv_heads,
                                            int32_t share_verify, int32_t* paged_kv_indices,
                                            int64_t indices_capacity, int32_t* paged_kv_indptr,
                                            int32_t indptr_fill_to, void* stream) {
  return aspire::launch_page_list(mode_flags, mode_flags_elem_size, selected, selected_width,
                                  int64_t(batch) * num_kv_heads, verify_indices, verify_width, verify_rows,
                                  selected_counts, verify_num_pages, batch, num_kv_heads, share_verify,
                                  paged_kv_indices, indices_capacity, paged_kv_indptr, indptr_fill_to, stream);
}
