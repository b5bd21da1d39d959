// (d) On-box HBM calibration: the bandwidth the attention kernel's roofline fraction is read
// against, measured on the box it runs on, beside the published 8 TB/s.
//
// * stream_read_kernel reads a buffer once as 1 KiB rows, one 128-bit non-temporal buffer load
//   per lane (a whole contiguous 1 KiB per wave instruction, R rows in flight per wave): the
//   access of the attention kernel's workgroup-staged K/V path. Consecutive waves take
//   consecutive rows, so the grid sweeps the buffer front to back. The loads feed an XOR that
//   reaches memory only through a store under a data-dependent condition, so none is dropped.
//   The best rows in flight depend on the grid (measured on MI355X: 2 rows at 3 workgroups per
//   CU, 4 at 1.5, 8 at 0.75-1 each reach 7.2-7.4 TB/s, other pairs 5.3-7.1), so callers sweep
//   both and keep the best.
// * copy_kernel copies a buffer with 128-bit loads and stores, R chunks in flight per thread
//   (read + write traffic).
#include "common.h"

namespace aspire {
namespace {

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
constexpr uint32_t kProbeBufferConfig = 0x00020000u;  // gfx9 raw buffer dword 3
constexpr int kProbeThreads = 256;
constexpr int kRowBytes = 1024;

__device__ __forceinline__ uint32_t load_row_xor(const char* row, int lane) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(row), (short)0, kRowBytes, kProbeBufferConfig);
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16, 0, 2);
  return v.x ^ v.y ^ v.z ^ v.w;
}

template <int R>
__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const char* src, int64_t rows, uint32_t* sink) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = int64_t(gridDim.x) * (kProbeThreads / 64);
  int64_t r = wave_uniform(blockIdx.x * (kProbeThreads / 64) + (threadIdx.x >> 6));
  uint32_t acc = 0;
  for (; r + (R - 1) * waves < rows; r += R * waves) {
    uint32_t v[R];
#pragma unroll
    for (int k = 0; k < R; ++k) v[k] = load_row_xor(src + (r + k * waves) * kRowBytes, lane);
#pragma unroll
    for (int k = 0; k < R; ++k) acc ^= v[k];
  }
  for (; r < rows; r += waves) acc ^= load_row_xor(src + r * kRowBytes, lane);
  if (acc == 0x9e3779b9u) sink[blockIdx.x * kProbeThreads + threadIdx.x] = acc;
}

template <int R>
__global__ __launch_bounds__(kProbeThreads) void copy_kernel(const uint4* src, uint4* dst, int64_t n16) {
  const int64_t stride = int64_t(gridDim.x) * kProbeThreads;
  int64_t i = int64_t(blockIdx.x) * kProbeThreads + threadIdx.x;
  for (; i + (R - 1) * stride < n16; i += R * stride) {
    uint4 v[R];
#pragma unroll
    for (int k = 0; k < R; ++k) v[k] = src[i + k * stride];
#pragma unroll
    for (int k = 0; k < R; ++k) dst[i + k * stride] = v[k];
  }
  for (; i < n16; i += stride) dst[i] = src[i];
}

}  // namespace
}  // namespace aspire

extern "C" int aspire_bandwidth_probe(int32_t mode, const void* src, int64_t bytes, void* dst, int64_t dst_bytes,
                                      int32_t workgroups, int32_t in_flight, void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(mode == 0 || mode == 1, "mode must be 0 (streaming read) or 1 (copy)");
  ASPIRE_CHECK_ARG(in_flight == 1 || in_flight == 2 || in_flight == 4 || in_flight == 8 || in_flight == 16,
                   "in_flight must be 1, 2, 4, 8 or 16");
  ASPIRE_CHECK_ARG(bytes >= 0 && bytes % kRowBytes == 0, "bytes must be a non-negative multiple of 1024");
  ASPIRE_CHECK_ARG(workgroups > 0 && workgroups <= (1 << 20), "workgroups must be in [1, 2^20]");
  if (bytes == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(src && dst, "null pointer");
  ASPIRE_CHECK_ARG(dst_bytes >= (mode == 0 ? int64_t(workgroups) * kProbeThreads * 4 : bytes),
                   "dst too small (a streaming read needs workgroups * 1024 bytes of sink, a copy `bytes`)");
  ASPIRE_CHECK_ARG((reinterpret_cast<uintptr_t>(src) & 15) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0,
                   "src and dst must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const char* rs = static_cast<const char*>(src);
  uint32_t* sink = static_cast<uint32_t*>(dst);
  const uint4* cs = static_cast<const uint4*>(src);
  uint4* cd = static_cast<uint4*>(dst);
  const int64_t rows = bytes / kRowBytes, n16 = bytes / 16;
  const dim3 grid(workgroups), block(kProbeThreads);
  switch (mode * 32 + in_flight) {
    case 1: hipLaunchKernelGGL(stream_read_kernel<1>, grid, block, 0, s, rs, rows, sink); break;
    case 2: hipLaunchKernelGGL(stream_read_kernel<2>, grid, block, 0, s, rs, rows, sink); break;
    case 4: hipLaunchKernelGGL(stream_read_kernel<4>, grid, block, 0, s, rs, rows, sink); break;
    case 8: hipLaunchKernelGGL(stream_read_kernel<8>, grid, block, 0, s, rs, rows, sink); break;
    case 16: hipLaunchKernelGGL(stream_read_kernel<16>, grid, block, 0, s, rs, rows, sink); break;
    case 33: hipLaunchKernelGGL(copy_kernel<1>, grid, block, 0, s, cs, cd, n16); break;
    case 34: hipLaunchKernelGGL(copy_kernel<2>, grid, block, 0, s, cs, cd, n16); break;
    case 36: hipLaunchKernelGGL(copy_kernel<4>, grid, block, 0, s, cs, cd, n16); break;
    case 40: hipLaunchKernelGGL(copy_kernel<8>, grid, block, 0, s, cs, cd, n16); break;
    default: hipLaunchKernelGGL(copy_kernel<16>, grid, block, 0, s, cs, cd, n16); break;
  }
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}
