// Elementwise and row-reduction steps of a decode step around the attention
// path: residual add + RMSNorm, SwiGLU's silu(gate) * up, and the greedy
// (argmax) token pick over the vocabulary. One workgroup per token row, no
// global scratch, so every launch is safe to record in a HIP graph.
//
// Numerics follow the reference modules in bf16:
//   * residual: h = x + y, one bf16 rounding (sparse_draft_transformer.py:232-238);
//   * RMSNorm (transformer.py:505-516): fp32 x * (1 / sqrt(mean(x^2) + eps)),
//     rounded to bf16, times the bf16 weight, rounded again;
//   * FeedForward (transformer.py:490-502): silu(w1 x) rounded to bf16, times
//     w3 x, rounded again;
//   * greedy pick: the first index of the row maximum (torch.argmax).
#include <cmath>

#include "common.h"

namespace aspire {
namespace {

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf_round(float f) { return __uint_as_float(bf16_rne_bits(f) << 16); }

constexpr int kNormThreads = 256;
constexpr int kNormMaxChunks = 4;  // dim <= 256 threads * 4 chunks * 8 = 8192

// out[r] = rmsnorm(x[r] (+ delta[r])) * w; with delta, x[r] is updated to the sum.
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(uint16_t* x, const uint16_t* delta,
                                                                     const uint16_t* w, uint16_t* out, int dim,
                                                                     int64_t x_stride, int64_t d_stride,
                                                                     int64_t o_stride, float eps) {
  __shared__ float partial[kNormThreads / 64];
  const int r = blockIdx.x;
  uint4* xr = reinterpret_cast<uint4*>(x + int64_t(r) * x_stride);
  const uint4* dr = delta ? reinterpret_cast<const uint4*>(delta + int64_t(r) * d_stride) : nullptr;
  const int chunks = dim / 8;
  // the weight is requested with the row (not after the reduction's barrier)
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4 wv[kNormMaxChunks];
#pragma unroll
  for (int c = 0; c < kNormMaxChunks; ++c) {
    const int i = threadIdx.x + c * kNormThreads;
    if (i < chunks) wv[c] = wr[i];
  }
  float v[kNormMaxChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kNormMaxChunks; ++c) {
    const int i = threadIdx.x + c * kNormThreads;
    if (i < chunks) {
      uint4 a = xr[i];
      const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
      float s[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s[2 * e] = bf_lo(aw[e]);
        s[2 * e + 1] = bf_hi(aw[e]);
      }
      if (dr) {
        const uint4 b = dr[i];
        const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s[2 * e] = bf_round(s[2 * e] + bf_lo(bw[e]));
          s[2 * e + 1] = bf_round(s[2 * e + 1] + bf_hi(bw[e]));
        }
        xr[i] = make_uint4(pack_bf16x2_exact(s[0], s[1]), pack_bf16x2_exact(s[2], s[3]),
                           pack_bf16x2_exact(s[4], s[5]), pack_bf16x2_exact(s[6], s[7]));
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[c][e] = s[e];
        ss += s[e] * s[e];
      }
    }
  }
  ss = wave_sum_f(ss);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < kNormThreads / 64; ++k) tot += partial[k];
  const float rs = 1.f / sqrtf(tot / float(dim) + eps);
  uint4* orow = reinterpret_cast<uint4*>(out + int64_t(r) * o_stride);
#pragma unroll
  for (int c = 0; c < kNormMaxChunks; ++c) {
    const int i = threadIdx.x + c * kNormThreads;
    if (i < chunks) {
      const uint4 g = wv[c];
      const uint32_t gw[8] = {g.x, g.x, g.y, g.y, g.z, g.z, g.w, g.w};
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float wv = (e & 1) ? bf_hi(gw[e]) : bf_lo(gw[e]);
        o[e] = bf_round(bf_round(v[c][e] * rs) * wv);
      }
      orow[i] = make_uint4(pack_bf16x2_exact(o[0], o[1]), pack_bf16x2_exact(o[2], o[3]),
                           pack_bf16x2_exact(o[4], o[5]), pack_bf16x2_exact(o[6], o[7]));
    }
  }
}

// out[t, i] = bf16(bf16(silu(g[t, i])) * u[t, i]) with g = gu[t, :I], u = gu[t, I:].
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* gu, uint16_t* out, int inter,
                                                       int64_t gu_stride, int64_t o_stride, int64_t total8) {
  const int per_row = inter / 8;
  for (int64_t u8 = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; u8 < total8;
       u8 += int64_t(gridDim.x) * blockDim.x) {
    const int64_t t = u8 / per_row;
    const int c = int(u8 - t * per_row);
    const uint4 g = reinterpret_cast<const uint4*>(gu + t * gu_stride)[c];
    const uint4 u = reinterpret_cast<const uint4*>(gu + t * gu_stride + inter)[c];
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
    const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
    uint32_t ow[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float g0 = bf_lo(gw[e]), g1 = bf_hi(gw[e]);
      const float s0 = bf_round(g0 / (1.f + expf(-g0)));
      const float s1 = bf_round(g1 / (1.f + expf(-g1)));
      ow[e] = pack_bf16x2_rne(s0 * bf_lo(uw[e]), s1 * bf_hi(uw[e]));
    }
    reinterpret_cast<uint4*>(out + t * o_stride)[c] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  }
}

constexpr int kArgmaxThreads = 1024;

// Order used by the pick: the larger value, then the smaller index.
__device__ __forceinline__ void better(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const uint16_t* logits, int vocab,
                                                                     int64_t stride, int64_t* ids) {
  __shared__ float sv[kArgmaxThreads / 64];
  __shared__ int si[kArgmaxThreads / 64];
  const uint16_t* row = logits + int64_t(blockIdx.x) * stride;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  const int vec = vocab / 8;
  for (int c = threadIdx.x; c < vec; c += kArgmaxThreads) {
    const uint4 q = reinterpret_cast<const uint4*>(row)[c];
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      better(best, bi, bf_lo(qw[e]), 8 * c + 2 * e);
      better(best, bi, bf_hi(qw[e]), 8 * c + 2 * e + 1);
    }
  }
  for (int j = vec * 8 + threadIdx.x; j < vocab; j += kArgmaxThreads) better(best, bi, bf_lo(row[j]), j);
  // the row's first element seeds every lane, so a row of -inf still picks a valid index
  if (bi == 0x7fffffff) {
    best = bf_lo(row[0]);
    bi = 0;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float v2 = __shfl_xor(best, m);
    const int i2 = __shfl_xor(bi, m);
    better(best, bi, v2, i2);
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = best;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = sv[0];
    int i = si[0];
    for (int k = 1; k < kArgmaxThreads / 64; ++k) better(v, i, sv[k], si[k]);
    ids[blockIdx.x] = i;
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace aspire

extern "C" int aspire_add_rms_norm(void* x, int64_t x_stride, const void* delta, int64_t delta_stride,
                                   const void* weight, void* out, int64_t out_stride, int32_t rows, int32_t dim,
                                   float eps, void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(rows >= 0, "negative rows");
  if (rows == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(x && weight && out, "null pointer");
  ASPIRE_CHECK_ARG(dim > 0 && dim % 8 == 0 && dim <= kNormThreads * kNormMaxChunks * 8,
                   "dim must be a multiple of 8 and at most 8192");
  ASPIRE_CHECK_ARG(aligned16(x) && aligned16(weight) && aligned16(out) && (delta == nullptr || aligned16(delta)),
                   "rows must be 16-byte aligned");
  ASPIRE_CHECK_ARG(x_stride % 8 == 0 && out_stride % 8 == 0 && (delta == nullptr || delta_stride % 8 == 0),
                   "row strides must be multiples of 8 elements");
  ASPIRE_CHECK_ARG(x_stride >= dim && out_stride >= dim && (delta == nullptr || delta_stride >= dim),
                   "row strides smaller than dim");
  hipLaunchKernelGGL(add_rms_norm_kernel, dim3(rows), dim3(kNormThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<uint16_t*>(x), static_cast<const uint16_t*>(delta),
                     static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out), dim, x_stride,
                     delta_stride, out_stride, eps);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}

extern "C" int aspire_silu_mul(const void* gate_up, int64_t gate_up_stride, void* out, int64_t out_stride,
                               int32_t rows, int32_t inter, void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(rows >= 0 && inter >= 0, "negative sizes");
  if (rows == 0 || inter == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(gate_up && out, "null pointer");
  ASPIRE_CHECK_ARG(inter % 8 == 0 && gate_up_stride % 8 == 0 && out_stride % 8 == 0,
                   "intermediate size and strides must be multiples of 8 elements");
  ASPIRE_CHECK_ARG(gate_up_stride >= 2 * int64_t(inter) && out_stride >= inter, "row strides too small");
  ASPIRE_CHECK_ARG(aligned16(gate_up) && aligned16(out), "rows must be 16-byte aligned");
  const int64_t total8 = int64_t(rows) * (inter / 8);
  const int64_t blocks = std::min<int64_t>((total8 + 255) / 256, 4096);
  hipLaunchKernelGGL(silu_mul_kernel, dim3(unsigned(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(out), inter, gate_up_stride,
                     out_stride, total8);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}

extern "C" int aspire_argmax_rows(const void* logits, int64_t stride, int32_t rows, int32_t vocab, int64_t* ids,
                                  void* stream) {
  using namespace aspire;
  ASPIRE_CHECK_ARG(rows >= 0, "negative rows");
  if (rows == 0) return ASPIRE_OK;
  ASPIRE_CHECK_ARG(logits && ids, "null pointer");
  ASPIRE_CHECK_ARG(vocab > 0 && stride >= vocab, "bad vocab / stride");
  ASPIRE_CHECK_ARG(aligned16(logits) && stride % 8 == 0, "rows must be 16-byte aligned");
  hipLaunchKernelGGL(argmax_rows_kernel, dim3(rows), dim3(kArgmaxThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(logits), vocab, stride, ids);
  ASPIRE_CHECK_LAUNCH();
  return ASPIRE_OK;
}
