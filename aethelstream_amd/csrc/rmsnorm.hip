// rmsnorm.hip - RMSNorm forward producing the fused GEMMs' bf16 operand.
//
// rms_norm_fwd (doublepass/src/math.rs:28-59), per token row b of x [m, d]:
//   mean_sq = (sum_i x[b,i]^2) / d      (each square rounded, then summed)
//   rms[b]  = sqrt(mean_sq + eps)
//   y[b,i]  = (x[b,i] / rms[b]) * w[i]
// in fp32, with correctly rounded division and square root.  y leaves as
// bf16 (RNE): the activation the fused NF4 GEMMs read right after it
// (forward.rs:173-176 for q/k/v, :249-252 for gate/up).  rms leaves as fp32
// for the backward pass.  The reference sums the squares in index order; here
// each thread sums its 4-element chunks in index order and the partial sums
// meet in a tree, so rms can differ from the sequential sum in its last bits.
//
// The kernel is HBM-bound (4 bytes read and 2 written per element), one
// workgroup per row.  The model widths (4096, 8192, 16384) keep the row in
// registers between the reduction and the output; other widths read it twice.
#include "abi_common.hpp"
#include "gemm_common.hpp"
#include "nf4_device.hpp"

namespace nf4s {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// The row's squares summed per thread in index order, then over the wave and
// the workgroup.
__device__ __forceinline__ float block_sum(float s, float *part) {
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += part[i];
  return tot;
}

__device__ __forceinline__ u32x2 norm_chunk(const floatx4 &v, const floatx4 &g, float r) {
  float o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float xh = fp32_rounded(v[i] / r);
    o[i] = fp32_rounded(xh * g[i]);
  }
  return (u32x2){pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
}

// d = 1024 * kChunks: the row stays in registers between the two passes
// (thread t holds 4-element chunks t, t + 256, ...), so x is read once.
template <int kChunks>
__global__ void __launch_bounds__(kNormThreads) rmsnorm_fwd_reg_kernel(const float *__restrict__ x,
                                                                      const float *__restrict__ w,
                                                                      float eps,
                                                                      uint16_t *__restrict__ y,
                                                                      float *__restrict__ rms) {
  __shared__ float part[kNormThreads / 64];
  constexpr int64_t d = 1024 * kChunks;
  const int64_t row = blockIdx.x;
  const floatx4 *xr = reinterpret_cast<const floatx4 *>(x + row * d) + threadIdx.x;
  floatx4 v[kChunks];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) v[c] = __builtin_nontemporal_load(xr + c * kNormThreads);
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kChunks; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sq = v[c][i] * v[c][i];
      s += sq;
    }
  const float tot = block_sum(s, part);
  const float r = __builtin_sqrtf(tot / (float)d + eps);
  if (threadIdx.x == 0) rms[row] = r;
  const floatx4 *wr = reinterpret_cast<const floatx4 *>(w) + threadIdx.x;
  u32x2 *yr = reinterpret_cast<u32x2 *>(y + row * d) + threadIdx.x;
#pragma unroll
  for (int c = 0; c < kChunks; ++c)
    __builtin_nontemporal_store(norm_chunk(v[c], wr[c * kNormThreads], r), yr + c * kNormThreads);
}

// Any d % 4 == 0: pass 1 sums the squares, pass 2 reads the row again (an L2
// hit: a resident workgroup's row is at most 128 KB) and writes y.
__global__ void __launch_bounds__(kNormThreads) rmsnorm_fwd_kernel(const float *__restrict__ x,
                                                                  const float *__restrict__ w,
                                                                  int64_t d, float eps,
                                                                  uint16_t *__restrict__ y,
                                                                  float *__restrict__ rms) {
  __shared__ float part[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  const floatx4 *xr = reinterpret_cast<const floatx4 *>(x + row * d);
  const floatx4 *wr = reinterpret_cast<const floatx4 *>(w);
  const int64_t chunks = d >> 2;
  float s = 0.0f;
  for (int64_t c = threadIdx.x; c < chunks; c += kNormThreads) {
    const floatx4 v = xr[c];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sq = v[i] * v[i];
      s += sq;
    }
  }
  const float tot = block_sum(s, part);
  const float r = __builtin_sqrtf(tot / (float)d + eps);
  if (threadIdx.x == 0) rms[row] = r;
  u32x2 *yr = reinterpret_cast<u32x2 *>(y + row * d);
  for (int64_t c = threadIdx.x; c < chunks; c += kNormThreads)
    __builtin_nontemporal_store(norm_chunk(xr[c], wr[c], r), yr + c);
}

}  // namespace nf4s

using namespace nf4s;

extern "C" {

int32_t nf4s_rmsnorm_fwd(const float *x, const float *w, int64_t m, int64_t d, float eps,
                         uint16_t *y, float *rms, void *stream) {
  clear_error();
  if (m < 0 || d <= 0)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "bad RMSNorm shape m=%lld d=%lld", (long long)m,
                (long long)d);
  if (m == 0) return NF4S_OK;
  if (x == nullptr || w == nullptr || y == nullptr || rms == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "NULL buffer");
  if (d % 4 != 0)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "RMSNorm needs d %% 4 == 0, got %lld", (long long)d);
  if (d > ((int64_t)1 << 15))
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "RMSNorm row of %lld elements is too long",
                (long long)d);
  if (m > 0x7fffffff) return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "too many rows");
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(y, 8) || !aligned(rms, 4))
    return fail(NF4S_ERR_MISALIGNED, "x and w must be 16-byte aligned, y 8-byte aligned");
  hipStream_t s = as_stream(stream);
  const dim3 grid((uint32_t)m), block(kNormThreads);
  switch (d) {
    case 4096: hipLaunchKernelGGL(rmsnorm_fwd_reg_kernel<4>, grid, block, 0, s, x, w, eps, y, rms); break;
    case 8192: hipLaunchKernelGGL(rmsnorm_fwd_reg_kernel<8>, grid, block, 0, s, x, w, eps, y, rms); break;
    case 16384: hipLaunchKernelGGL(rmsnorm_fwd_reg_kernel<16>, grid, block, 0, s, x, w, eps, y, rms); break;
    default: hipLaunchKernelGGL(rmsnorm_fwd_kernel, grid, block, 0, s, x, w, d, eps, y, rms); break;
  }
  return check_launch("rmsnorm_fwd_kernel");
}

}  // extern "C"
