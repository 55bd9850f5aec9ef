// Elementwise and row-reduction kernels of the decoder block, for gfx950.
//
// The block is the mlx-lm Qwen2 / Llama decoder layer the reference tunes
// against (mround/pipeline/blocks.py:578-606):
//   x1 = rmsnorm(h) w1; q, k, v = x1 Wq^T + bq, ...; rope(q, k); o = attn;
//   h2 = h + o Wo^T; x2 = rmsnorm(h2) w2; out = h2 + (silu(x2 Wg^T) * x2 Wu^T) Wd^T
// The fp32 residual stream stays fp32; GEMM operands are bf16.
#include <cmath>

#include "mr_common.h"

namespace mr {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float block_sum_f32(float x, float* smem) {
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) smem[wave] = x;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < kBlock / 64; ++i) t += smem[i];
  __syncthreads();
  return t;  // every thread
}

// y = h * rsqrt(mean(h^2) + eps) * w, written as bf16; rstd saved for the backward.
__global__ __launch_bounds__(kBlock) void rmsnorm_fwd(const float* __restrict__ h,
                                                      const float* __restrict__ w, int64_t H,
                                                      float eps, uint16_t* __restrict__ y,
                                                      float* __restrict__ rstd) {
  __shared__ float smem[kBlock / 64];
  const int64_t row = blockIdx.x;
  const float* hr = h + row * H;
  float ss = 0.0f;
  for (int64_t i = threadIdx.x; i < H; i += kBlock) {
    const float x = hr[i];
    ss += x * x;
  }
  ss = block_sum_f32(ss, smem);
  const float r = rsqrtf(ss / static_cast<float>(H) + eps);
  if (threadIdx.x == 0 && rstd) rstd[row] = r;
  uint16_t* yr = y + row * H;
  for (int64_t i = threadIdx.x; i < H; i += kBlock) yr[i] = f32_to_bf16(hr[i] * r * w[i]);
}

// dh = dres + r w dy - (r^3 h / H) sum_j(dy_j w_j h_j), written as bf16 (and
// optionally fp32). The derivative of y = h r w with r = (mean(h^2) + eps)^-1/2.
__global__ __launch_bounds__(kBlock) void rmsnorm_bwd(const float* __restrict__ dy,
                                                      const float* __restrict__ h,
                                                      const float* __restrict__ w,
                                                      const float* __restrict__ rstd,
                                                      const float* __restrict__ dres, int64_t H,
                                                      uint16_t* __restrict__ dh_bf16,
                                                      float* __restrict__ dh_f32) {
  __shared__ float smem[kBlock / 64];
  const int64_t row = blockIdx.x;
  const float* dyr = dy + row * H;
  const float* hr = h + row * H;
  float dot = 0.0f;
  for (int64_t i = threadIdx.x; i < H; i += kBlock) dot += dyr[i] * w[i] * hr[i];
  dot = block_sum_f32(dot, smem);
  const float r = rstd[row];
  const float c = r * r * r * dot / static_cast<float>(H);
  for (int64_t i = threadIdx.x; i < H; i += kBlock) {
    float g = r * w[i] * dyr[i] - c * hr[i];
    if (dres) g += dres[row * H + i];
    if (dh_bf16) dh_bf16[row * H + i] = f32_to_bf16(g);
    if (dh_f32) dh_f32[row * H + i] = g;
  }
}

// Rotary embedding over the first n_heads heads of each token row (q heads
// then k heads of the packed qkv row), non-interleaved halves: for i < d/2,
//   fwd: (x_i, x_{i+d/2}) -> (x_i c - x_{i+d/2} s, x_{i+d/2} c + x_i s)
//   bwd: the transpose rotation, (g_i c + g_{i+d/2} s, g_{i+d/2} c - g_i s).
// cs holds cos and sin for every (position, i), fp32 [S, d/2, 2].
template <bool BWD>
__global__ __launch_bounds__(kBlock) void rope_kernel(uint16_t* __restrict__ x, int64_t ld,
                                                      int64_t T, int S, int n_heads, int d,
                                                      const float* __restrict__ cs) {
  const int half = d / 2;
  const int64_t total = T * n_heads * half;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (idx >= total) return;
  const int i = static_cast<int>(idx % half);
  const int64_t th = idx / half;
  const int hd = static_cast<int>(th % n_heads);
  const int64_t t = th / n_heads;
  const int pos = static_cast<int>(t % S);
  uint16_t* p = x + t * ld + static_cast<int64_t>(hd) * d;
  const float a = bf16_to_f32(p[i]);
  const float b = bf16_to_f32(p[i + half]);
  const float c = cs[(static_cast<int64_t>(pos) * half + i) * 2];
  const float s = cs[(static_cast<int64_t>(pos) * half + i) * 2 + 1];
  float ya, yb;
  if constexpr (BWD) {
    ya = a * c + b * s;
    yb = b * c - a * s;
  } else {
    ya = a * c - b * s;
    yb = b * c + a * s;
  }
  p[i] = f32_to_bf16(ya);
  p[i + half] = f32_to_bf16(yb);
}

__global__ __launch_bounds__(kBlock) void cast_kernel(const float* __restrict__ x,
                                                      uint16_t* __restrict__ y, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
    y[i] = f32_to_bf16(x[i]);
}

}  // namespace
}  // namespace mr

extern "C" {

int mr_cast_f32_bf16(const float* x, void* y, int64_t n, void* stream) {
  using namespace mr;
  clear_error();
  if (n <= 0) return MR_OK;
  if (!x || !y) return fail(MR_EINVAL, "mr_cast_f32_bf16: null pointer");
  int64_t blocks = (n + kBlock - 1) / kBlock;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(cast_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), x, static_cast<uint16_t*>(y), n);
  MR_LAUNCH_CHECK("mr_cast_f32_bf16");
  return MR_OK;
}

int mr_rmsnorm_fwd(const float* h, const float* w, int64_t T, int64_t H, float eps, void* y_bf16,
                   float* rstd_out, void* stream) {
  using namespace mr;
  clear_error();
  if (T <= 0 || H <= 0) return MR_OK;
  if (!h || !w || !y_bf16) return fail(MR_EINVAL, "mr_rmsnorm_fwd: null pointer");
  if (T > 0x7fffffff) return fail(MR_EINVAL, "mr_rmsnorm_fwd: too many rows");
  hipLaunchKernelGGL(rmsnorm_fwd, dim3(static_cast<unsigned>(T)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), h, w, H, eps,
                     static_cast<uint16_t*>(y_bf16), rstd_out);
  MR_LAUNCH_CHECK("mr_rmsnorm_fwd");
  return MR_OK;
}

int mr_rmsnorm_bwd(const float* dy, const float* h, const float* w, const float* rstd,
                   const float* dres, int64_t T, int64_t H, void* dh_bf16, float* dh_f32,
                   void* stream) {
  using namespace mr;
  clear_error();
  if (T <= 0 || H <= 0) return MR_OK;
  if (!dy || !h || !w || !rstd || (!dh_bf16 && !dh_f32))
    return fail(MR_EINVAL, "mr_rmsnorm_bwd: null pointer");
  if (T > 0x7fffffff) return fail(MR_EINVAL, "mr_rmsnorm_bwd: too many rows");
  hipLaunchKernelGGL(rmsnorm_bwd, dim3(static_cast<unsigned>(T)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), dy, h, w, rstd, dres, H,
                     static_cast<uint16_t*>(dh_bf16), dh_f32);
  MR_LAUNCH_CHECK("mr_rmsnorm_bwd");
  return MR_OK;
}

int mr_rope(void* x_bf16, int64_t ld, int64_t T, int S, int n_heads, int head_dim,
            const float* cos_sin, int backward, void* stream) {
  using namespace mr;
  clear_error();
  if (T <= 0 || n_heads <= 0) return MR_OK;
  if (!x_bf16 || !cos_sin) return fail(MR_EINVAL, "mr_rope: null pointer");
  if (head_dim <= 0 || head_dim % 2 || S <= 0 || ld < static_cast<int64_t>(n_heads) * head_dim)
    return fail(MR_EINVAL, "mr_rope: bad shape");
  const int64_t total = T * n_heads * (head_dim / 2);
  const int64_t blocks = (total + kBlock - 1) / kBlock;
  if (blocks > 0x7fffffff) return fail(MR_EINVAL, "mr_rope: too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint16_t* x = static_cast<uint16_t*>(x_bf16);
  if (backward)
    hipLaunchKernelGGL(rope_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, x,
                       ld, T, S, n_heads, head_dim, cos_sin);
  else
    hipLaunchKernelGGL(rope_kernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s,
                       x, ld, T, S, n_heads, head_dim, cos_sin);
  MR_LAUNCH_CHECK("mr_rope");
  return MR_OK;
}

}  // extern "C"
