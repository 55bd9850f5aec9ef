// The v2 candidate-scale grid search and the per-channel activation
// importance it weights by, for gfx950.
//
// Search (mround/core/scale_search.py:71-187; oracle
// mround/reference/scale_search.py:130-211): one thread per quantization
// group, the group (and its channels' importance) held in registers, every
// candidate evaluated against it with the loss summed element by element in
// column order. The work is VALU-bound (about 7 operations per weight per
// candidate, 181-201 candidates) and reads each weight once.
//
// Importance (the collecting forward of mround/pipeline/runner.py:346-363,
// `sum(square(x), axis=0)` of each linear's input): per-column sums of
// squares in two deterministic passes, row blocks into a workspace, then the
// blocks summed in order and added to the running total.
#include <cmath>

#include "mr_common.h"

namespace mr {
namespace {

constexpr int kBlock = 256;
constexpr int kRowBlocks = 64;

template <typename WT>
__device__ __forceinline__ float ld_as_f32(const WT* p, int64_t i) {
  if constexpr (sizeof(WT) == 4) return reinterpret_cast<const float*>(p)[i];
  else return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

template <int GS, typename WT, bool IMP>
__global__ __launch_bounds__(kBlock) void search_kernel(const WT* __restrict__ w,
                                                        const float* __restrict__ imp,
                                                        int64_t n_groups, int groups_per_row,
                                                        int bits, double step, int half,
                                                        float* __restrict__ scale_out) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (g >= n_groups) return;
  float x[GS];
  float q[GS];
#pragma unroll
  for (int j = 0; j < GS; ++j) x[j] = ld_as_f32(w, g * GS + j);
  if constexpr (IMP) {
    const int64_t col0 = static_cast<int64_t>(g % groups_per_row) * GS;
#pragma unroll
    for (int j = 0; j < GS; ++j) q[j] = imp[col0 + j];
  }
  // anchor: the signed element of largest magnitude, first occurrence
  float gmax = x[0], amax = fabsf(x[0]);
#pragma unroll
  for (int j = 1; j < GS; ++j)
    if (fabsf(x[j]) > amax) {
      amax = fabsf(x[j]);
      gmax = x[j];
    }
  const float recip = gmax == 0.0f ? 0.0f : 1.0f / gmax;
  const double nmax_d = static_cast<double>(1 << (bits - 1));
  const float nmax = static_cast<float>(nmax_d);
  const float lo = -nmax, hi = nmax - 1.0f;

  auto evaluate = [&](float eff, float& scale) -> float {
    const float inverse = (-eff) * recip;
    scale = inverse == 0.0f ? 0.0f : 1.0f / inverse;
    float loss = 0.0f;
#pragma unroll
    for (int j = 0; j < GS; ++j) {
      const float c = fminf(fmaxf(rintf(inverse * x[j]), lo), hi);
      const float r = scale * c - x[j];
      float t = r * r;
      if constexpr (IMP) t = t * q[j];
      loss = loss + t;
    }
    return loss;
  };
  float best_s;
  float best_l = evaluate(nmax, best_s);
  for (int i = -half; i <= half; ++i) {
    if (i == 0) continue;
    const float eff = static_cast<float>(nmax_d - step * static_cast<double>(i));
    float s;
    const float l = evaluate(eff, s);
    if (l < best_l) {
      best_l = l;
      best_s = s;
    }
  }
  scale_out[g] = best_s;
}

template <typename XT>
__global__ __launch_bounds__(kBlock) void colsumsq_partial(const XT* __restrict__ x, int64_t rows,
                                                           int64_t cols, int64_t ld,
                                                           float* __restrict__ partial) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (c >= cols) return;
  const int64_t per = (rows + kRowBlocks - 1) / kRowBlocks;
  const int64_t r0 = blockIdx.y * per;
  const int64_t r1 = min(rows, r0 + per);
  float acc = 0.0f;
  for (int64_t r = r0; r < r1; ++r) {
    const float v = ld_as_f32(x, r * ld + c);
    acc = acc + v * v;
  }
  partial[blockIdx.y * cols + c] = acc;
}

__global__ __launch_bounds__(kBlock) void colsumsq_final(const float* __restrict__ partial,
                                                         int64_t cols, float* __restrict__ out) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (c >= cols) return;
  float acc = 0.0f;
  for (int b = 0; b < kRowBlocks; ++b) acc = acc + partial[b * cols + c];
  out[c] = out[c] + acc;
}

template <int GS, typename WT>
int launch_search(const void* w, const float* imp, int64_t n_groups, int gpr, int bits, double step,
                  int half, float* out, hipStream_t s) {
  const unsigned blocks = static_cast<unsigned>((n_groups + kBlock - 1) / kBlock);
  if (imp)
    hipLaunchKernelGGL((search_kernel<GS, WT, true>), dim3(blocks), dim3(kBlock), 0, s,
                       static_cast<const WT*>(w), imp, n_groups, gpr, bits, step, half, out);
  else
    hipLaunchKernelGGL((search_kernel<GS, WT, false>), dim3(blocks), dim3(kBlock), 0, s,
                       static_cast<const WT*>(w), imp, n_groups, gpr, bits, step, half, out);
  MR_LAUNCH_CHECK("mr_search_scales");
  return MR_OK;
}

}  // namespace
}  // namespace mr

extern "C" {

int mr_search_scales(const void* w, int w_dtype, const float* importance, int64_t rows,
                     int64_t cols, int group_size, int bits, double step, int half_count,
                     float* scale_out, void* stream) {
  using namespace mr;
  clear_error();
  if (rows <= 0 || cols <= 0) return MR_OK;
  if (!w || !scale_out) return fail(MR_EINVAL, "mr_search_scales: null pointer");
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(MR_EINVAL, "mr_search_scales: group size must be 32, 64 or 128, got %d", group_size);
  if (cols % group_size)
    return fail(MR_EINVAL, "search expects a 2-D weight whose last dimension is a multiple of "
                "group_size=%d, got %lld columns", group_size, (long long)cols);
  if (bits < 2 || bits > 8) return fail(MR_EINVAL, "mr_search_scales: bits must be 2..8");
  if (half_count < 0 || half_count > 100000 || !(step >= 0.0))
    return fail(MR_EINVAL, "mr_search_scales: bad grid");
  if (w_dtype != MR_F32 && w_dtype != MR_BF16)
    return fail(MR_EINVAL, "mr_search_scales: weight must be fp32 or bf16");
  const int64_t n_groups = rows * (cols / group_size);
  const int gpr = static_cast<int>(cols / group_size);
  if ((n_groups + kBlock - 1) / kBlock > 0x7fffffff) return fail(MR_EINVAL, "mr_search_scales: too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool f32 = w_dtype == MR_F32;
#define MR_SEARCH_CASE(GS)                                                                            \
  return f32 ? launch_search<GS, float>(w, importance, n_groups, gpr, bits, step, half_count, scale_out, s) \
             : launch_search<GS, uint16_t>(w, importance, n_groups, gpr, bits, step, half_count, scale_out, s);
  switch (group_size) {
    case 32: { MR_SEARCH_CASE(32) }
    case 64: { MR_SEARCH_CASE(64) }
    default: { MR_SEARCH_CASE(128) }
  }
#undef MR_SEARCH_CASE
}

int64_t mr_colsumsq_workspace_bytes(int64_t cols) {
  return cols > 0 ? static_cast<int64_t>(mr::kRowBlocks) * cols * 4 : 0;
}

int mr_colsumsq(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ld, float* out,
                void* workspace, void* stream) {
  using namespace mr;
  clear_error();
  if (rows <= 0 || cols <= 0) return MR_OK;
  if (!x || !out || !workspace) return fail(MR_EINVAL, "mr_colsumsq: null pointer");
  if (ld < cols) return fail(MR_EINVAL, "mr_colsumsq: ld smaller than the row");
  if (x_dtype != MR_F32 && x_dtype != MR_BF16) return fail(MR_EINVAL, "mr_colsumsq: fp32 or bf16 input");
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* partial = static_cast<float*>(workspace);
  const unsigned cb = static_cast<unsigned>((cols + kBlock - 1) / kBlock);
  if (x_dtype == MR_F32)
    hipLaunchKernelGGL(colsumsq_partial<float>, dim3(cb, kRowBlocks), dim3(kBlock), 0, s,
                       static_cast<const float*>(x), rows, cols, ld, partial);
  else
    hipLaunchKernelGGL(colsumsq_partial<uint16_t>, dim3(cb, kRowBlocks), dim3(kBlock), 0, s,
                       static_cast<const uint16_t*>(x), rows, cols, ld, partial);
  hipLaunchKernelGGL(colsumsq_final, dim3(cb), dim3(kBlock), 0, s, partial, cols, out);
  MR_LAUNCH_CHECK("mr_colsumsq");
  return MR_OK;
}

}  // extern "C"
