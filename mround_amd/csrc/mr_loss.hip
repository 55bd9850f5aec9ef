// Block reconstruction losses with their gradient, for gfx950.
//
// mround/core/losses.py:42-130: r = pred - target in fp32; the plain loss keeps
// every element, the outlier loss keeps |r| < t where t is the k-th largest
// |r| of the whole batch (sort(|r|)[n - k]); every element tied at t is
// excluded. loss = sum(r_kept^2) / denom and dL/dpred = 2 r_kept / denom.
//
// The threshold is found exactly by a three-pass radix select on the bit
// pattern of |r| (non-negative floats order like their bit patterns): 11, 11
// and 10 bits from the top, each pass a histogram of the next digit among
// the elements that share the digits chosen so far, followed by a one-block
// select. Everything stays on the device; no host synchronisation.
//
// Sums are deterministic: a fixed grid of kBlocks blocks, fp64 accumulation
// per thread, a fixed-order block reduction, then one block adding the block
// partials in order.
#include "mr_common.h"

namespace mr {
namespace {

constexpr int kBlock = 256;
constexpr int kBlocks = 1024;
constexpr int kBins = 2048;

struct Workspace {
  double partial[kBlocks];
  uint32_t hist[kBins];
  uint32_t state[4];  // [0] key prefix, [1] remaining rank k, [2] final key
};

__device__ __forceinline__ double block_sum(double x, double* smem) {
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  const int wave = threadIdx.x / 64;
  if ((threadIdx.x % 64) == 0) smem[wave] = x;
  __syncthreads();
  double total = 0.0;
  if (threadIdx.x == 0) {
    for (int i = 0; i < kBlock / 64; ++i) total += smem[i];
  }
  return total;  // valid in thread 0
}

__global__ __launch_bounds__(kBlock) void zero_hist(Workspace* ws) {
  for (int i = threadIdx.x; i < kBins; i += kBlock) ws->hist[i] = 0;
}

__global__ void set_rank(Workspace* ws, uint32_t k) {
  ws->state[0] = 0;
  ws->state[1] = k;
}

// Histogram of digit (key >> shift) & (nbins-1) among keys whose bits above
// `shift + digit_bits` equal the prefix chosen so far.
__global__ __launch_bounds__(kBlock) void radix_hist(const float* __restrict__ pred,
                                                     const float* __restrict__ target, int64_t n,
                                                     int shift, int nbits, int prefix_shift,
                                                     Workspace* __restrict__ ws) {
  __shared__ uint32_t h[kBins];
  for (int i = threadIdx.x; i < kBins; i += kBlock) h[i] = 0;
  __syncthreads();
  const uint32_t prefix = ws->state[0];
  const uint32_t dmask = (1u << nbits) - 1u;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    const float r = pred[i] - target[i];
    const uint32_t key = __float_as_uint(r) & 0x7fffffffu;
    const bool match = prefix_shift >= 32 || (key >> prefix_shift) == prefix;
    if (match) atomicAdd(&h[(key >> shift) & dmask], 1u);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kBins; i += kBlock) {
    if (h[i]) atomicAdd(&ws->hist[i], h[i]);
  }
}

// Finds the digit holding the k-th largest key: the largest d with
// count(digit > d) < k <= count(digit >= d). Appends d to the prefix and
// subtracts the count above from k. One block; each thread owns 8 bins.
__global__ __launch_bounds__(kBlock) void radix_select(int nbits, int last, Workspace* ws,
                                                       float* __restrict__ threshold_out) {
  __shared__ uint32_t totals[kBlock];
  __shared__ uint32_t above[kBlock];
  const int nb = 1 << nbits;
  const int per = (nb + kBlock - 1) / kBlock;
  const int t = threadIdx.x;
  uint32_t mine = 0;
  for (int j = 0; j < per; ++j) {
    int b = t * per + j;
    if (b < nb) mine += ws->hist[b];
  }
  totals[t] = mine;
  __syncthreads();
  if (t == 0) {
    uint32_t run = 0;
    for (int i = kBlock - 1; i >= 0; --i) {
      above[i] = run;  // count in bins owned by threads > i
      run += totals[i];
    }
  }
  __syncthreads();
  const uint32_t k = ws->state[1];
  uint32_t run = above[t];
  if (run < k && k <= run + totals[t]) {
    for (int j = per - 1; j >= 0; --j) {
      int b = t * per + j;
      if (b >= nb) continue;
      uint32_t c = ws->hist[b];
      if (run < k && k <= run + c) {
        const uint32_t prefix = (ws->state[0] << nbits) | static_cast<uint32_t>(b);
        ws->state[0] = prefix;
        ws->state[1] = k - run;
        if (last) {
          ws->state[2] = prefix;
          if (threshold_out) *threshold_out = __uint_as_float(prefix);
        }
        break;
      }
      run += c;
    }
  }
}

// Loss and gradient. keep = |r| < threshold when a threshold is given.
__global__ __launch_bounds__(kBlock) void loss_pass(const float* __restrict__ pred,
                                                    const float* __restrict__ target, int64_t n,
                                                    float grad_scale, const float* __restrict__ thr_in,
                                                    const Workspace* __restrict__ thr_ws, int use_thr,
                                                    float* __restrict__ grad, Workspace* __restrict__ ws) {
  __shared__ double smem[kBlock / 64];
  float thr = 0.0f;
  if (use_thr) thr = thr_in ? *thr_in : __uint_as_float(thr_ws->state[2]);
  double acc = 0.0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  const bool vec = (n % 4) == 0;
  if (vec) {
    const int64_t n4 = n / 4;
    const float4* p4 = reinterpret_cast<const float4*>(pred);
    const float4* t4 = reinterpret_cast<const float4*>(target);
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n4; i += stride) {
      float4 p = p4[i], q = t4[i];
      float r[4] = {p.x - q.x, p.y - q.y, p.z - q.z, p.w - q.w};
      float gout[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float kept = r[k];
        if (use_thr) kept = (fabsf(r[k]) < thr) ? r[k] : 0.0f;
        float sq = kept * kept;
        acc += static_cast<double>(sq);
        gout[k] = kept * grad_scale;
      }
      if (grad) reinterpret_cast<float4*>(grad)[i] = make_float4(gout[0], gout[1], gout[2], gout[3]);
    }
  } else {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
      float r = pred[i] - target[i];
      float kept = r;
      if (use_thr) kept = (fabsf(r) < thr) ? r : 0.0f;
      acc += static_cast<double>(kept * kept);
      if (grad) grad[i] = kept * grad_scale;
    }
  }
  double total = block_sum(acc, smem);
  if (threadIdx.x == 0) ws->partial[blockIdx.x] = total;
}

__global__ __launch_bounds__(kBlock) void finalize(const Workspace* __restrict__ ws, int nparts,
                                                   double denom, float* __restrict__ loss_out) {
  __shared__ double smem[kBlock / 64];
  double acc = 0.0;
  // Fixed assignment of partials to threads and a fixed tree: deterministic.
  for (int i = threadIdx.x; i < nparts; i += kBlock) acc += ws->partial[i];
  double total = block_sum(acc, smem);
  if (threadIdx.x == 0) *loss_out = static_cast<float>(total / denom);
}

int grid_for(int64_t n) {
  int64_t want = (n / 4 + kBlock - 1) / kBlock;
  if (want < 1) want = 1;
  return static_cast<int>(want < kBlocks ? want : kBlocks);
}

int check_loss(const char* fn, const float* pred, const float* target, int64_t n, int64_t denom,
               float* loss_out, void* workspace) {
  if (!pred || !target || !loss_out || !workspace) return fail(MR_EINVAL, "%s: null pointer", fn);
  if (n <= 0) return fail(MR_EINVAL, "%s: empty input", fn);
  if (denom <= 0) return fail(MR_EINVAL, "%s: denominator must be positive", fn);
  if ((n % 4) == 0 && (!aligned16(pred) || !aligned16(target)))
    return fail(MR_EINVAL, "%s: inputs must be 16-byte aligned", fn);
  return MR_OK;
}

}  // namespace
}  // namespace mr

extern "C" {

size_t mr_loss_workspace_bytes(int64_t n) {
  (void)n;
  return sizeof(mr::Workspace);
}

int mr_loss_mse(const float* pred, const float* target, int64_t n, int64_t denom,
                float* loss_out, float* grad_out, void* workspace, void* stream) {
  using namespace mr;
  clear_error();
  int rc = check_loss("mr_loss_mse", pred, target, n, denom, loss_out, workspace);
  if (rc) return rc;
  if (grad_out && (n % 4) == 0 && !aligned16(grad_out))
    return fail(MR_EINVAL, "mr_loss_mse: gradient must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  Workspace* ws = static_cast<Workspace*>(workspace);
  const int grid = grid_for(n);
  const float gscale = static_cast<float>(2.0 / static_cast<double>(denom));
  hipLaunchKernelGGL(loss_pass, dim3(grid), dim3(kBlock), 0, s, pred, target, n, gscale, nullptr,
                     nullptr, 0, grad_out, ws);
  hipLaunchKernelGGL(finalize, dim3(1), dim3(kBlock), 0, s, ws, grid, static_cast<double>(denom),
                     loss_out);
  MR_LAUNCH_CHECK("mr_loss_mse");
  return MR_OK;
}

int mr_loss_outlier(const float* pred, const float* target, int64_t n, int64_t k, int64_t denom,
                    const float* threshold_in, float* threshold_out, float* loss_out,
                    float* grad_out, void* workspace, void* stream) {
  using namespace mr;
  clear_error();
  int rc = check_loss("mr_loss_outlier", pred, target, n, denom, loss_out, workspace);
  if (rc) return rc;
  if (!threshold_in && (k < 1 || k > n))
    return fail(MR_EINVAL, "mr_loss_outlier: rank k=%lld outside [1, n]", static_cast<long long>(k));
  if (n > 0xffffffffLL) return fail(MR_EINVAL, "mr_loss_outlier: more than 2^32 elements");
  if (grad_out && (n % 4) == 0 && !aligned16(grad_out))
    return fail(MR_EINVAL, "mr_loss_outlier: gradient must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  Workspace* ws = static_cast<Workspace*>(workspace);
  const int grid = grid_for(n);
  const int hist_grid = grid;
  if (!threshold_in) {
    hipLaunchKernelGGL(set_rank, dim3(1), dim3(1), 0, s, ws, static_cast<uint32_t>(k));
    // digits: bits [21, 32) then [10, 21) then [0, 10)
    const int shifts[3] = {21, 10, 0};
    const int widths[3] = {11, 11, 10};
    const int pshift[3] = {32, 21, 10};
    for (int pass = 0; pass < 3; ++pass) {
      hipLaunchKernelGGL(zero_hist, dim3(1), dim3(kBlock), 0, s, ws);
      hipLaunchKernelGGL(radix_hist, dim3(hist_grid), dim3(kBlock), 0, s, pred, target, n,
                         shifts[pass], widths[pass], pshift[pass], ws);
      hipLaunchKernelGGL(radix_select, dim3(1), dim3(kBlock), 0, s, widths[pass], pass == 2 ? 1 : 0,
                         ws, threshold_out);
    }
  } else if (threshold_out) {
    return fail(MR_EINVAL, "mr_loss_outlier: threshold_out is only written when it is computed");
  }
  const float gscale = static_cast<float>(2.0 / static_cast<double>(denom));
  hipLaunchKernelGGL(loss_pass, dim3(grid), dim3(kBlock), 0, s, pred, target, n, gscale,
                     threshold_in, ws, 1, grad_out, ws);
  hipLaunchKernelGGL(finalize, dim3(1), dim3(kBlock), 0, s, ws, grid, static_cast<double>(denom),
                     loss_out);
  MR_LAUNCH_CHECK("mr_loss_outlier");
  return MR_OK;
}

}  // extern "C"
