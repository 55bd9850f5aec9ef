// Block reconstruction losses with their gradient, for gfx950.
//
// mround/core/losses.py:42-130: r = pred - target in fp32; the plain loss keeps
// every element, the outlier loss keeps |r| < t where t is the k-th largest
// |r| of the whole batch (sort(|r|)[n - k]); every element tied at t is
// excluded. loss = sum(r_kept^2) / denom and dL/dpred = 2 r_kept / denom.
//
// The threshold is found exactly by a two-pass radix select on the bit
// pattern of |r| (non-negative floats order like their bit patterns, and the
// sign bit is dropped): a histogram of the top 15 bits (30..16) built in LDS
// per block, a one-block select of the bin holding the k-th largest, then a
// histogram of the low 16 bits among the elements of that bin only (global
// atomics, few elements), and a second select. Everything stays on the
// device; no host synchronisation.
//
// One pass over the data in the common case. A guess comes first: the top
// bits of the (2 ceil(k / 37) + 64)-th largest key in a sample of a 37th of
// the elements (every 37th run of 64), from a sample histogram and a select.
// The first pass then, besides the top-bits histogram, writes the gradient of
// every element, sums r^2 over the elements whose key lies below the guess
// (all of them kept whatever the threshold turns out to be, if it is at least
// the guess) and lists the others, the candidates, per wave (at most
// kCandCap each, in a fixed order: lanes in order within an iteration). When the guess lies at or below the
// selected top-bits bin and no wave's list overflowed, every element of that
// bin and above is a candidate: the low-bits histogram, the exclusion (the
// candidates at or above the threshold: their gradient set to zero) and the
// kept candidates' share of the loss are then formed from the lists alone.
// Otherwise, decided on the device, the low-bits histogram and the loss are
// passes over every element, and the first pass's gradient is overwritten.
// Both ways give the same threshold and gradient; the loss sums the same fp32
// squares in fp64, grouped differently. Which way is taken depends on the
// inputs alone, so equal inputs give equal bits.
//
// Sums are deterministic: a fixed grid of blocks, fp64 accumulation per
// thread (over a candidate list, lane j takes entries j, j + 64, ... in order,
// then a fixed butterfly), a fixed-order block reduction, then one block
// adding the partials in order.
#include <mutex>

#include "mr_common.h"

namespace mr {
namespace {

constexpr int kBlock = 256;
constexpr int kBlocks = 1024;
constexpr int kHiBits = 15, kLoBits = 16;
constexpr int kHiBins = 1 << kHiBits, kLoBins = 1 << kLoBits;
constexpr int kSelThreads = 1024;
constexpr int kHistThreads = 1024;

constexpr int kHistBlocks = 256;                             // the first pass's grid, at most
constexpr int kCandWaves = kHistBlocks * (kHistThreads / 64);  // one candidate list per wave
constexpr int kCandCap = 128;                                 // candidates listed per wave
struct Workspace {
  double partial[kBlocks];
  uint32_t hist_hi[kHiBins];
  uint32_t hist_lo[kLoBins];
  // [0] top-15-bit digit, [1] remaining rank k, [2] final key, [3] some wave
  // listed more than kCandCap candidates, [4] the guess key (all ones: none)
  uint32_t state[8];
  uint32_t hist_s[kHiBins];       // top bits of the sampled keys
  double low_part[kHistBlocks];   // first pass: sums below the guess, per block
  double seg_sum[kCandWaves];     // kept candidates' sums, per wave list
  uint32_t cand_count[kCandWaves];
  uint32_t cand_idx[kCandWaves * kCandCap];
  float cand_r[kCandWaves * kCandCap];
};
constexpr size_t kScratchBytes = sizeof(Workspace);
static_assert(kScratchBytes == 4778016, "the documented workspace size");
constexpr int64_t kMaxElements = 0xffffffffLL;  // histogram counts are 32-bit
constexpr int kMaxDevices = 64;

template <int THREADS = kBlock>
__device__ __forceinline__ double block_sum(double x, double* smem) {
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  const int wave = threadIdx.x / 64;
  if ((threadIdx.x % 64) == 0) smem[wave] = x;
  __syncthreads();
  double total = 0.0;
  if (threadIdx.x == 0) {
    for (int i = 0; i < THREADS / 64; ++i) total += smem[i];
  }
  return total;  // valid in thread 0
}

__device__ __forceinline__ uint32_t abs_key(float r) { return __float_as_uint(r) & 0x7fffffffu; }

// (The guess starts as none, an all-ones key: no element is listed.)
__global__ __launch_bounds__(kBlock) void zero_hist(Workspace* ws, uint32_t k) {
  const int i = blockIdx.x * kBlock + threadIdx.x;
  if (i < kHiBins) {
    ws->hist_hi[i] = 0;
    ws->hist_s[i] = 0;
  }
  if (i < kLoBins) ws->hist_lo[i] = 0;
  if (i == 0) {
    ws->state[0] = 0;
    ws->state[1] = k;
    ws->state[3] = 0;
    ws->state[4] = 0xffffffffu;
  }
}

// The sample: every 37th run of 64 consecutive elements (whole 256-byte
// pieces, so that the sample reads a 37th of the data; 37 is prime, so over
// rows of a multiple of 64 elements the runs visit every column alike).
constexpr int64_t kSampleStride = 37;
constexpr int64_t kSampleRun = 64;

__host__ __device__ constexpr int64_t sample_count(int64_t n) {
  return (n / (kSampleRun * kSampleStride)) * kSampleRun +
         ((n % (kSampleRun * kSampleStride)) < kSampleRun ? n % (kSampleRun * kSampleStride) : kSampleRun);
}

// Top bits of the sampled keys, per block in LDS.
__global__ __launch_bounds__(kHistThreads) void sample_hist(const float* __restrict__ pred,
                                                            const float* __restrict__ target, int64_t n,
                                                            Workspace* __restrict__ ws) {
  __shared__ uint32_t h[kHiBins];
  for (int i = threadIdx.x; i < kHiBins; i += kHistThreads) h[i] = 0;
  __syncthreads();
  const int64_t ns = sample_count(n);
  for (int64_t j = static_cast<int64_t>(blockIdx.x) * kHistThreads + threadIdx.x; j < ns;
       j += static_cast<int64_t>(gridDim.x) * kHistThreads) {
    const int64_t i = (j / kSampleRun) * (kSampleRun * kSampleStride) + j % kSampleRun;
    atomicAdd(&h[abs_key(pred[i] - target[i]) >> kLoBits], 1u);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kHiBins; i += kHistThreads)
    if (h[i]) atomicAdd(&ws->hist_s[i], h[i]);
}

// The candidate lists hold every element of the selected top-bits bin and above.
__device__ __forceinline__ bool lists_cover(const Workspace* ws) {
  return ws->state[3] == 0 && ws->state[4] <= (ws->state[0] << kLoBits);
}

// ... and the threshold is not a NaN (then |r| < t keeps nothing, which the
// key order would not say), so the loss can be formed from the lists.
__device__ __forceinline__ bool lists_serve_loss(const Workspace* ws) {
  return lists_cover(ws) && ws->state[2] <= 0x7f800000u;
}

// Pass 1, fused: the histogram of key >> 16 over every element (per block in
// LDS, 128 KB, then the block's non-empty bins added to the global one), the
// gradient of every element (2 r / denom, as if kept), r^2 summed over the
// elements under the guess key, and each wave's candidates (index and r, in
// lane order within an iteration). The lanes of a wave step through the data
// together, so a list's order and count are the wave's, not a lane's.
__global__ __launch_bounds__(kHistThreads) void loss_first_pass(const float* __restrict__ pred,
                                                                const float* __restrict__ target,
                                                                int64_t n, float grad_scale,
                                                                float* __restrict__ grad,
                                                                Workspace* __restrict__ ws) {
  __shared__ uint32_t h[kHiBins];
  __shared__ double smem[kHistThreads / 64];
  for (int i = threadIdx.x; i < kHiBins; i += kHistThreads) h[i] = 0;
  __syncthreads();
  const uint32_t gkey = ws->state[4];
  const int lane = threadIdx.x & 63;
  const int seg = blockIdx.x * (kHistThreads / 64) + (threadIdx.x >> 6);
  uint32_t* const cidx = ws->cand_idx + static_cast<int64_t>(seg) * kCandCap;
  float* const cr = ws->cand_r + static_cast<int64_t>(seg) * kCandCap;
  const uint64_t below = (1ull << lane) - 1ull;
  uint32_t wc = 0;  // candidates this wave has seen
  double acc = 0.0;
  auto take = [&](bool valid, float r, uint32_t idx) __attribute__((always_inline)) {
    const uint32_t key = abs_key(r);
    bool cand = false;
    if (valid) {
      atomicAdd(&h[key >> kLoBits], 1u);
      cand = key >= gkey;
      if (!cand) acc += static_cast<double>(r * r);
    }
    const uint64_t m = __ballot(cand);
    if (m) {
      if (cand) {
        const uint32_t slot = wc + static_cast<uint32_t>(__popcll(m & below));
        if (slot < kCandCap) {
          cidx[slot] = idx;
          cr[slot] = r;
        }
      }
      wc += static_cast<uint32_t>(__popcll(m));
    }
  };
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kHistThreads;
  const int64_t wave_first = static_cast<int64_t>(blockIdx.x) * kHistThreads + (threadIdx.x & ~63);
  if ((n & 3) == 0) {
    const int64_t n4 = n / 4;
    const float4* p4 = reinterpret_cast<const float4*>(pred);
    const float4* t4 = reinterpret_cast<const float4*>(target);
    for (int64_t w0 = wave_first; w0 < n4; w0 += stride) {
      const int64_t i = w0 + lane;
      const bool valid = i < n4;
      float4 p = make_float4(0.f, 0.f, 0.f, 0.f), q = p;
      if (valid) {
        p = p4[i];
        q = t4[i];
      }
      const float r0 = p.x - q.x, r1 = p.y - q.y, r2 = p.z - q.z, r3 = p.w - q.w;
      const uint32_t e = static_cast<uint32_t>(4 * i);
      take(valid, r0, e);
      take(valid, r1, e + 1);
      take(valid, r2, e + 2);
      take(valid, r3, e + 3);
      if (grad && valid)
        reinterpret_cast<float4*>(grad)[i] =
            make_float4(r0 * grad_scale, r1 * grad_scale, r2 * grad_scale, r3 * grad_scale);
    }
  } else {
    for (int64_t w0 = wave_first; w0 < n; w0 += stride) {
      const int64_t i = w0 + lane;
      const bool valid = i < n;
      const float r = valid ? pred[i] - target[i] : 0.0f;
      take(valid, r, static_cast<uint32_t>(i));
      if (grad && valid) grad[i] = r * grad_scale;
    }
  }
  if (lane == 0) {
    ws->cand_count[seg] = wc;
    if (wc > kCandCap) atomicOr(&ws->state[3], 1u);
  }
  const double total = block_sum<kHistThreads>(acc, smem);
  if (threadIdx.x == 0) ws->low_part[blockIdx.x] = total;
  for (int i = threadIdx.x; i < kHiBins; i += kHistThreads)
    if (h[i]) atomicAdd(&ws->hist_hi[i], h[i]);
}

// With the lists covering the threshold: zero the gradient of the listed
// elements at or above it, and sum r^2 of the others, per list in list order.
__global__ __launch_bounds__(kHistThreads) void loss_lists(float* __restrict__ grad, Workspace* __restrict__ ws,
                                                           int nseg) {
  if (!lists_serve_loss(ws)) return;
  const uint32_t tkey = ws->state[2];
  const int lane = threadIdx.x & 63;
  const int seg = blockIdx.x * (kHistThreads / 64) + (threadIdx.x >> 6);
  if (seg >= nseg) return;
  const uint32_t* const cidx = ws->cand_idx + static_cast<int64_t>(seg) * kCandCap;
  const float* const cr = ws->cand_r + static_cast<int64_t>(seg) * kCandCap;
  const int cnt = static_cast<int>(ws->cand_count[seg]);  // at most kCandCap here
  double acc = 0.0;
  for (int j = lane; j < cnt; j += 64) {
    const float r = cr[j];
    if (abs_key(r) >= tkey) {
      if (grad) grad[cidx[j]] = 0.0f;
    } else {
      acc += static_cast<double>(r * r);
    }
  }
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) ws->seg_sum[seg] = acc;
}

// Pass 2: histogram of the low 16 bits among the elements whose top 15 bits
// are the chosen digit, straight into global memory.
// (nseg > 0: after the fused first pass; when its lists cover the chosen bin,
// the histogram is formed from the lists, a wave per list.)
__global__ __launch_bounds__(kHistThreads) void radix_hist_lo(const float* __restrict__ pred,
                                                              const float* __restrict__ target,
                                                              int64_t n, Workspace* __restrict__ ws,
                                                              int nseg) {
  const uint32_t digit = ws->state[0];
  if (nseg > 0 && lists_cover(ws)) {
    const int seg = blockIdx.x * (kHistThreads / 64) + (threadIdx.x >> 6);
    if (seg >= nseg) return;
    const float* const cr = ws->cand_r + static_cast<int64_t>(seg) * kCandCap;
    const int cnt = static_cast<int>(ws->cand_count[seg]);
    for (int j = threadIdx.x & 63; j < cnt; j += 64) {
      const uint32_t key = abs_key(cr[j]);
      if ((key >> kLoBits) == digit) atomicAdd(&ws->hist_lo[key & (kLoBins - 1)], 1u);
    }
    return;
  }
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kHistThreads;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kHistThreads + threadIdx.x;
  auto one = [&](float r) {
    const uint32_t key = abs_key(r);
    if ((key >> kLoBits) == digit) {
      // lanes sharing one key (ties, the common case among few matches)
      // add once: keeps a degenerate input from serialising on one address
      const uint32_t k0 = __builtin_amdgcn_readfirstlane(key);
      const uint64_t same = __ballot(key == k0), all = __ballot(1);
      if (same == all) {
        if (__lane_id() == static_cast<unsigned>(__builtin_ctzll(all)))
          atomicAdd(&ws->hist_lo[k0 & (kLoBins - 1)], static_cast<uint32_t>(__popcll(all)));
      } else {
        atomicAdd(&ws->hist_lo[key & (kLoBins - 1)], 1u);
      }
    }
  };
  if ((n & 3) == 0) {
    const float4* p4 = reinterpret_cast<const float4*>(pred);
    const float4* t4 = reinterpret_cast<const float4*>(target);
    for (int64_t i = first; i < n / 4; i += stride) {
      const float4 p = p4[i], q = t4[i];
      one(p.x - q.x);
      one(p.y - q.y);
      one(p.z - q.z);
      one(p.w - q.w);
    }
  } else {
    for (int64_t i = first; i < n; i += stride) one(pred[i] - target[i]);
  }
}

// The bin holding the k-th largest key: the largest b with
// count(bins > b) < k <= count(bins >= b). One block; thread t owns the
// per = nbins / kSelThreads consecutive bins starting at t * per (read as
// 16-byte vectors). A suffix sum over the threads finds the owner of that
// bin; one wave then scans the owner's bins, a lane per bin. Pass 1 records
// the digit and the rank left inside its bin; pass 2 forms the final key;
// the sample select (hi = 2, rank ks, at most the sample count) the guess,
// the lower edge of the bin.
__global__ __launch_bounds__(kSelThreads) void radix_select(int hi, Workspace* ws,
                                                            float* __restrict__ threshold_out,
                                                            uint32_t ks) {
  __shared__ uint32_t wave_total[kSelThreads / 64];
  __shared__ uint32_t win[2];  // owner thread, count strictly above its bins
  const uint32_t* hist = hi == 2 ? ws->hist_s : hi ? ws->hist_hi : ws->hist_lo;
  const int per = (hi ? kHiBins : kLoBins) / kSelThreads;  // 32 or 64
  const int t = threadIdx.x;
  const uint4* h4 = reinterpret_cast<const uint4*>(hist + t * per);
  uint32_t mine = 0;
  for (int j = 0; j < per / 4; ++j) {
    const uint4 v = h4[j];
    mine += v.x + v.y + v.z + v.w;
  }
  // suffix sums over threads: within each wave by shuffles, then the totals
  // of the waves above (integer sums, so the order does not matter)
  uint32_t above = mine;
  const int lane_t = t & 63, wave_t = t >> 6;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t v = __shfl_down(above, off, 64);
    if (lane_t + off < 64) above += v;
  }
  if (lane_t == 0) wave_total[wave_t] = above;
  __syncthreads();
  for (int w = wave_t + 1; w < kSelThreads / 64; ++w) above += wave_total[w];
  const uint32_t k = hi == 2 ? ks : ws->state[1];
  const uint32_t run0 = above - mine;  // strictly above thread t's bins
  if (run0 < k && k <= run0 + mine) {
    win[0] = static_cast<uint32_t>(t);
    win[1] = run0;
  }
  __syncthreads();
  if (t >= 64) return;
  // wave 0: lane l holds bin win[0] * per + l; suffix sums over the lanes
  const int lane = t;
  const int b = static_cast<int>(win[0]) * per + lane;
  const uint32_t c = lane < per ? hist[b] : 0u;
  uint32_t suf = c;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t v = __shfl_down(suf, off, 64);
    if (lane + off < 64) suf += v;
  }
  const uint32_t above_b = win[1] + suf - c;  // count in bins > b
  if (lane < per && above_b < k && k <= above_b + c) {
    if (hi == 2) {
      ws->state[4] = static_cast<uint32_t>(b) << kLoBits;
    } else if (hi) {
      ws->state[0] = static_cast<uint32_t>(b);
      ws->state[1] = k - above_b;
    } else {
      const uint32_t key = (ws->state[0] << kLoBits) | static_cast<uint32_t>(b);
      ws->state[2] = key;
      if (threshold_out) *threshold_out = __uint_as_float(key);
    }
  }
}

// Loss and gradient. keep = |r| < threshold when a threshold is given.
// (after_lists: the fused first pass ran; nothing to do when its lists serve.)
__global__ __launch_bounds__(kBlock) void loss_pass(const float* __restrict__ pred,
                                                    const float* __restrict__ target, int64_t n,
                                                    float grad_scale, const float* __restrict__ thr_in,
                                                    const Workspace* __restrict__ thr_ws, int use_thr,
                                                    float* __restrict__ grad, Workspace* __restrict__ ws,
                                                    int after_lists) {
  if (after_lists && lists_serve_loss(ws)) return;
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

// (nseg > 0: after the fused first pass; when its lists serve, the loss is
// the first pass's block sums plus the lists' sums.)
__global__ __launch_bounds__(kBlock) void finalize(const Workspace* __restrict__ ws, int nparts,
                                                   double denom, float* __restrict__ loss_out, int nlow,
                                                   int nseg) {
  __shared__ double smem[kBlock / 64];
  double acc = 0.0;
  // Fixed assignment of partials to threads and a fixed tree: deterministic.
  if (nseg > 0 && lists_serve_loss(ws)) {
    for (int i = threadIdx.x; i < nlow; i += kBlock) acc += ws->low_part[i];
    for (int i = threadIdx.x; i < nseg; i += kBlock) acc += ws->seg_sum[i];
  } else {
    for (int i = threadIdx.x; i < nparts; i += kBlock) acc += ws->partial[i];
  }
  double total = block_sum(acc, smem);
  if (threadIdx.x == 0) *loss_out = static_cast<float>(total / denom);
}

int grid_for(int64_t n) {
  int64_t want = (n / 4 + kBlock - 1) / kBlock;
  if (want < 1) want = 1;
  return static_cast<int>(want < kBlocks ? want : kBlocks);
}

int check_loss(const char* fn, const float* pred, const float* target, int64_t n, int64_t denom,
               float* loss_out) {
  if (!pred || !target || !loss_out) return fail(MR_EINVAL, "%s: null pointer", fn);
  if (n <= 0) return fail(MR_EINVAL, "%s: empty input", fn);
  if (denom <= 0) return fail(MR_EINVAL, "%s: denominator must be positive", fn);
  if ((n % 4) == 0 && (!aligned16(pred) || !aligned16(target)))
    return fail(MR_EINVAL, "%s: inputs must be 16-byte aligned", fn);
  return MR_OK;
}

// The outlier loss on workspace ws (checked by the caller).
int outlier(const char* fn, const float* pred, const float* target, int64_t n, int64_t k, int64_t denom,
            const float* threshold_in, float* threshold_out, float* loss_out, float* grad_out,
            Workspace* ws, hipStream_t s) {
  if (!threshold_in && (k < 1 || k > n))
    return fail(MR_EINVAL, "%s: rank k=%lld outside [1, n]", fn, static_cast<long long>(k));
  if (n > kMaxElements)
    return fail(MR_EINVAL, "%s: %lld elements, more than the %lld the select counts", fn,
                static_cast<long long>(n), static_cast<long long>(kMaxElements));
  if (grad_out && (n % 4) == 0 && !aligned16(grad_out))
    return fail(MR_EINVAL, "%s: gradient must be 16-byte aligned", fn);
  // the select's later passes read pred and target again after the first
  // pass has written the gradient
  if (!threshold_in && grad_out &&
      (overlap(grad_out, n * 4, pred, n * 4) || overlap(grad_out, n * 4, target, n * 4)))
    return fail(MR_EINVAL, "%s: grad_out must not overlap pred or target", fn);
  const int grid = grid_for(n);
  const float gscale = static_cast<float>(2.0 / static_cast<double>(denom));
  if (!threshold_in) {
    int64_t hg = ((n & 3) == 0 ? n / 4 : n) / kHistThreads + 1;
    const int hist_grid = static_cast<int>(hg < kHistBlocks ? hg : kHistBlocks);
    const int nseg = hist_grid * (kHistThreads / 64);
    hipLaunchKernelGGL(zero_hist, dim3(kLoBins / kBlock), dim3(kBlock), 0, s, ws, static_cast<uint32_t>(k));
    // the guess: rank 2 ceil(k / 37) + 64 among the samples (none when the sample is smaller)
    const int64_t ns = sample_count(n);
    const int64_t ks = 2 * ((k + kSampleStride - 1) / kSampleStride) + 64;
    if (ks <= ns) {
      const int64_t sg = ns / kHistThreads + 1;
      hipLaunchKernelGGL(sample_hist, dim3(static_cast<unsigned>(sg < kHistBlocks ? sg : kHistBlocks)),
                         dim3(kHistThreads), 0, s, pred, target, n, ws);
      hipLaunchKernelGGL(radix_select, dim3(1), dim3(kSelThreads), 0, s, 2, ws, nullptr,
                         static_cast<uint32_t>(ks));
    }
    hipLaunchKernelGGL(loss_first_pass, dim3(hist_grid), dim3(kHistThreads), 0, s, pred, target, n, gscale,
                       grad_out, ws);
    hipLaunchKernelGGL(radix_select, dim3(1), dim3(kSelThreads), 0, s, 1, ws, threshold_out, 0u);
    hipLaunchKernelGGL(radix_hist_lo, dim3(hist_grid), dim3(kHistThreads), 0, s, pred, target, n, ws, nseg);
    hipLaunchKernelGGL(radix_select, dim3(1), dim3(kSelThreads), 0, s, 0, ws, threshold_out, 0u);
    hipLaunchKernelGGL(loss_lists, dim3(hist_grid), dim3(kHistThreads), 0, s, grad_out, ws, nseg);
    hipLaunchKernelGGL(loss_pass, dim3(grid), dim3(kBlock), 0, s, pred, target, n, gscale, nullptr, ws, 1,
                       grad_out, ws, 1);
    hipLaunchKernelGGL(finalize, dim3(1), dim3(kBlock), 0, s, ws, grid, static_cast<double>(denom), loss_out,
                       hist_grid, nseg);
    MR_LAUNCH_CHECK(fn);
    return MR_OK;
  }
  if (threshold_out) return fail(MR_EINVAL, "%s: threshold_out is only written when it is computed", fn);
  hipLaunchKernelGGL(loss_pass, dim3(grid), dim3(kBlock), 0, s, pred, target, n, gscale,
                     threshold_in, ws, 1, grad_out, ws, 0);
  hipLaunchKernelGGL(finalize, dim3(1), dim3(kBlock), 0, s, ws, grid, static_cast<double>(denom),
                     loss_out, 0, 0);
  MR_LAUNCH_CHECK(fn);
  return MR_OK;
}

}  // namespace
}  // namespace mr

// The allocation-free outlier loss keeps its workspace in this array, one
// copy per GPU, held until the process ends (kScratchBytes = the Workspace,
// 4,778,016 bytes). Host code never passes the array's name to a kernel: that
// name is a host-side stand-in. The device address comes from
// hipGetSymbolAddress, once per device, on the first call there.
static __device__ __align__(256) unsigned char scratch[mr::kScratchBytes];

namespace mr {
namespace {

int scratch_address(void** out) {
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "mr_loss_outlier_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MR_EINVAL, "mr_loss_outlier_noalloc: device %d past the %d supported", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "mr_loss_outlier_noalloc: hipGetSymbolAddress(scratch)");
    addr[dev] = p;
  }
  *out = addr[dev];
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
  int rc = check_loss("mr_loss_mse", pred, target, n, denom, loss_out);
  if (rc) return rc;
  if (!workspace) return fail(MR_EINVAL, "mr_loss_mse: null workspace");
  if (grad_out && (n % 4) == 0 && !aligned16(grad_out))
    return fail(MR_EINVAL, "mr_loss_mse: gradient must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  Workspace* ws = static_cast<Workspace*>(workspace);
  const int grid = grid_for(n);
  const float gscale = static_cast<float>(2.0 / static_cast<double>(denom));
  hipLaunchKernelGGL(loss_pass, dim3(grid), dim3(kBlock), 0, s, pred, target, n, gscale, nullptr,
                     nullptr, 0, grad_out, ws, 0);
  hipLaunchKernelGGL(finalize, dim3(1), dim3(kBlock), 0, s, ws, grid, static_cast<double>(denom),
                     loss_out, 0, 0);
  MR_LAUNCH_CHECK("mr_loss_mse");
  return MR_OK;
}

int mr_loss_outlier(const float* pred, const float* target, int64_t n, int64_t k, int64_t denom,
                    const float* threshold_in, float* threshold_out, float* loss_out,
                    float* grad_out, void* workspace, void* stream) {
  using namespace mr;
  clear_error();
  int rc = check_loss("mr_loss_outlier", pred, target, n, denom, loss_out);
  if (rc) return rc;
  if (!workspace) return fail(MR_EINVAL, "mr_loss_outlier: null workspace");
  return outlier("mr_loss_outlier", pred, target, n, k, denom, threshold_in, threshold_out, loss_out,
                 grad_out, static_cast<Workspace*>(workspace), static_cast<hipStream_t>(stream));
}

int mr_loss_outlier_noalloc(const float* pred, const float* target, int64_t n, int64_t k,
                            int64_t denom, const float* threshold_in, float* threshold_out,
                            float* loss_out, float* grad_out, void* stream) {
  using namespace mr;
  clear_error();
  int rc = check_loss("mr_loss_outlier_noalloc", pred, target, n, denom, loss_out);
  if (rc) return rc;
  void* ws = nullptr;
  rc = scratch_address(&ws);
  if (rc) return rc;
  return outlier("mr_loss_outlier_noalloc", pred, target, n, k, denom, threshold_in, threshold_out,
                 loss_out, grad_out, static_cast<Workspace*>(ws), static_cast<hipStream_t>(stream));
}

}  // extern "C"
