// Error reporting and small utilities of libmround_hip.
#include <cstdarg>
#include <cstdio>

#include "mr_common.h"

namespace mr {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t err, const char* what) {
  snprintf(g_last_error, sizeof(g_last_error), "%s: HIP error %d (%s)", what,
           static_cast<int>(err), hipGetErrorString(err));
  return MR_EHIP - static_cast<int>(err);
}

void clear_error() { g_last_error[0] = '\0'; }

// Grid-stride copy in 16-byte units plus a byte tail.
__global__ __launch_bounds__(256) void copy_kernel(const uint4* __restrict__ src,
                                                   uint4* __restrict__ dst, int64_t n16,
                                                   const uint8_t* __restrict__ src_tail,
                                                   uint8_t* __restrict__ dst_tail, int tail) {
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n16;
       i += stride) {
    dst[i] = src[i];
  }
  if (blockIdx.x == 0 && static_cast<int>(threadIdx.x) < tail) {
    dst_tail[threadIdx.x] = src_tail[threadIdx.x];
  }
}

// counter[0] += delta, one lane (a vector store).
__global__ void counter_add_kernel(int* counter, int delta) {
  if (threadIdx.x == 0) counter[0] = counter[0] + delta;
}

}  // namespace mr

extern "C" {

const char* mr_last_error(void) { return mr::g_last_error; }

int mr_counter_add(int* counter, int delta, void* stream) {
  mr::clear_error();
  if (!counter) return mr::fail(MR_EINVAL, "mr_counter_add: null counter");
  hipLaunchKernelGGL(mr::counter_add_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream),
                     counter, delta);
  MR_LAUNCH_CHECK("mr_counter_add");
  return MR_OK;
}

int mr_abi_version(void) { return 2; }

int mr_copy_bytes(const void* src, void* dst, size_t bytes, void* stream) {
  mr::clear_error();
  if (bytes == 0) return MR_OK;
  if (!src || !dst) return mr::fail(MR_EINVAL, "mr_copy_bytes: null pointer");
  if (!mr::aligned16(src) || !mr::aligned16(dst))
    return mr::fail(MR_EINVAL, "mr_copy_bytes: buffers must be 16-byte aligned");
  int64_t n16 = static_cast<int64_t>(bytes / 16);
  int tail = static_cast<int>(bytes % 16);
  int64_t want = (n16 + 255) / 256;
  int blocks = static_cast<int>(want < 8192 ? (want > 0 ? want : 1) : 8192);
  const uint8_t* s8 = static_cast<const uint8_t*>(src) + n16 * 16;
  uint8_t* d8 = static_cast<uint8_t*>(dst) + n16 * 16;
  hipLaunchKernelGGL(mr::copy_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint4*>(src),
                     static_cast<uint4*>(dst), n16, s8, d8, tail);
  MR_LAUNCH_CHECK("mr_copy_bytes");
  return MR_OK;
}

}  // extern "C"
