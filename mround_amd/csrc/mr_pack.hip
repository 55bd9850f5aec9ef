// MLX uint32 packing, unpacking and affine metadata, for gfx950.
//
// Layout (mround/formats/packing.py:84-206; oracle mround/reference/packing.py):
// a row of codes is a little-endian bitstream, element i occupying bits
// [i*b, (i+1)*b). For b in {2, 4, 8} no element straddles a word and this is
// the "even" layout; for b in {3, 5, 6, 7} it is the cross-word layout. In
// both, 32 consecutive codes fill exactly b words, so the fast kernels give
// each lane one 32-code chunk: two 16-byte loads in, b words out, with the
// chunk's bits assembled in a 64-bit shift register. Rows whose length is not
// a multiple of 32 (possible only for even widths) use a word-per-lane kernel.
#include <climits>

#include "mr_common.h"

namespace mr {
namespace {

constexpr int kBlock = 256;

__global__ void init_range(int32_t* range) {
  range[0] = INT_MAX;
  range[1] = INT_MIN;
}

__device__ __forceinline__ void report_range(int32_t* range, int lo, int hi) {
  for (int off = 32; off > 0; off >>= 1) {
    lo = min(lo, __shfl_xor(lo, off, 64));
    hi = max(hi, __shfl_xor(hi, off, 64));
  }
  if ((threadIdx.x % 64) == 0) {
    atomicMin(range, lo);
    atomicMax(range + 1, hi);
  }
}

template <int BITS>
__global__ __launch_bounds__(kBlock) void pack_fast(const uint8_t* __restrict__ codes, int sgn,
                                                    int offset, int64_t n_chunks,
                                                    uint32_t* __restrict__ out,
                                                    int32_t* __restrict__ range) {
  int64_t chunk = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const bool active = chunk < n_chunks;
  int lo = INT_MAX, hi = INT_MIN;
  if (active) {
    const uint4* src = reinterpret_cast<const uint4*>(codes + chunk * 32);
    uint4 q0 = src[0], q1 = src[1];
    uint32_t raw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    uint64_t acc = 0;
    int nbits = 0;
    int word = 0;
    uint32_t words[BITS];
    constexpr uint32_t mask = (1u << BITS) - 1u;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      uint32_t byte = (raw[i >> 2] >> (8 * (i & 3))) & 0xffu;
      int val = (sgn ? static_cast<int>(static_cast<int8_t>(byte)) : static_cast<int>(byte)) + offset;
      lo = min(lo, val);
      hi = max(hi, val);
      acc |= static_cast<uint64_t>(static_cast<uint32_t>(val) & mask) << nbits;
      nbits += BITS;
      if (nbits >= 32) {
        words[word++] = static_cast<uint32_t>(acc);
        acc >>= 32;
        nbits -= 32;
      }
    }
    uint32_t* dst = out + chunk * BITS;
#pragma unroll
    for (int k = 0; k < BITS; ++k) dst[k] = words[k];
  }
  if (range) report_range(range, lo, hi);
}

// Even widths, any row length that tiles words: one word per lane.
__global__ __launch_bounds__(kBlock) void pack_words(const uint8_t* __restrict__ codes, int sgn,
                                                     int offset, int64_t rows, int64_t cols,
                                                     int bits, int64_t words,
                                                     uint32_t* __restrict__ out,
                                                     int32_t* __restrict__ range) {
  int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  int lo = INT_MAX, hi = INT_MIN;
  if (idx < rows * words) {
    int64_t r = idx / words, wd = idx % words;
    int per = 32 / bits;
    uint32_t mask = (1u << bits) - 1u;
    uint32_t acc = 0;
    for (int i = 0; i < per; ++i) {
      uint32_t byte = codes[r * cols + wd * per + i];
      int val = (sgn ? static_cast<int>(static_cast<int8_t>(byte)) : static_cast<int>(byte)) + offset;
      lo = min(lo, val);
      hi = max(hi, val);
      acc |= (static_cast<uint32_t>(val) & mask) << (i * bits);
    }
    out[idx] = acc;
  }
  if (range) report_range(range, lo, hi);
}

template <int BITS>
__global__ __launch_bounds__(kBlock) void unpack_fast(const uint32_t* __restrict__ packed,
                                                      int64_t n_chunks, uint8_t* __restrict__ codes) {
  int64_t chunk = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (chunk >= n_chunks) return;
  const uint32_t* src = packed + chunk * BITS;
  uint32_t words[BITS];
#pragma unroll
  for (int k = 0; k < BITS; ++k) words[k] = src[k];
  uint32_t out[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  constexpr uint32_t mask = (1u << BITS) - 1u;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const int bit = i * BITS;
    const int wd = bit >> 5, off = bit & 31;
    uint32_t val = words[wd] >> off;
    if (off + BITS > 32) val |= words[wd + 1] << (32 - off);
    out[i >> 2] |= (val & mask) << (8 * (i & 3));
  }
  uint4* dst = reinterpret_cast<uint4*>(codes + chunk * 32);
  dst[0] = make_uint4(out[0], out[1], out[2], out[3]);
  dst[1] = make_uint4(out[4], out[5], out[6], out[7]);
}

__global__ __launch_bounds__(kBlock) void unpack_words(const uint32_t* __restrict__ packed,
                                                       int64_t rows, int64_t cols, int bits,
                                                       int64_t words, uint8_t* __restrict__ codes) {
  int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (idx >= rows * words) return;
  int64_t r = idx / words, wd = idx % words;
  int per = 32 / bits;
  uint32_t mask = (1u << bits) - 1u;
  uint32_t word = packed[idx];
  for (int i = 0; i < per; ++i) codes[r * cols + wd * per + i] = static_cast<uint8_t>((word >> (i * bits)) & mask);
}

template <int OT>
__global__ __launch_bounds__(kBlock) void affine_kernel(const float* __restrict__ scale,
                                                        const float* __restrict__ zp, int64_t n,
                                                        float sym_offset, void* __restrict__ scales,
                                                        void* __restrict__ biases) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= n) return;
  // Round the scale to the stored dtype first; the bias is formed from the
  // stored value (mround/formats/mlx_export.py:186-195). A bf16/fp16 scale times
  // an integer zero point below 2^8 is exact in fp32, so one rounding remains.
  const float s = round_to<OT>(scale[i]);
  const float z = zp ? round_to<OT>(zp[i]) : sym_offset;
  store_elem<OT>(scales, i, s);
  store_elem<OT>(biases, i, -s * z);
}

}  // namespace
}  // namespace mr

extern "C" {

int64_t mr_packed_width(int64_t cols, int bits) {
  using namespace mr;
  clear_error();
  if (bits < 2 || bits > 8)
    return fail(MR_EINVAL, "bits must be one of {2, 3, 4, 5, 6, 7, 8}, got %d", bits);
  if (cols < 0) return fail(MR_EINVAL, "negative row length");
  if (32 % bits == 0) {
    int per = 32 / bits;
    if (cols % per)
      return fail(MR_EINVAL, "in_features=%lld is not a multiple of %d codes per word at %d bits",
                  static_cast<long long>(cols), per, bits);
    return cols / per;
  }
  if (cols % 32)
    return fail(MR_EINVAL,
                "in_features=%lld is not a multiple of 32, which the cross-word bitstream "
                "layout requires at %d bits",
                static_cast<long long>(cols), bits);
  return cols / 32 * bits;
}

int mr_pack_codes(const void* codes, int codes_signed, int code_offset, int64_t rows,
                  int64_t cols, int bits, uint32_t* packed_out, int32_t* range_out,
                  void* stream) {
  using namespace mr;
  int64_t words = mr_packed_width(cols, bits);
  if (words < 0) return static_cast<int>(words);
  clear_error();
  if (!codes || !packed_out) return fail(MR_EINVAL, "mr_pack_codes: null pointer");
  if (rows < 0) return fail(MR_EINVAL, "mr_pack_codes: negative rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (range_out) {
    hipLaunchKernelGGL(init_range, dim3(1), dim3(1), 0, s, range_out);
    MR_LAUNCH_CHECK("mr_pack_codes");
  }
  if (rows == 0 || cols == 0) return MR_OK;
  const uint8_t* c8 = static_cast<const uint8_t*>(codes);
  if (cols % 32 == 0 && aligned16(codes)) {
    int64_t n_chunks = rows * cols / 32;
    int64_t blocks = (n_chunks + kBlock - 1) / kBlock;
    switch (bits) {
#define MR_PACK_CASE(B)                                                                       \
  case B:                                                                                     \
    hipLaunchKernelGGL(pack_fast<B>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, \
                       c8, codes_signed, code_offset, n_chunks, packed_out, range_out);       \
    break;
      MR_PACK_CASE(2) MR_PACK_CASE(3) MR_PACK_CASE(4) MR_PACK_CASE(5) MR_PACK_CASE(6)
      MR_PACK_CASE(7) MR_PACK_CASE(8)
#undef MR_PACK_CASE
    }
  } else {
    if (32 % bits != 0) return fail(MR_EINVAL, "mr_pack_codes: unaligned codes buffer");
    int64_t blocks = (rows * words + kBlock - 1) / kBlock;
    hipLaunchKernelGGL(pack_words, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, c8,
                       codes_signed, code_offset, rows, cols, bits, words, packed_out, range_out);
  }
  MR_LAUNCH_CHECK("mr_pack_codes");
  return MR_OK;
}

int mr_unpack_codes(const uint32_t* packed, int64_t rows, int64_t cols, int bits,
                    uint8_t* codes_out, void* stream) {
  using namespace mr;
  int64_t words = mr_packed_width(cols, bits);
  if (words < 0) return static_cast<int>(words);
  clear_error();
  if (!packed || !codes_out) return fail(MR_EINVAL, "mr_unpack_codes: null pointer");
  if (rows <= 0 || cols == 0) return MR_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (cols % 32 == 0 && aligned16(codes_out)) {
    int64_t n_chunks = rows * cols / 32;
    int64_t blocks = (n_chunks + kBlock - 1) / kBlock;
    switch (bits) {
#define MR_UNPACK_CASE(B)                                                                      \
  case B:                                                                                      \
    hipLaunchKernelGGL(unpack_fast<B>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, \
                       packed, n_chunks, codes_out);                                           \
    break;
      MR_UNPACK_CASE(2) MR_UNPACK_CASE(3) MR_UNPACK_CASE(4) MR_UNPACK_CASE(5) MR_UNPACK_CASE(6)
      MR_UNPACK_CASE(7) MR_UNPACK_CASE(8)
#undef MR_UNPACK_CASE
    }
  } else {
    if (32 % bits != 0) return fail(MR_EINVAL, "mr_unpack_codes: unaligned codes buffer");
    int64_t blocks = (rows * words + kBlock - 1) / kBlock;
    hipLaunchKernelGGL(unpack_words, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s,
                       packed, rows, cols, bits, words, codes_out);
  }
  MR_LAUNCH_CHECK("mr_unpack_codes");
  return MR_OK;
}

int mr_to_affine(const float* scale, const float* zp, int64_t n_groups, int bits, int out_dtype,
                 void* scales_out, void* biases_out, void* stream) {
  using namespace mr;
  clear_error();
  if (!scale || !scales_out || !biases_out) return fail(MR_EINVAL, "mr_to_affine: null pointer");
  if (!valid_dtype(out_dtype)) return fail(MR_EINVAL, "mr_to_affine: unknown dtype %d", out_dtype);
  if (bits < 2 || bits > 8) return fail(MR_EINVAL, "mr_to_affine: bad bits %d", bits);
  if (n_groups <= 0) return MR_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int64_t blocks = (n_groups + kBlock - 1) / kBlock;
  float off = static_cast<float>(1 << (bits - 1));
  if (out_dtype == MR_BF16)
    hipLaunchKernelGGL(affine_kernel<MR_BF16>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0,
                       s, scale, zp, n_groups, off, scales_out, biases_out);
  else if (out_dtype == MR_F16)
    hipLaunchKernelGGL(affine_kernel<MR_F16>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0,
                       s, scale, zp, n_groups, off, scales_out, biases_out);
  else
    hipLaunchKernelGGL(affine_kernel<MR_F32>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0,
                       s, scale, zp, n_groups, off, scales_out, biases_out);
  MR_LAUNCH_CHECK("mr_to_affine");
  return MR_OK;
}

}  // extern "C"
