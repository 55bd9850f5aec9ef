// Shared helpers for the libmround_hip kernels (gfx950).
//
// Element conversions: bf16 and fp16 widen exactly, and narrowing rounds to
// nearest, ties to even, which is what torch and MLX do.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/mround_hip.h"

namespace mr {

// Error plumbing: a thread-local message and status codes (mr_common.hip).
int fail(int code, const char* fmt, ...);
int hip_fail(hipError_t err, const char* what);
void clear_error();

#define MR_LAUNCH_CHECK(what)                                        \
  do {                                                               \
    hipError_t e_ = hipGetLastError();                               \
    if (e_ != hipSuccess) return ::mr::hip_fail(e_, what);           \
  } while (0)

inline bool valid_dtype(int dt) { return dt == MR_F32 || dt == MR_BF16 || dt == MR_F16; }
inline int dtype_bytes(int dt) { return dt == MR_F32 ? 4 : 2; }

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Narrowing to bfloat16 rounds to nearest even; a NaN keeps its sign and high
// payload bits and is made quiet. gfx950 does this in one instruction for two
// values (v_cvt_pk_bf16_f32, low half from the first operand); the device
// test of mr_cast_f32_bf16 compares it with that bit-pattern rule on all 2^32
// inputs.
typedef float mr_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 mr_bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const mr_f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, mr_bf16x2));
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

// Logistic function with the hardware reciprocal (1 ulp), shared by the
// SwiGLU GEMM epilogues and the split-precision SwiGLU kernel: the epilogues
// are tolerance-checked, not bit-exact, and an IEEE division per element keeps
// the unrolled epilogue from fitting in registers.
__device__ __forceinline__ float sigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float silu(float x) { return x * sigmoid(x); }

template <int DT>
__device__ __forceinline__ float load_elem(const void* p, int64_t i) {
  if constexpr (DT == MR_F32) {
    return static_cast<const float*>(p)[i];
  } else if constexpr (DT == MR_BF16) {
    return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else {
    return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
}

template <int DT>
__device__ __forceinline__ void store_elem(void* p, int64_t i, float x) {
  if constexpr (DT == MR_F32) {
    static_cast<float*>(p)[i] = x;
  } else if constexpr (DT == MR_BF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(x);
  } else {
    static_cast<uint16_t*>(p)[i] = f32_to_f16(x);
  }
}

// x narrowed to DT and widened back: the value store_elem<DT> would store.
template <int DT>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (DT == MR_F32) {
    return x;
  } else if constexpr (DT == MR_BF16) {
    return bf16_to_f32(f32_to_bf16(x));
  } else {
    return f16_to_f32(f32_to_f16(x));
  }
}

// 16-byte streaming accesses. Data read or written exactly once per pass goes
// through these nontemporal forms, which keep it from displacing reused lines
// in the caches; measured faster than plain accesses on the fake-quant passes.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld16_stream(const void* p) {
  u32x4_t r = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(r.x, r.y, r.z, r.w);
}

__device__ __forceinline__ void st16_stream(void* p, uint4 v) {
  u32x4_t r = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(r, reinterpret_cast<u32x4_t*>(p));
}

// Eight consecutive elements starting at element index i (i % 8 == 0 and the
// base pointer 16-byte aligned): one 16-byte load for 2-byte types, two for fp32.
template <int DT>
__device__ __forceinline__ void load8(const void* p, int64_t i, float (&out)[8]) {
  if constexpr (DT == MR_F32) {
    const float* q = static_cast<const float*>(p) + i;
    uint4 a = ld16_stream(q), b = ld16_stream(q + 4);
    out[0] = __uint_as_float(a.x); out[1] = __uint_as_float(a.y);
    out[2] = __uint_as_float(a.z); out[3] = __uint_as_float(a.w);
    out[4] = __uint_as_float(b.x); out[5] = __uint_as_float(b.y);
    out[6] = __uint_as_float(b.z); out[7] = __uint_as_float(b.w);
  } else {
    uint4 r = ld16_stream(static_cast<const uint16_t*>(p) + i);
    uint32_t words[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint16_t lo = static_cast<uint16_t>(words[k] & 0xffffu);
      uint16_t hi = static_cast<uint16_t>(words[k] >> 16);
      if constexpr (DT == MR_BF16) {
        out[2 * k] = bf16_to_f32(lo);
        out[2 * k + 1] = bf16_to_f32(hi);
      } else {
        out[2 * k] = f16_to_f32(lo);
        out[2 * k + 1] = f16_to_f32(hi);
      }
    }
  }
}

template <int DT>
__device__ __forceinline__ void store8(void* p, int64_t i, const float (&x)[8]) {
  if constexpr (DT == MR_F32) {
    float* q = static_cast<float*>(p) + i;
    st16_stream(q, make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]),
                              __float_as_uint(x[3])));
    st16_stream(q + 4, make_uint4(__float_as_uint(x[4]), __float_as_uint(x[5]),
                                  __float_as_uint(x[6]), __float_as_uint(x[7])));
  } else {
    uint32_t words[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (DT == MR_BF16) {
        words[k] = pack_bf16x2(x[2 * k], x[2 * k + 1]);
      } else {
        words[k] = static_cast<uint32_t>(f32_to_f16(x[2 * k])) |
                   (static_cast<uint32_t>(f32_to_f16(x[2 * k + 1])) << 16);
      }
    }
    st16_stream(static_cast<uint16_t*>(p) + i, make_uint4(words[0], words[1], words[2], words[3]));
  }
}

__device__ __forceinline__ void load8_f32(const float* p, int64_t i, float (&out)[8]) {
  load8<MR_F32>(p, i, out);
}

__device__ __forceinline__ void store8_f32(float* p, int64_t i, const float (&x)[8]) {
  store8<MR_F32>(p, i, x);
}

// Eight fp32 through the caches (plain 16-byte accesses). Measured on the
// fake-quant passes over the learnable v (read, then rewritten in place by the
// update): 8-10 % faster than the streaming forms above.
__device__ __forceinline__ void load8_f32_cached(const float* p, int64_t i, float (&out)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p + i);
  const float4 b = *reinterpret_cast<const float4*>(p + i + 4);
  out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}

__device__ __forceinline__ void store8_f32_cached(float* p, int64_t i, const float (&x)[8]) {
  *reinterpret_cast<float4*>(p + i) = make_float4(x[0], x[1], x[2], x[3]);
  *reinterpret_cast<float4*>(p + i + 4) = make_float4(x[4], x[5], x[6], x[7]);
}

// sign(x) as numpy/MLX define it: -1, 0 or +1 (NaN propagates).
__device__ __forceinline__ float signf(float x) {
  return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : x * 0.0f);
}

__device__ __forceinline__ float clampf(float x, float lo, float hi) {
  return fminf(fmaxf(x, lo), hi);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
// Whether the byte ranges [a, a + na) and [b, b + nb) share a byte.
inline bool overlap(const void* a, int64_t na, const void* b, int64_t nb) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + static_cast<uintptr_t>(nb) && y < x + static_cast<uintptr_t>(na);
}

// f(integral_constant<int, I>) for I = B .. E-1, unrolled by the front end.
template <int B, int E>
struct StaticFor {
  template <typename F>
  __device__ __forceinline__ static void run(F& f) {
    if constexpr (B < E) {
      f(std::integral_constant<int, B>{});
      StaticFor<B + 1, E>::run(f);
    }
  }
};

}  // namespace mr
