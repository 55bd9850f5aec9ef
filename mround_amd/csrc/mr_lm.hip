// Language-model ends of the whole-model scoring pass, for gfx950: the
// embedding lookup that starts the residual stream and the causal-LM
// cross-entropy that ends it.
//
// The reference scores layers with the gradient of the mean shifted
// cross-entropy of the whole model (mround/pipeline/scoring.py:183-192):
// logits = model(tokens[:, :-1]) cast to fp32, loss = mean over positions of
// logsumexp(logits) - logits[label]. Its gradient with respect to the logits
// is (softmax - onehot(label)) / n, which is what the cross-entropy kernel
// writes, as the bf16 operand of the head's input-gradient GEMM.
//
// Logits are bf16 (the model-dtype matmul output the reference casts up); every
// reduction over a row runs in fp32, the loss in fp64 across rows.
#include "mr_common.h"

namespace mr {
namespace {

constexpr int kCeBlock = 512;
constexpr int kCeWaves = kCeBlock / 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// (max, sum of exp(x - max)) pairs, merged; an empty pair has s == 0.
struct MaxSum {
  float m, s;
};

__device__ __forceinline__ MaxSum merge(MaxSum a, MaxSum b) {
  if (a.s == 0.0f) return b;
  if (b.s == 0.0f) return a;
  const float m = fmaxf(a.m, b.m);
  return {m, a.s * exp2f((a.m - m) * kLog2e) + b.s * exp2f((b.m - m) * kLog2e)};
}

// Adds n values held in x[] to the running pair with one rescale.
template <int N>
__device__ __forceinline__ MaxSum absorb(MaxSum acc, const float (&x)[N]) {
  float mx = x[0];
#pragma unroll
  for (int k = 1; k < N; ++k) mx = fmaxf(mx, x[k]);
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < N; ++k) s += exp2f((x[k] - mx) * kLog2e);
  return merge(acc, MaxSum{mx, s});
}

__device__ __forceinline__ void unpack8(uint4 r, float (&x)[8]) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    x[2 * k] = __uint_as_float(w[k] << 16);
    x[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
  }
}

// One workgroup per row. Pass 1 reads the row once for (max, sum); pass 2
// reads it again and writes the gradient. dlogits may be the logits buffer:
// every element is read and then written by the same thread, after the
// barrier that ends pass 1.
template <bool VEC>
__global__ __launch_bounds__(kCeBlock) void ce_rows(const uint16_t* logits, int64_t ld, int64_t V,
                                                    const int32_t* __restrict__ labels, float scale,
                                                    float* __restrict__ row_loss, uint16_t* dlogits,
                                                    int64_t ldd) {
  __shared__ float sm[kCeWaves], ss[kCeWaves];
  const int64_t row = blockIdx.x;
  const uint16_t* x = logits + row * ld;
  const int label = labels[row];
  MaxSum acc{0.0f, 0.0f};
  if constexpr (VEC) {
    const int64_t n8 = V / 8;
    const uint4* x8 = reinterpret_cast<const uint4*>(x);
    int64_t i = threadIdx.x;
    // Two 16-byte loads in flight per thread per step.
    for (; i + kCeBlock < n8; i += 2 * kCeBlock) {
      const uint4 a = x8[i], b = x8[i + kCeBlock];
      float v[16];
      float lo[8], hi[8];
      unpack8(a, lo);
      unpack8(b, hi);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        v[k] = lo[k];
        v[8 + k] = hi[k];
      }
      acc = absorb<16>(acc, v);
    }
    if (i < n8) {
      float v[8];
      unpack8(x8[i], v);
      acc = absorb<8>(acc, v);
    }
  } else {
    for (int64_t i = threadIdx.x; i < V; i += kCeBlock) {
      const float v[1] = {bf16_to_f32(x[i])};
      acc = absorb<1>(acc, v);
    }
  }
  // The label's logit is read before the barrier: after it, pass 2 may
  // overwrite the row in place.
  const bool ignored = label < 0;
  const bool bad = label >= V;
  float x_label = 0.0f;
  if (threadIdx.x == 0 && !ignored && !bad) x_label = bf16_to_f32(x[label]);
  // Block merge: waves by shuffles, then the eight wave results.
  for (int off = 32; off > 0; off >>= 1) {
    MaxSum o{__shfl_xor(acc.m, off, 64), __shfl_xor(acc.s, off, 64)};
    acc = merge(acc, o);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sm[wave] = acc.m;
    ss[wave] = acc.s;
  }
  __syncthreads();
  MaxSum t{sm[0], ss[0]};
#pragma unroll
  for (int w = 1; w < kCeWaves; ++w) t = merge(t, MaxSum{sm[w], ss[w]});
  const float m = t.m, inv_s = 1.0f / t.s;
  if (threadIdx.x == 0) {
    float l = 0.0f;
    if (bad) {
      l = __builtin_nanf("");
    } else if (!ignored) {
      l = m + log2f(t.s) * kLn2 - x_label;
    }
    row_loss[row] = l;
  }
  if (!dlogits) return;
  uint16_t* d = dlogits + row * ldd;
  const float g = ignored ? 0.0f : scale * inv_s;
  if constexpr (VEC) {
    const int64_t n8 = V / 8;
    const uint4* x8 = reinterpret_cast<const uint4*>(x);
    uint4* d8 = reinterpret_cast<uint4*>(d);
    for (int64_t i = threadIdx.x; i < n8; i += kCeBlock) {
      float v[8];
      unpack8(x8[i], v);
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float p0 = exp2f((v[2 * k] - m) * kLog2e) * g;
        float p1 = exp2f((v[2 * k + 1] - m) * kLog2e) * g;
        const int64_t j = i * 8 + 2 * k;
        if (!ignored && j == label) p0 -= scale;
        if (!ignored && j + 1 == label) p1 -= scale;
        w[k] = pack_bf16x2(p0, p1);
      }
      d8[i] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  } else {
    for (int64_t i = threadIdx.x; i < V; i += kCeBlock) {
      float p = exp2f((bf16_to_f32(x[i]) - m) * kLog2e) * g;
      if (!ignored && i == label) p -= scale;
      d[i] = f32_to_bf16(p);
    }
  }
}

// loss = scale * sum of the row losses, in a fixed order (fp64 partials).
__global__ __launch_bounds__(1024) void ce_finalize(const float* __restrict__ row_loss, int64_t T,
                                                    float scale, float* __restrict__ loss_out) {
  __shared__ double sm[16];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < T; i += 1024) acc += static_cast<double>(row_loss[i]);
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < 16; ++w) t += sm[w];
    loss_out[0] = static_cast<float>(t * static_cast<double>(scale));
  }
}

constexpr int kEmbBlock = 256;

// out[t, :] = table[ids[t], :] widened to fp32; an id outside [0, V) gives a
// row of NaN so that a bad token cannot pass unnoticed.
template <int DT, bool VEC>
__global__ __launch_bounds__(kEmbBlock) void embed_rows(const void* __restrict__ table, int64_t ldt,
                                                        int64_t V, int64_t H,
                                                        const int32_t* __restrict__ ids,
                                                        float* __restrict__ out, int64_t ldo) {
  const int64_t t = blockIdx.x;
  const int id = ids[t];
  float* o = out + t * ldo;
  const bool bad = id < 0 || id >= V;
  if constexpr (VEC) {
    const int64_t n8 = H / 8;
    for (int64_t i = threadIdx.x; i < n8; i += kEmbBlock) {
      float v[8];
      if (bad) {
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = __builtin_nanf("");
      } else {
        load8<DT>(table, static_cast<int64_t>(id) * ldt + i * 8, v);
      }
      float4* o4 = reinterpret_cast<float4*>(o + i * 8);
      o4[0] = make_float4(v[0], v[1], v[2], v[3]);
      o4[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
  } else {
    for (int64_t i = threadIdx.x; i < H; i += kEmbBlock)
      o[i] = bad ? __builtin_nanf("") : load_elem<DT>(table, static_cast<int64_t>(id) * ldt + i);
  }
}

}  // namespace
}  // namespace mr

extern "C" {

int mr_cross_entropy(const void* logits, int64_t ld, int64_t T, int64_t V, const int32_t* labels,
                     float scale, float* row_loss, float* loss_out, void* dlogits, int64_t ldd,
                     void* stream) {
  using namespace mr;
  clear_error();
  if (T < 0 || V <= 0) return fail(MR_EINVAL, "mr_cross_entropy: bad sizes T=%lld V=%lld",
                                   static_cast<long long>(T), static_cast<long long>(V));
  if (!logits || !labels || !row_loss) return fail(MR_EINVAL, "mr_cross_entropy: null pointer");
  if (ld < V || (dlogits && ldd < V))
    return fail(MR_EINVAL, "mr_cross_entropy: a leading dimension is smaller than V");
  if (T > 0x7fffffff) return fail(MR_EINVAL, "mr_cross_entropy: too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (T > 0) {
    const uint16_t* x = static_cast<const uint16_t*>(logits);
    uint16_t* d = static_cast<uint16_t*>(dlogits);
    const bool vec = V % 8 == 0 && ld % 8 == 0 && aligned16(x) &&
                     (!d || (ldd % 8 == 0 && aligned16(d)));
    if (vec)
      hipLaunchKernelGGL(ce_rows<true>, dim3(static_cast<unsigned>(T)), dim3(kCeBlock), 0, s, x, ld,
                         V, labels, scale, row_loss, d, ldd);
    else
      hipLaunchKernelGGL(ce_rows<false>, dim3(static_cast<unsigned>(T)), dim3(kCeBlock), 0, s, x,
                         ld, V, labels, scale, row_loss, d, ldd);
    MR_LAUNCH_CHECK("mr_cross_entropy");
  }
  if (loss_out) {
    hipLaunchKernelGGL(ce_finalize, dim3(1), dim3(1024), 0, s, row_loss, T, scale, loss_out);
    MR_LAUNCH_CHECK("mr_cross_entropy");
  }
  return MR_OK;
}

int mr_embed_rows(const void* table, int dtype, int64_t V, int64_t H, int64_t ldt,
                  const int32_t* ids, int64_t T, float* out, int64_t ldo, void* stream) {
  using namespace mr;
  clear_error();
  if (T < 0 || V <= 0 || H <= 0) return fail(MR_EINVAL, "mr_embed_rows: bad sizes");
  if (T == 0) return MR_OK;
  if (!table || !ids || !out) return fail(MR_EINVAL, "mr_embed_rows: null pointer");
  if (!valid_dtype(dtype)) return fail(MR_EINVAL, "mr_embed_rows: bad table dtype %d", dtype);
  if (ldt < H || ldo < H) return fail(MR_EINVAL, "mr_embed_rows: a leading dimension is smaller than H");
  if (T > 0x7fffffff) return fail(MR_EINVAL, "mr_embed_rows: too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = H % 8 == 0 && ldt % 8 == 0 && ldo % 4 == 0 && aligned16(table) && aligned16(out);
  const dim3 g(static_cast<unsigned>(T)), b(kEmbBlock);
#define MR_EMB(DT)                                                                          \
  if (vec)                                                                                  \
    hipLaunchKernelGGL((embed_rows<DT, true>), g, b, 0, s, table, ldt, V, H, ids, out, ldo); \
  else                                                                                      \
    hipLaunchKernelGGL((embed_rows<DT, false>), g, b, 0, s, table, ldt, V, H, ids, out, ldo);
  if (dtype == MR_BF16) {
    MR_EMB(MR_BF16)
  } else if (dtype == MR_F16) {
    MR_EMB(MR_F16)
  } else {
    MR_EMB(MR_F32)
  }
#undef MR_EMB
  MR_LAUNCH_CHECK("mr_embed_rows");
  return MR_OK;
}

}  // extern "C"
