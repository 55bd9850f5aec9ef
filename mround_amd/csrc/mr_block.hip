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


// ---- vectorized forms (16-byte loads, rows held in registers) ---------------
// Used when every row starts 16-byte aligned and H is a multiple of 4: a
// thread owns float4 columns tid, tid + kBlock, ... of its row (NV of them),
// so each row is read from HBM once.

__device__ __forceinline__ uint2 pack4_bf16(float a, float b, float c, float d) {
  return make_uint2(pack_bf16x2(a, b),
                    pack_bf16x2(c, d));
}

template <int NV>
__global__ __launch_bounds__(kBlock) void rmsnorm_fwd_v(const float* __restrict__ h,
                                                        const float* __restrict__ w, int64_t H,
                                                        float eps, uint16_t* __restrict__ y,
                                                        float* __restrict__ rstd) {
  __shared__ float smem[kBlock / 64];
  const int64_t row = blockIdx.x;
  const int n4 = static_cast<int>(H / 4);
  const float4* hr = reinterpret_cast<const float4*>(h + row * H);
  float4 v[NV];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = threadIdx.x + k * kBlock;
    v[k] = i < n4 ? hr[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    ss += v[k].x * v[k].x + v[k].y * v[k].y + v[k].z * v[k].z + v[k].w * v[k].w;
  }
  ss = block_sum_f32(ss, smem);
  const float r = rsqrtf(ss / static_cast<float>(H) + eps);
  if (threadIdx.x == 0 && rstd) rstd[row] = r;
  const float4* w4 = reinterpret_cast<const float4*>(w);
  uint2* yr = reinterpret_cast<uint2*>(y + row * H);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = threadIdx.x + k * kBlock;
    if (i < n4) {
      const float4 g = w4[i];
      yr[i] = pack4_bf16(v[k].x * r * g.x, v[k].y * r * g.y, v[k].z * r * g.z, v[k].w * r * g.w);
    }
  }
}

template <int NV>
__global__ __launch_bounds__(kBlock) void rmsnorm_bwd_v(const float* __restrict__ dy,
                                                        const float* __restrict__ h,
                                                        const float* __restrict__ w,
                                                        const float* __restrict__ rstd,
                                                        const float* __restrict__ dres, int64_t H,
                                                        uint16_t* __restrict__ dh_bf16,
                                                        float* __restrict__ dh_f32) {
  __shared__ float smem[kBlock / 64];
  const int64_t row = blockIdx.x;
  const int n4 = static_cast<int>(H / 4);
  const float4* dyr = reinterpret_cast<const float4*>(dy + row * H);
  const float4* hr = reinterpret_cast<const float4*>(h + row * H);
  const float4* w4 = reinterpret_cast<const float4*>(w);
  const float4* qr = dres ? reinterpret_cast<const float4*>(dres + row * H) : nullptr;
  const float r = rstd[row];
  float4 gy[NV], hv[NV], rq[NV];
  // Every load of the row is issued before any is used (indices clamped into
  // the row, the excess lanes' values zeroed afterwards): predicated loads
  // made the compiler wait for each column group's loads before issuing the
  // next group's. The residual gradient comes with them, ahead of the
  // reduction.
  float4 dv[NV], wv[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = min(static_cast<int>(threadIdx.x) + k * kBlock, n4 - 1);
    hv[k] = hr[i];
    dv[k] = dyr[i];
    wv[k] = w4[i];
  }
  const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (qr) {
#pragma unroll
    for (int k = 0; k < NV; ++k) rq[k] = qr[min(static_cast<int>(threadIdx.x) + k * kBlock, n4 - 1)];
  } else {
#pragma unroll
    for (int k = 0; k < NV; ++k) rq[k] = z;
  }
  float dot = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const bool in = static_cast<int>(threadIdx.x) + k * kBlock < n4;
    if (!in) hv[k] = z;
    const float4 d = in ? dv[k] : z;
    gy[k] = make_float4(d.x * wv[k].x, d.y * wv[k].y, d.z * wv[k].z, d.w * wv[k].w);  // dy w
    dot += gy[k].x * hv[k].x + gy[k].y * hv[k].y + gy[k].z * hv[k].z + gy[k].w * hv[k].w;
  }
  dot = block_sum_f32(dot, smem);
  const float c = r * r * r * dot / static_cast<float>(H);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = threadIdx.x + k * kBlock;
    if (i >= n4) continue;
    float4 g = make_float4(r * gy[k].x - c * hv[k].x, r * gy[k].y - c * hv[k].y,
                           r * gy[k].z - c * hv[k].z, r * gy[k].w - c * hv[k].w);
    g.x += rq[k].x; g.y += rq[k].y; g.z += rq[k].z; g.w += rq[k].w;  // zero without dres
    if (dh_bf16) reinterpret_cast<uint2*>(dh_bf16 + row * H)[i] = pack4_bf16(g.x, g.y, g.z, g.w);
    if (dh_f32) reinterpret_cast<float4*>(dh_f32 + row * H)[i] = g;
  }
}

// Rotary embedding, 8 pairs per thread: 16-byte loads of x_i.. and
// x_{i+d/2}.., 64 bytes of the cos/sin table. Needs d % 16 == 0 and 16-byte
// aligned rows.
template <bool BWD>
__global__ __launch_bounds__(kBlock) void rope_v(uint16_t* __restrict__ x, int64_t ld, int64_t T,
                                                 int S, int n_heads, int d,
                                                 const float* __restrict__ cs) {
  const int half = d / 2, groups = half / 8;
  const int64_t total = T * n_heads * groups;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (idx >= total) return;
  const int gi = static_cast<int>(idx % groups);
  const int64_t th = idx / groups;
  const int hd = static_cast<int>(th % n_heads);
  const int64_t t = th / n_heads;
  const int pos = static_cast<int>(t % S);
  uint16_t* p = x + t * ld + static_cast<int64_t>(hd) * d + gi * 8;
  const uint4 av = *reinterpret_cast<const uint4*>(p);
  const uint4 bv = *reinterpret_cast<const uint4*>(p + half);
  const float4* c4 = reinterpret_cast<const float4*>(cs + (static_cast<int64_t>(pos) * half + gi * 8) * 2);
  const uint32_t aw[4] = {av.x, av.y, av.z, av.w}, bw[4] = {bv.x, bv.y, bv.z, bv.w};
  uint32_t ow_a[4], ow_b[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {  // pairs 2k, 2k + 1
    const float4 t4 = c4[k];      // cos, sin of pair 2k; cos, sin of pair 2k + 1
    const float a0 = __uint_as_float(aw[k] << 16), a1 = __uint_as_float(aw[k] & 0xffff0000u);
    const float b0 = __uint_as_float(bw[k] << 16), b1 = __uint_as_float(bw[k] & 0xffff0000u);
    float ya0, yb0, ya1, yb1;
    if constexpr (BWD) {
      ya0 = a0 * t4.x + b0 * t4.y; yb0 = b0 * t4.x - a0 * t4.y;
      ya1 = a1 * t4.z + b1 * t4.w; yb1 = b1 * t4.z - a1 * t4.w;
    } else {
      ya0 = a0 * t4.x - b0 * t4.y; yb0 = b0 * t4.x + a0 * t4.y;
      ya1 = a1 * t4.z - b1 * t4.w; yb1 = b1 * t4.z + a1 * t4.w;
    }
    ow_a[k] = pack_bf16x2(ya0, ya1);
    ow_b[k] = pack_bf16x2(yb0, yb1);
  }
  *reinterpret_cast<uint4*>(p) = make_uint4(ow_a[0], ow_a[1], ow_a[2], ow_a[3]);
  *reinterpret_cast<uint4*>(p + half) = make_uint4(ow_b[0], ow_b[1], ow_b[2], ow_b[3]);
}

__global__ __launch_bounds__(kBlock) void cast_v(const float4* __restrict__ x, uint2* __restrict__ y,
                                                 int64_t n4) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n4; i += stride) {
    const float4 v = x[i];
    y[i] = pack4_bf16(v.x, v.y, v.z, v.w);
  }
}

// ---- Split-precision operands -----------------------------------------------
//
// An fp32 value y is carried as two bfloat16 halves: hi = bf16(y) and
// lo = bf16(y - hi) (y - hi is exact in fp32), so hi + lo holds y to about 16
// significant bits. A product A B^T then runs as one bf16 GEMM over K' = 3K
// with A' = [A_hi | A_hi | A_lo] and B' = [B_hi | B_lo | B_hi] along K: the
// three products A_hi B_hi + A_hi B_lo + A_lo B_hi, the low-by-low term left
// out. Rows of activation operands are written in the first order, rows of
// weights in the second.
__device__ __forceinline__ float bf16_round(float x) { return bf16_to_f32(f32_to_bf16(x)); }

__device__ __forceinline__ uint2 pack4_bf16_lo(float a, float b, float c, float d) {
  return pack4_bf16(a - bf16_round(a), b - bf16_round(b), c - bf16_round(c), d - bf16_round(d));
}

// Three 8-byte pieces of one split row: segment s of SEGS at column group i
// (n4 groups of 4 per segment).
__device__ __forceinline__ void store_split4(uint2* row, int64_t n4, int64_t i, float a, float b, float c,
                                             float d, bool weight_order) {
  const uint2 hi = pack4_bf16(a, b, c, d);
  const uint2 lo = pack4_bf16_lo(a, b, c, d);
  row[i] = hi;
  row[n4 + i] = weight_order ? lo : hi;
  row[2 * n4 + i] = weight_order ? hi : lo;
}

// RMSNorm forward whose output is also written split, [hi | hi | lo] per row
// of 3H (and hi alone into y when given).
template <int NV>
__global__ __launch_bounds__(kBlock) void rmsnorm_fwd_split_v(const float* __restrict__ h,
                                                              const float* __restrict__ w, int64_t H,
                                                              float eps, uint16_t* __restrict__ ys,
                                                              uint16_t* __restrict__ y,
                                                              float* __restrict__ rstd) {
  __shared__ float smem[kBlock / 64];
  const int64_t row = blockIdx.x;
  const int n4 = static_cast<int>(H / 4);
  const float4* hr = reinterpret_cast<const float4*>(h + row * H);
  float4 v[NV];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = threadIdx.x + k * kBlock;
    v[k] = i < n4 ? hr[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    ss += v[k].x * v[k].x + v[k].y * v[k].y + v[k].z * v[k].z + v[k].w * v[k].w;
  }
  ss = block_sum_f32(ss, smem);
  const float r = rsqrtf(ss / static_cast<float>(H) + eps);
  if (threadIdx.x == 0 && rstd) rstd[row] = r;
  const float4* w4 = reinterpret_cast<const float4*>(w);
  uint2* ysr = reinterpret_cast<uint2*>(ys + row * 3 * H);
  uint2* yr = y ? reinterpret_cast<uint2*>(y + row * H) : nullptr;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = threadIdx.x + k * kBlock;
    if (i < n4) {
      const float4 g = w4[i];
      const float a = v[k].x * r * g.x, b = v[k].y * r * g.y, c = v[k].z * r * g.z, d = v[k].w * r * g.w;
      store_split4(ysr, n4, i, a, b, c, d, false);
      if (yr) yr[i] = pack4_bf16(a, b, c, d);
    }
  }
}

// fp32 rows -> split rows (activation or weight order), hi alone into plain
// when given. One block per row.
__global__ __launch_bounds__(kBlock) void split_rows(const float* __restrict__ src, int64_t ld_src,
                                                     int64_t n4, bool weight_order, uint16_t* __restrict__ dst,
                                                     int64_t ld_dst, uint16_t* __restrict__ plain,
                                                     int64_t ld_plain) {
  const int64_t row = blockIdx.x;
  const float4* sr = reinterpret_cast<const float4*>(src + row * ld_src);
  uint2* dr = reinterpret_cast<uint2*>(dst + row * ld_dst);
  uint2* pr = plain ? reinterpret_cast<uint2*>(plain + row * ld_plain) : nullptr;
  for (int64_t i = threadIdx.x; i < n4; i += kBlock) {
    const float4 x = sr[i];
    store_split4(dr, n4, i, x.x, x.y, x.z, x.w, weight_order);
    if (pr) pr[i] = pack4_bf16(x.x, x.y, x.z, x.w);
  }
}

// act = silu(g) * u from fp32 gate/up rows interleaved every 32 columns
// (columns 64 b .. 64 b + 31 gate, the next 32 up, for act columns
// 32 b .. 32 b + 31), written split [hi | hi | lo] per row of 3N, hi alone
// into act, and the gate/up values in bf16 for the backward. One block per row.
__global__ __launch_bounds__(kBlock) void swiglu_split_rows(const float* __restrict__ gu32, int64_t N,
                                                            uint16_t* __restrict__ act_split,
                                                            uint16_t* __restrict__ act,
                                                            uint16_t* __restrict__ gu) {
  const int64_t row = blockIdx.x;
  const int64_t n4 = N / 4;
  const float4* src = reinterpret_cast<const float4*>(gu32 + row * 2 * N);
  uint2* sr = reinterpret_cast<uint2*>(act_split + row * 3 * N);
  uint2* ar = reinterpret_cast<uint2*>(act + row * N);
  uint2* gr = reinterpret_cast<uint2*>(gu + row * 2 * N);
  for (int64_t i = threadIdx.x; i < n4; i += kBlock) {
    // act columns 4 i .. 4 i + 3 lie in interleave block b = 4 i / 32
    const int64_t b = i >> 3, j4 = i & 7;
    const int64_t gi = b * 16 + j4, ui = gi + 8;  // float4 indices of the gate and up values
    const float4 g = src[gi], u = src[ui];
    const float a = silu(g.x) * u.x, bb = silu(g.y) * u.y, c = silu(g.z) * u.z, d = silu(g.w) * u.w;
    store_split4(sr, n4, i, a, bb, c, d, false);
    ar[i] = pack4_bf16(a, bb, c, d);
    gr[gi] = pack4_bf16(g.x, g.y, g.z, g.w);
    gr[ui] = pack4_bf16(u.x, u.y, u.z, u.w);
  }
}

// Split precision for the attention: fp32 q/k/v rows (the split q/k/v
// product's output) rotated in fp32 (the rotary embedding over the first
// n_rope heads, q then k, as rope_kernel; the v heads pass through) and
// written as bf16 hi and lo halves. One block per token row; thread i takes
// pair i of each head (columns i and i + d/2).
__global__ __launch_bounds__(kBlock) void rope_split_rows(const float* __restrict__ x, int64_t ldx, int S,
                                                          int n_rope, int n_heads, int d,
                                                          const float* __restrict__ cs, uint16_t* __restrict__ hi,
                                                          uint16_t* __restrict__ lo, int64_t ld) {
  const int64_t t = blockIdx.x;
  const int half = d / 2;
  const int pos = static_cast<int>(t % S);
  const float* xr = x + t * ldx;
  uint16_t* hr = hi + t * ld;
  uint16_t* lr = lo + t * ld;
  for (int p = threadIdx.x; p < n_heads * half; p += kBlock) {
    const int hd = p / half, i = p % half;
    const int64_t ca = static_cast<int64_t>(hd) * d + i, cb = ca + half;
    float ya = xr[ca], yb = xr[cb];
    if (hd < n_rope) {
      const float c = cs[(static_cast<int64_t>(pos) * half + i) * 2];
      const float sn = cs[(static_cast<int64_t>(pos) * half + i) * 2 + 1];
      const float a = ya, b = yb;
      ya = a * c - b * sn;
      yb = b * c + a * sn;
    }
    const uint16_t ha = f32_to_bf16(ya), hb = f32_to_bf16(yb);
    hr[ca] = ha;
    hr[cb] = hb;
    lr[ca] = f32_to_bf16(ya - bf16_to_f32(ha));
    lr[cb] = f32_to_bf16(yb - bf16_to_f32(hb));
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool al8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// float4 columns per thread for a row of H floats, or 0 when H is too wide.
int row_nv(int64_t H) {
  const int64_t n4 = H / 4;
  for (int nv : {1, 2, 4, 8, 16})
    if (n4 <= static_cast<int64_t>(nv) * kBlock) return nv;
  return 0;
}

}  // namespace
}  // namespace mr

extern "C" {

int mr_cast_f32_bf16(const float* x, void* y, int64_t n, void* stream) {
  using namespace mr;
  clear_error();
  if (n <= 0) return MR_OK;
  if (!x || !y) return fail(MR_EINVAL, "mr_cast_f32_bf16: null pointer");
  if (n % 4 == 0 && al16(x) && (reinterpret_cast<uintptr_t>(y) & 7u) == 0) {
    int64_t blocks = (n / 4 + kBlock - 1) / kBlock;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(cast_v, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), reinterpret_cast<const float4*>(x),
                       static_cast<uint2*>(y), n / 4);
    MR_LAUNCH_CHECK("mr_cast_f32_bf16");
    return MR_OK;
  }
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint16_t* y = static_cast<uint16_t*>(y_bf16);
  const int nv = row_nv(H);
  if (H % 4 == 0 && nv && al16(h) && al16(w) && (reinterpret_cast<uintptr_t>(y) & 7u) == 0) {
    const dim3 g(static_cast<unsigned>(T));
    switch (nv) {
      case 1: hipLaunchKernelGGL(rmsnorm_fwd_v<1>, g, dim3(kBlock), 0, s, h, w, H, eps, y, rstd_out); break;
      case 2: hipLaunchKernelGGL(rmsnorm_fwd_v<2>, g, dim3(kBlock), 0, s, h, w, H, eps, y, rstd_out); break;
      case 4: hipLaunchKernelGGL(rmsnorm_fwd_v<4>, g, dim3(kBlock), 0, s, h, w, H, eps, y, rstd_out); break;
      case 8: hipLaunchKernelGGL(rmsnorm_fwd_v<8>, g, dim3(kBlock), 0, s, h, w, H, eps, y, rstd_out); break;
      default: hipLaunchKernelGGL(rmsnorm_fwd_v<16>, g, dim3(kBlock), 0, s, h, w, H, eps, y, rstd_out); break;
    }
    MR_LAUNCH_CHECK("mr_rmsnorm_fwd");
    return MR_OK;
  }
  hipLaunchKernelGGL(rmsnorm_fwd, dim3(static_cast<unsigned>(T)), dim3(kBlock), 0, s, h, w, H, eps,
                     y, rstd_out);
  MR_LAUNCH_CHECK("mr_rmsnorm_fwd");
  return MR_OK;
}

int mr_rmsnorm_fwd_split(const float* h, const float* w, int64_t T, int64_t H, float eps, void* y_split,
                         void* y_bf16, float* rstd_out, void* stream) {
  using namespace mr;
  clear_error();
  if (T <= 0 || H <= 0) return MR_OK;
  if (!h || !w || !y_split) return fail(MR_EINVAL, "mr_rmsnorm_fwd_split: null pointer");
  if (T > 0x7fffffff) return fail(MR_EINVAL, "mr_rmsnorm_fwd_split: too many rows");
  const int nv = row_nv(H);
  if (H % 4 || !nv || !al16(h) || !al16(w) || !al8(y_split) || (y_bf16 && !al8(y_bf16)))
    return fail(MR_EINVAL, "mr_rmsnorm_fwd_split: the width must be a multiple of 4 up to %d, h and w "
                "16-byte aligned, the outputs 8-byte aligned", 16 * kBlock * 4);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint16_t* ys = static_cast<uint16_t*>(y_split);
  uint16_t* y = static_cast<uint16_t*>(y_bf16);
  const dim3 g(static_cast<unsigned>(T));
  switch (nv) {
    case 1: hipLaunchKernelGGL(rmsnorm_fwd_split_v<1>, g, dim3(kBlock), 0, s, h, w, H, eps, ys, y, rstd_out); break;
    case 2: hipLaunchKernelGGL(rmsnorm_fwd_split_v<2>, g, dim3(kBlock), 0, s, h, w, H, eps, ys, y, rstd_out); break;
    case 4: hipLaunchKernelGGL(rmsnorm_fwd_split_v<4>, g, dim3(kBlock), 0, s, h, w, H, eps, ys, y, rstd_out); break;
    case 8: hipLaunchKernelGGL(rmsnorm_fwd_split_v<8>, g, dim3(kBlock), 0, s, h, w, H, eps, ys, y, rstd_out); break;
    default: hipLaunchKernelGGL(rmsnorm_fwd_split_v<16>, g, dim3(kBlock), 0, s, h, w, H, eps, ys, y, rstd_out); break;
  }
  MR_LAUNCH_CHECK("mr_rmsnorm_fwd_split");
  return MR_OK;
}

int mr_split_bf16(const float* src, int64_t ld_src, int64_t rows, int64_t cols, int order, void* dst,
                  int64_t ld_dst, void* plain, int64_t ld_plain, void* stream) {
  using namespace mr;
  clear_error();
  if (rows <= 0 || cols <= 0) return MR_OK;
  if (!src || !dst) return fail(MR_EINVAL, "mr_split_bf16: null pointer");
  if (order != 0 && order != 1) return fail(MR_EINVAL, "mr_split_bf16: order must be 0 or 1, got %d", order);
  if (rows > 0x7fffffff) return fail(MR_EINVAL, "mr_split_bf16: too many rows");
  if (cols % 4 || ld_src < cols || ld_src % 4 || ld_dst < 3 * cols || ld_dst % 4 ||
      (plain && (ld_plain < cols || ld_plain % 4)))
    return fail(MR_EINVAL, "mr_split_bf16: cols and every leading dimension must be multiples of 4, "
                "ld_src >= cols, ld_dst >= 3 cols, ld_plain >= cols");
  if (!al16(src) || !al8(dst) || (plain && !al8(plain)))
    return fail(MR_EINVAL, "mr_split_bf16: src must be 16-byte and the outputs 8-byte aligned");
  hipLaunchKernelGGL(split_rows, dim3(static_cast<unsigned>(rows)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), src, ld_src, cols / 4, order == 1,
                     static_cast<uint16_t*>(dst), ld_dst, static_cast<uint16_t*>(plain), ld_plain);
  MR_LAUNCH_CHECK("mr_split_bf16");
  return MR_OK;
}

int mr_swiglu_split(const float* gu32, int64_t T, int64_t N, void* act_split, void* act, void* gu,
                    void* stream) {
  using namespace mr;
  clear_error();
  if (T <= 0 || N <= 0) return MR_OK;
  if (!gu32 || !act_split || !act || !gu) return fail(MR_EINVAL, "mr_swiglu_split: null pointer");
  if (T > 0x7fffffff) return fail(MR_EINVAL, "mr_swiglu_split: too many rows");
  if (N % 32) return fail(MR_EINVAL, "mr_swiglu_split: N must be a multiple of 32 (the gate/up interleave)");
  if (!al16(gu32) || !al8(act_split) || !al8(act) || !al8(gu))
    return fail(MR_EINVAL, "mr_swiglu_split: gu32 must be 16-byte and the outputs 8-byte aligned");
  hipLaunchKernelGGL(swiglu_split_rows, dim3(static_cast<unsigned>(T)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), gu32, N, static_cast<uint16_t*>(act_split),
                     static_cast<uint16_t*>(act), static_cast<uint16_t*>(gu));
  MR_LAUNCH_CHECK("mr_swiglu_split");
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint16_t* db = static_cast<uint16_t*>(dh_bf16);
  const int nv = row_nv(H);
  if (H % 4 == 0 && nv && al16(dy) && al16(h) && al16(w) && (!dres || al16(dres)) &&
      (!dh_f32 || al16(dh_f32)) && (reinterpret_cast<uintptr_t>(db) & 7u) == 0) {
    const dim3 g(static_cast<unsigned>(T));
    switch (nv) {
      case 1: hipLaunchKernelGGL(rmsnorm_bwd_v<1>, g, dim3(kBlock), 0, s, dy, h, w, rstd, dres, H, db, dh_f32); break;
      case 2: hipLaunchKernelGGL(rmsnorm_bwd_v<2>, g, dim3(kBlock), 0, s, dy, h, w, rstd, dres, H, db, dh_f32); break;
      case 4: hipLaunchKernelGGL(rmsnorm_bwd_v<4>, g, dim3(kBlock), 0, s, dy, h, w, rstd, dres, H, db, dh_f32); break;
      case 8: hipLaunchKernelGGL(rmsnorm_bwd_v<8>, g, dim3(kBlock), 0, s, dy, h, w, rstd, dres, H, db, dh_f32); break;
      default: hipLaunchKernelGGL(rmsnorm_bwd_v<16>, g, dim3(kBlock), 0, s, dy, h, w, rstd, dres, H, db, dh_f32); break;
    }
    MR_LAUNCH_CHECK("mr_rmsnorm_bwd");
    return MR_OK;
  }
  hipLaunchKernelGGL(rmsnorm_bwd, dim3(static_cast<unsigned>(T)), dim3(kBlock), 0, s, dy, h, w,
                     rstd, dres, H, db, dh_f32);
  MR_LAUNCH_CHECK("mr_rmsnorm_bwd");
  return MR_OK;
}

int mr_rope_split(const float* x, int64_t ldx, int64_t T, int S, int n_rope_heads, int n_heads, int head_dim,
                  const float* cos_sin, void* hi, void* lo, int64_t ld, void* stream) {
  using namespace mr;
  clear_error();
  if (T <= 0 || n_heads <= 0) return MR_OK;
  if (!x || !cos_sin || !hi || !lo) return fail(MR_EINVAL, "mr_rope_split: null pointer");
  if (head_dim <= 0 || head_dim % 2 || S <= 0 || n_rope_heads < 0 || n_rope_heads > n_heads ||
      ldx < static_cast<int64_t>(n_heads) * head_dim || ld < static_cast<int64_t>(n_heads) * head_dim)
    return fail(MR_EINVAL, "mr_rope_split: bad shape");
  if (T > 0x7fffffff) return fail(MR_EINVAL, "mr_rope_split: too many rows");
  hipLaunchKernelGGL(rope_split_rows, dim3(static_cast<unsigned>(T)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), x, ldx, S, n_rope_heads, n_heads, head_dim, cos_sin,
                     static_cast<uint16_t*>(hi), static_cast<uint16_t*>(lo), ld);
  MR_LAUNCH_CHECK("mr_rope_split");
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint16_t* x = static_cast<uint16_t*>(x_bf16);
  if (head_dim % 16 == 0 && ld % 8 == 0 && al16(x) && al16(cos_sin)) {
    const int64_t total_v = T * n_heads * (head_dim / 16);
    const int64_t blocks_v = (total_v + kBlock - 1) / kBlock;
    if (blocks_v > 0x7fffffff) return fail(MR_EINVAL, "mr_rope: too large");
    if (backward)
      hipLaunchKernelGGL(rope_v<true>, dim3(static_cast<unsigned>(blocks_v)), dim3(kBlock), 0, s, x,
                         ld, T, S, n_heads, head_dim, cos_sin);
    else
      hipLaunchKernelGGL(rope_v<false>, dim3(static_cast<unsigned>(blocks_v)), dim3(kBlock), 0, s, x,
                         ld, T, S, n_heads, head_dim, cos_sin);
    MR_LAUNCH_CHECK("mr_rope");
    return MR_OK;
  }
  const int64_t total = T * n_heads * (head_dim / 2);
  const int64_t blocks = (total + kBlock - 1) / kBlock;
  if (blocks > 0x7fffffff) return fail(MR_EINVAL, "mr_rope: too large");
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
