// Causal grouped-query attention, forward and backward, on gfx950 MFMA.
//
// Replaces the scaled-dot-product attention of the mlx-lm block the reference
// differentiates through (mround/pipeline/blocks.py:605; its backward is MLX
// autodiff at mround/pipeline/runner.py:920). Inputs are the packed bf16 qkv
// rows of the block ([T, (Hq + 2 Hkv) d], token t = b S + s, q heads, then k
// heads, then v heads); query head h reads kv head h / (Hq / Hkv); key j is
// visible to query i iff j <= i; softmax in fp32 on scores scaled by 1/sqrt(d).
//
// Layout trick: each MFMA v_mfma_f32_32x32x16_bf16 leaves a 32 x 32 tile with
// one column per lane. Computing S^T = K Q^T puts one query per lane, so the
// softmax row reductions are in-register (plus one swap of lane halves), and
// the probability registers are already the B operand of O^T += V^T P^T once
// the 16 keys of each MFMA step are taken in the order the accumulator holds
// them (any permutation of a reduction index, applied to both operands,
// leaves the product unchanged). The backward uses the same trick in both
// orientations. All sums are in a fixed order: no atomics, deterministic.
#include <cmath>

#include "mr_common.h"

namespace mr {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int QB = 128;  // queries per block (4 waves x 32)
constexpr int KT = 64;   // keys per LDS tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
}

// 8 fp32 -> bf16x8 operand
__device__ __forceinline__ bf16x8 to_bf16x8(const float* x) {
  uint4 v = make_uint4(pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3]), pack_bf16(x[4], x[5]),
                       pack_bf16(x[6], x[7]));
  return as_bf16x8(v);
}

// ---- LDS tiles --------------------------------------------------------------
// Row-major tile of ROWS rows x D bf16 (K-major for the MFMA: row = m or n,
// D = reduction), 16-byte chunk c of row r at position c ^ (r & 7).
template <int D>
__device__ __forceinline__ int rowtile_off(int r, int c) {
  return r * (D * 2) + ((c ^ (r & 7)) << 4);
}
// Transposed tile: D rows (one per d) x 64 bf16 (128 bytes), chunk c (8
// consecutive rows of the source) of row d at position c ^ (d & 7).
__device__ __forceinline__ int ttile_off(int d, int c) { return d * 128 + ((c ^ (d & 7)) << 4); }

// Rows [r0, r0 + 64) of a [T, ld] bf16 matrix, columns [col, col + D), into a rowtile.
template <int D>
__device__ __forceinline__ void load_rowtile(const uint16_t* src, int64_t ld, int64_t r0, int col,
                                             uint8_t* lds) {
  constexpr int CH = D / 8;
  for (int c = threadIdx.x; c < 64 * CH; c += kThreads) {
    const int r = c / CH, ch = c % CH;
    const uint4 v = *reinterpret_cast<const uint4*>(src + (r0 + r) * ld + col + ch * 8);
    *reinterpret_cast<uint4*>(lds + rowtile_off<D>(r, ch)) = v;
  }
}

// The same 64 x D source block stored transposed (D rows of 64).
template <int D>
__device__ __forceinline__ void load_ttile(const uint16_t* src, int64_t ld, int64_t r0, int col,
                                           uint8_t* lds) {
  constexpr int NB = 8 * (D / 8);  // 8x8 blocks
  for (int b = threadIdx.x; b < NB; b += kThreads) {
    const int kb = b & 7;   // 8-row block of the source (one transposed chunk)
    const int db = b >> 3;  // 8-column block of the source (8 transposed rows)
    uint4 r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      r[j] = *reinterpret_cast<const uint4*>(src + (r0 + kb * 8 + j) * ld + col + db * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
      const int c = e >> 1;
      uint32_t d[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) d[q] = __builtin_amdgcn_perm((&r[2 * q + 1].x)[c], (&r[2 * q].x)[c], sel);
      *reinterpret_cast<uint4*>(lds + ttile_off(db * 8 + e, kb)) = make_uint4(d[0], d[1], d[2], d[3]);
    }
  }
}

// MFMA operand from a rowtile: row (m or n) `r`, k16 step s, lane half h.
template <int D>
__device__ __forceinline__ bf16x8 frag_row(const uint8_t* lds, int r, int s, int h) {
  return *reinterpret_cast<const bf16x8*>(lds + rowtile_off<D>(r, 2 * s + h));
}
// MFMA operand from a transposed tile for k16 step s (within the 64-row
// source block) in accumulator key order: source rows 16s + 4h + {0..3} and
// 16s + 8 + 4h + {0..3}.
__device__ __forceinline__ bf16x8 frag_t(const uint8_t* lds, int d, int s, int h) {
  const uint2 lo = *reinterpret_cast<const uint2*>(lds + ttile_off(d, 2 * s) + h * 8);
  const uint2 hi = *reinterpret_cast<const uint2*>(lds + ttile_off(d, 2 * s + 1) + h * 8);
  return as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
}

// Accumulator register r of a 32x32 tile, lane half h: row within the tile.
__device__ __forceinline__ int acc_row(int r, int h) { return (r >> 2) * 8 + h * 4 + (r & 3); }

// Writes a wave's O^T-layout accumulators (acc[dt][r] = value at d = dt*32 +
// acc_row(r, h), query = lane & 31) as bf16 rows [32 queries][D] through LDS.
template <int D>
__device__ __forceinline__ void store_qrows(const f32x16 (&acc)[D / 32], float mul, uint8_t* lds,
                                           uint16_t* dst, int64_t ld, int64_t row0) {
  const int lane = threadIdx.x & 63, h = lane >> 5, q = lane & 31;
  uint16_t* t = reinterpret_cast<uint16_t*>(lds);  // [32][D]
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) t[q * D + dt * 32 + acc_row(r, h)] = f32_to_bf16(acc[dt][r] * mul);
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  constexpr int CH = D / 8;
  for (int c = lane; c < 32 * CH; c += 64) {
    const int row = c / CH, ch = c % CH;
    *reinterpret_cast<uint4*>(dst + (row0 + row) * ld + ch * 8) =
        *reinterpret_cast<const uint4*>(t + row * D + ch * 8);
  }
}

// ---- forward ----------------------------------------------------------------

template <int D>
__global__ __launch_bounds__(kThreads) void attn_fwd(const uint16_t* __restrict__ qkv, int64_t ld,
                                                     int S, int Hq, int Hkv, float scale_log2,
                                                     uint16_t* __restrict__ out, int64_t ldo,
                                                     float* __restrict__ lse) {
  constexpr int NS = D / 16;
  __shared__ __attribute__((aligned(16))) uint8_t smem[KT * D * 2 * 2];
  uint8_t* Ks = smem;
  uint8_t* Vt = smem + KT * D * 2;
  const int qb = blockIdx.x, hq = blockIdx.y, b = blockIdx.z;
  const int g = hq / (Hq / Hkv);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
  const int q0 = qb * QB + wave * 32;
  const int qi = q0 + l32;
  const int64_t tok0 = static_cast<int64_t>(b) * S;
  const int kcol = (Hq + g) * D, vcol = (Hq + Hkv + g) * D;

  bf16x8 qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s)
    qf[s] = *reinterpret_cast<const bf16x8*>(qkv + (tok0 + qi) * ld + hq * D + s * 16 + h * 8);

  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) o[dt] = f32x16{};
  float m = -INFINITY, l = 0.0f;

  const int kv_end = min(S, qb * QB + QB);
  for (int kv0 = 0; kv0 < kv_end; kv0 += KT) {
    __syncthreads();
    load_rowtile<D>(qkv, ld, tok0 + kv0, kcol, Ks);
    load_ttile<D>(qkv, ld, tok0 + kv0, vcol, Vt);
    __syncthreads();
    if (kv0 > q0 + 31) continue;  // every key of the tile is after every query of the wave

    f32x16 st[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int s = 0; s < NS; ++s)
        st[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_row<D>(Ks, mt * 32 + l32, s, h), qf[s],
                                                         st[mt], 0, 0, 0);
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kv0 + mt * 32 + acc_row(r, h);
        const float v = key <= qi ? st[mt][r] * scale_log2 : -INFINITY;
        st[mt][r] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m, mx);
    const float alpha = exp2f(m - m_new);
    float ps = 0.0f;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2f(st[mt][r] - m_new);
        st[mt][r] = p;
        ps += p;
      }
    ps += __shfl_xor(ps, 32, 64);
    l = l * alpha + ps;
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) o[dt] *= alpha;
#pragma unroll
    for (int s = 0; s < KT / 16; ++s) {
      float pv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) pv[j] = st[s >> 1][8 * (s & 1) + j];
      const bf16x8 pb = to_bf16x8(pv);
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_t(Vt, dt * 32 + l32, s, h), pb, o[dt], 0,
                                                        0, 0);
    }
  }
  __syncthreads();
  if (h == 0) lse[(static_cast<int64_t>(b) * Hq + hq) * S + qi] = (m + log2f(l)) * kLn2;
  store_qrows<D>(o, 1.0f / l, smem + wave * (32 * D * 2), out + hq * D, ldo, tok0 + q0);
}

// ---- backward ---------------------------------------------------------------

// D[b, h, q] = sum_d dO[q, h d] * O[q, h d]: one wave per (token, head).
template <int D>
__global__ __launch_bounds__(kThreads) void attn_bwd_dot(const uint16_t* __restrict__ dout,
                                                         const uint16_t* __restrict__ out,
                                                         int64_t ldo, int64_t T, int S, int Hq,
                                                         float* __restrict__ dsum) {
  const int64_t w = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (w >= T * Hq) return;
  const int64_t t = w / Hq;
  const int hq = static_cast<int>(w % Hq);
  float acc = 0.0f;
  for (int d = lane; d < D; d += 64)
    acc += bf16_to_f32(dout[t * ldo + hq * D + d]) * bf16_to_f32(out[t * ldo + hq * D + d]);
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) {
    const int64_t b = t / S, s = t % S;
    dsum[(b * Hq + hq) * S + s] = acc;
  }
}

// dK, dV: keys along lanes. A block owns 128 keys of one kv head (32 per
// wave) and walks every query head of its group and every query tile at or
// after its first key.
template <int D>
__global__ __launch_bounds__(kThreads) void attn_bwd_dkdv(
    const uint16_t* __restrict__ qkv, int64_t ld, const uint16_t* __restrict__ dout, int64_t ldo,
    const float* __restrict__ lse, const float* __restrict__ dsum, int S, int Hq, int Hkv,
    float scale, uint16_t* __restrict__ dqkv) {
  constexpr int NS = D / 16;
  constexpr int TILE = 64 * D * 2;
  __shared__ __attribute__((aligned(16))) uint8_t smem[4 * TILE + 2 * 64 * 4];
  uint8_t* Qs = smem;
  uint8_t* Qt = smem + TILE;
  uint8_t* Os = smem + 2 * TILE;
  uint8_t* Ot = smem + 3 * TILE;
  float* Ls = reinterpret_cast<float*>(smem + 4 * TILE);
  float* Ds = Ls + 64;
  const int kb = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int G = Hq / Hkv;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
  const int k0w = kb * QB + wave * 32;
  const int kj = k0w + l32;  // this lane's key
  const int64_t tok0 = static_cast<int64_t>(b) * S;
  const int kcol = (Hq + g) * D, vcol = (Hq + Hkv + g) * D;
  const float scale_log2 = scale * kLog2e;

  bf16x8 kf[NS], vf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    kf[s] = *reinterpret_cast<const bf16x8*>(qkv + (tok0 + kj) * ld + kcol + s * 16 + h * 8);
    vf[s] = *reinterpret_cast<const bf16x8*>(qkv + (tok0 + kj) * ld + vcol + s * 16 + h * 8);
  }
  f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
    dk[dt] = f32x16{};
    dv[dt] = f32x16{};
  }

  for (int gq = 0; gq < G; ++gq) {
    const int hq = g * G + gq;
    const float* lse_h = lse + (static_cast<int64_t>(b) * Hq + hq) * S;
    const float* d_h = dsum + (static_cast<int64_t>(b) * Hq + hq) * S;
    for (int qt0 = (kb * QB) / 64 * 64; qt0 < S; qt0 += 64) {
      __syncthreads();
      load_rowtile<D>(qkv, ld, tok0 + qt0, hq * D, Qs);
      load_ttile<D>(qkv, ld, tok0 + qt0, hq * D, Qt);
      load_rowtile<D>(dout, ldo, tok0 + qt0, hq * D, Os);
      load_ttile<D>(dout, ldo, tok0 + qt0, hq * D, Ot);
      if (threadIdx.x < 64) Ls[threadIdx.x] = lse_h[qt0 + threadIdx.x] * kLog2e;
      else if (threadIdx.x < 128) Ds[threadIdx.x - 64] = d_h[qt0 + threadIdx.x - 64];
      __syncthreads();
#pragma unroll
      for (int mq = 0; mq < 2; ++mq) {
        const int qs0 = qt0 + mq * 32;
        if (qs0 + 31 < k0w) continue;  // every query before every key of the wave
        f32x16 sacc = f32x16{}, dp = f32x16{};
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_row<D>(Qs, mq * 32 + l32, s, h), kf[s],
                                                         sacc, 0, 0, 0);
          dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_row<D>(Os, mq * 32 + l32, s, h), vf[s],
                                                       dp, 0, 0, 0);
        }
        float pr[16], dsr[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qrow = mq * 32 + acc_row(r, h);
          const float p = (kj <= qt0 + qrow) ? exp2f(sacc[r] * scale_log2 - Ls[qrow]) : 0.0f;
          pr[r] = p;
          dsr[r] = p * (dp[r] - Ds[qrow]);
        }
#pragma unroll
        for (int ss = 0; ss < 2; ++ss) {
          const bf16x8 pa = to_bf16x8(pr + 8 * ss);
          const bf16x8 da = to_bf16x8(dsr + 8 * ss);
#pragma unroll
          for (int dt = 0; dt < D / 32; ++dt) {
            dv[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa, frag_t(Ot, dt * 32 + l32, 2 * mq + ss, h),
                                                             dv[dt], 0, 0, 0);
            dk[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(da, frag_t(Qt, dt * 32 + l32, 2 * mq + ss, h),
                                                             dk[dt], 0, 0, 0);
          }
        }
      }
    }
  }
  // dk[dt][r]: key k0w + acc_row(r, h), d = dt * 32 + l32.
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = tok0 + k0w + acc_row(r, h);
      dqkv[row * ld + kcol + dt * 32 + l32] = f32_to_bf16(dk[dt][r] * scale);
      dqkv[row * ld + vcol + dt * 32 + l32] = f32_to_bf16(dv[dt][r]);
    }
}

// dQ: queries along lanes; a block owns 128 queries of one query head.
template <int D>
__global__ __launch_bounds__(kThreads) void attn_bwd_dq(
    const uint16_t* __restrict__ qkv, int64_t ld, const uint16_t* __restrict__ dout, int64_t ldo,
    const float* __restrict__ lse, const float* __restrict__ dsum, int S, int Hq, int Hkv,
    float scale, uint16_t* __restrict__ dqkv) {
  constexpr int NS = D / 16;
  constexpr int TILE = 64 * D * 2;
  __shared__ __attribute__((aligned(16))) uint8_t smem[3 * TILE];
  uint8_t* Ks = smem;
  uint8_t* Kt = smem + TILE;
  uint8_t* Vs = smem + 2 * TILE;
  const int qb = blockIdx.x, hq = blockIdx.y, b = blockIdx.z;
  const int g = hq / (Hq / Hkv);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
  const int q0 = qb * QB + wave * 32;
  const int qi = q0 + l32;
  const int64_t tok0 = static_cast<int64_t>(b) * S;
  const int kcol = (Hq + g) * D, vcol = (Hq + Hkv + g) * D;
  const float scale_log2 = scale * kLog2e;
  const float lse2 = lse[(static_cast<int64_t>(b) * Hq + hq) * S + qi] * kLog2e;
  const float dq_sum = dsum[(static_cast<int64_t>(b) * Hq + hq) * S + qi];

  bf16x8 qf[NS], of[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    qf[s] = *reinterpret_cast<const bf16x8*>(qkv + (tok0 + qi) * ld + hq * D + s * 16 + h * 8);
    of[s] = *reinterpret_cast<const bf16x8*>(dout + (tok0 + qi) * ldo + hq * D + s * 16 + h * 8);
  }
  f32x16 dq[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) dq[dt] = f32x16{};

  const int kv_end = min(S, qb * QB + QB);
  for (int kv0 = 0; kv0 < kv_end; kv0 += KT) {
    __syncthreads();
    load_rowtile<D>(qkv, ld, tok0 + kv0, kcol, Ks);
    load_ttile<D>(qkv, ld, tok0 + kv0, kcol, Kt);
    load_rowtile<D>(qkv, ld, tok0 + kv0, vcol, Vs);
    __syncthreads();
    if (kv0 > q0 + 31) continue;
    f32x16 st[2] = {f32x16{}, f32x16{}}, dpt[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        st[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_row<D>(Ks, mt * 32 + l32, s, h), qf[s],
                                                         st[mt], 0, 0, 0);
        dpt[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_row<D>(Vs, mt * 32 + l32, s, h), of[s],
                                                          dpt[mt], 0, 0, 0);
      }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kv0 + mt * 32 + acc_row(r, h);
        const float p = key <= qi ? exp2f(st[mt][r] * scale_log2 - lse2) : 0.0f;
        st[mt][r] = p * (dpt[mt][r] - dq_sum);  // dS^T
      }
#pragma unroll
    for (int s = 0; s < KT / 16; ++s) {
      float dv8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) dv8[j] = st[s >> 1][8 * (s & 1) + j];
      const bf16x8 db = to_bf16x8(dv8);
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
        dq[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_t(Kt, dt * 32 + l32, s, h), db, dq[dt], 0,
                                                         0, 0);
    }
  }
  __syncthreads();
  store_qrows<D>(dq, scale, smem + wave * (32 * D * 2), dqkv + hq * D, ld, tok0 + q0);
}

template <int D>
int launch_fwd(const uint16_t* qkv, int64_t ld, int B, int S, int Hq, int Hkv, float scale,
               uint16_t* out, int64_t ldo, float* lse, hipStream_t s) {
  hipLaunchKernelGGL(attn_fwd<D>, dim3(S / QB, Hq, B), dim3(kThreads), 0, s, qkv, ld, S, Hq, Hkv,
                     scale * kLog2e, out, ldo, lse);
  MR_LAUNCH_CHECK("mr_attn_fwd");
  return MR_OK;
}

template <int D>
int launch_bwd(const uint16_t* qkv, int64_t ld, const uint16_t* out, const uint16_t* dout,
               int64_t ldo, const float* lse, float* dsum, int B, int S, int Hq, int Hkv,
               float scale, uint16_t* dqkv, hipStream_t s) {
  const int64_t T = static_cast<int64_t>(B) * S;
  const int64_t waves = T * Hq;
  hipLaunchKernelGGL(attn_bwd_dot<D>, dim3(static_cast<unsigned>((waves + 3) / 4)), dim3(kThreads), 0,
                     s, dout, out, ldo, T, S, Hq, dsum);
  hipLaunchKernelGGL(attn_bwd_dkdv<D>, dim3(S / QB, Hkv, B), dim3(kThreads), 0, s, qkv, ld, dout, ldo,
                     lse, dsum, S, Hq, Hkv, scale, dqkv);
  hipLaunchKernelGGL(attn_bwd_dq<D>, dim3(S / QB, Hq, B), dim3(kThreads), 0, s, qkv, ld, dout, ldo,
                     lse, dsum, S, Hq, Hkv, scale, dqkv);
  MR_LAUNCH_CHECK("mr_attn_bwd");
  return MR_OK;
}

int check(const char* fn, const void* qkv, int64_t ld, int B, int S, int Hq, int Hkv, int d,
          int64_t ldo) {
  if (!qkv) return fail(MR_EINVAL, "%s: null pointer", fn);
  if (d != 64 && d != 128) return fail(MR_EINVAL, "%s: head_dim must be 64 or 128, got %d", fn, d);
  if (S <= 0 || S % QB) return fail(MR_EINVAL, "%s: the sequence length must be a multiple of %d", fn, QB);
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv)
    return fail(MR_EINVAL, "%s: query heads must be a multiple of kv heads", fn);
  if (ld < static_cast<int64_t>(Hq + 2 * Hkv) * d || ld % 8 || ldo < static_cast<int64_t>(Hq) * d ||
      ldo % 8)
    return fail(MR_EINVAL, "%s: bad leading dimension", fn);
  if (!aligned16(qkv)) return fail(MR_EINVAL, "%s: qkv must be 16-byte aligned", fn);
  return MR_OK;
}

}  // namespace
}  // namespace mr

extern "C" {

int mr_attn_fwd(const void* qkv, int64_t ld, int B, int S, int Hq, int Hkv, int head_dim,
                float scale, void* out, int64_t ldo, float* lse, void* stream) {
  using namespace mr;
  clear_error();
  int rc = check("mr_attn_fwd", qkv, ld, B, S, Hq, Hkv, head_dim, ldo);
  if (rc) return rc;
  if (!out || !lse || !aligned16(out)) return fail(MR_EINVAL, "mr_attn_fwd: bad output");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* q = static_cast<const uint16_t*>(qkv);
  uint16_t* o = static_cast<uint16_t*>(out);
  if (head_dim == 128) return launch_fwd<128>(q, ld, B, S, Hq, Hkv, scale, o, ldo, lse, s);
  return launch_fwd<64>(q, ld, B, S, Hq, Hkv, scale, o, ldo, lse, s);
}

int mr_attn_bwd(const void* qkv, int64_t ld, const void* out, const void* dout, int64_t ldo,
                const float* lse, float* dsum_ws, int B, int S, int Hq, int Hkv, int head_dim,
                float scale, void* dqkv, void* stream) {
  using namespace mr;
  clear_error();
  int rc = check("mr_attn_bwd", qkv, ld, B, S, Hq, Hkv, head_dim, ldo);
  if (rc) return rc;
  if (!out || !dout || !lse || !dsum_ws || !dqkv || !aligned16(dout) || !aligned16(dqkv))
    return fail(MR_EINVAL, "mr_attn_bwd: bad argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* q = static_cast<const uint16_t*>(qkv);
  const uint16_t* o = static_cast<const uint16_t*>(out);
  const uint16_t* dO = static_cast<const uint16_t*>(dout);
  uint16_t* dq = static_cast<uint16_t*>(dqkv);
  if (head_dim == 128) return launch_bwd<128>(q, ld, o, dO, ldo, lse, dsum_ws, B, S, Hq, Hkv, scale, dq, s);
  return launch_bwd<64>(q, ld, o, dO, ldo, lse, dsum_ws, B, S, Hq, Hkv, scale, dq, s);
}

}  // extern "C"
