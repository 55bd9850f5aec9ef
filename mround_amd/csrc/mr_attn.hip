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
// Transposed operands of the dK/dV pair kernel are read this many MFMAs
// ahead (3 and 7 measured no faster: they spill).
constexpr int kAhead = 1;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
template <int V>
using Ic = std::integral_constant<int, V>;

// s_waitcnt immediate (gfx9 encoding) for vmcnt(vm) lgkmcnt(0), expcnt not
// waited on: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8. Through the
// builtin, unlike inline assembly, the compiler's own wait insertion knows
// the wait happened and adds none of its own for the loads it covers.
constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4); }

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return pack_bf16x2(a, b);
}

// ---- LDS tiles --------------------------------------------------------------
// Row-major tile of ROWS rows x D bf16 (K-major for the MFMA: row = m or n,
// D = reduction), 16-byte chunk c of row r at position c ^ swz_bits(r).
// The XOR applied to a row's 16-byte chunk index. An LDS cycle serves 16
// lanes of a 16-byte read or 32 lanes of an 8-byte read (256 bytes, all 64
// banks): the row operand reads take 16 consecutive rows at one chunk, the
// transposing reads 4 consecutive rows (from a multiple of 4) at 4
// consecutive chunks. D = 128 (a row spans all banks): a 4-bit rotation of
// the row, so 16 rows are 16 positions and rows r0..r0+3 differ in the two
// high bits. D = 64 (two rows per bank cycle, split by parity): a 3-bit
// rotation of r / 2 with the same two properties within each half.
template <int D>
__device__ __forceinline__ int swz_bits(int r) {
  if constexpr (D == 128) return ((r & 3) << 2) | ((r >> 2) & 3);
  else return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
}
template <int D>
__device__ __forceinline__ int rowtile_off(int r, int c) {
  return r * (D * 2) + ((c ^ swz_bits<D>(r)) << 4);
}
template <int D>
__device__ __forceinline__ bf16x8 frag_row(const uint8_t* lds, int r, int s, int h) {
  return *reinterpret_cast<const bf16x8*>(lds + rowtile_off<D>(r, 2 * s + h));
}
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16_t;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8_t;
typedef const __attribute__((address_space(3))) uint8_t* lds_cptr;
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void gbl_void_t;

// 64 rows x D bf16 of a [*, ld] matrix (rows r0.., columns col..) into a
// rowtile by direct-to-LDS loads (16 B per lane, no registers). One wave
// instruction fills 1 KB = 64 / (D / 8) rows; lane l covers row l / (D / 8)
// of it at physical chunk l % (D / 8), i.e. logical chunk (l % (D/8)) ^ swz_bits(row).
template <int D, int NW = 4>
__device__ __forceinline__ void dma_rowtile_one(const uint16_t* src, int64_t ld, int64_t r0, int col,
                                                uint8_t* lds, int i, int wave) {
  constexpr int CPR = D / 8;
  constexpr int RPI = 64 / CPR;
  const int lane = threadIdx.x & 63;
  const int sub = lane / CPR, pchunk = lane % CPR;
  const int rb = (i * NW + wave) * RPI;
  const int row = rb + sub;
  const int c = pchunk ^ swz_bits<D>(row);
  const uint16_t* g = src + (r0 + row) * ld + col + c * 8;
  __builtin_amdgcn_global_load_lds((const gbl_void_t*)g, (lds_void_t*)(lds + rb * (2 * D)), 16, 0, 0);
}
// The INSTR instructions of one wave (dma_rowtile_one issues instruction i alone).
template <int D, int NW = 4>
__device__ __forceinline__ void dma_rowtile(const uint16_t* src, int64_t ld, int64_t r0, int col,
                                            uint8_t* lds, int wave = -1) {
  constexpr int RPI = 64 / (D / 8);
  constexpr int INSTR = 64 / RPI / NW;
  static_assert(INSTR * RPI * NW == 64, "the waves must split the tile evenly");
  if (wave < 0) wave = threadIdx.x >> 6;  // else: this wave's index among the NW
#pragma unroll
  for (int i = 0; i < INSTR; ++i) dma_rowtile_one<D, NW>(src, ld, r0, col, lds, i, wave);
}

// Transposed MFMA operand from a rowtile with ds_read_b64_tr_b16. In each
// group of 16 lanes, lane i receives, for j = 0..3, element i % 4 of the
// 8 bytes addressed by lane 4 j + i / 4; so when source lane s addresses row
// k0 + s / 4 at column c0 + 4 (s % 4), lane i gets rows k0..k0+3 of column
// c0 + i. For the operand of MFMA k16 step `s` (rows 16 s.. of the tile) at
// columns cb + (lane / 16 % 2) * 16 + lane % 16, in accumulator key order:
// rows 16 s + 4 h + {0..3} and 16 s + 8 + 4 h + {0..3} (h = lane / 32).
template <int D>
__device__ __forceinline__ bf16x8 frag_tr(const uint8_t* lds, int cb, int s, int lane) {
  const int h = lane >> 5, q = (lane >> 4) & 1, i = lane & 15;
  const int c = (cb + q * 16) / 8 + ((i & 3) >> 1);
  const int byte = (i & 1) * 8;
  const int row0 = 16 * s + 4 * h + (i >> 2);
  const int row1 = row0 + 8;
  const __attribute__((address_space(3))) uint8_t* base = (const __attribute__((address_space(3))) uint8_t*)lds;
  const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16_t*)(base + rowtile_off<D>(row0, c) + byte));
  const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16_t*)(base + rowtile_off<D>(row1, c) + byte));
  typedef short v8i16 __attribute__((ext_vector_type(8)));
  const v8i16 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ bf16x8 cvt8(const f32x16& x, int off) {
  f32x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = x[off + j];
  return __builtin_convertvector(v, bf16x8);
}

// The low bf16 half of 8 accumulator values: bf16(x - bf16(x)), exact in the
// subtraction (split precision carries x as the two halves).
__device__ __forceinline__ bf16x8 cvt8_lo(const f32x16& x, int off) {
  f32x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = x[off + j];
  const f32x8 hi = __builtin_convertvector(__builtin_convertvector(v, bf16x8), f32x8);
  return __builtin_convertvector(v - hi, bf16x8);
}

// Accumulator register r of a 32x32 tile, lane half h: row within the tile.
__device__ __forceinline__ int acc_row(int r, int h) { return (r >> 2) * 8 + h * 4 + (r & 3); }

// Writes a wave's O^T-layout accumulators (acc[dt][r] = value at d = dt*32 +
// acc_row(r, h), query = lane & 31), times `mul`, as bf16 rows [32 queries][D]
// through LDS: packed 8-byte writes into rows padded to 2 D + 8 bytes (no
// bank conflicts), then 16-byte row-contiguous global stores.
// (store_qrows_f: the value written is bf16(f(acc)) instead.)
template <int D, typename F>
__device__ __forceinline__ void store_qrows_f(const f32x16 (&acc)[D / 32], F f, uint8_t* lds,
                                             uint16_t* dst, int64_t ld, int64_t row0) {
  constexpr int STAGE_ROW = 2 * D + 8;
  const int lane = threadIdx.x & 63, h = lane >> 5, q = lane & 31;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const uint32_t w0 = pack_bf16(f(acc[dt][rg * 4 + 0]), f(acc[dt][rg * 4 + 1]));
      const uint32_t w1 = pack_bf16(f(acc[dt][rg * 4 + 2]), f(acc[dt][rg * 4 + 3]));
      const int col = dt * 32 + rg * 8 + h * 4;
      *reinterpret_cast<uint2*>(lds + q * STAGE_ROW + col * 2) = make_uint2(w0, w1);
    }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  constexpr int CH = D / 8;
  for (int c = lane; c < 32 * CH; c += 64) {
    const int row = c / CH, ch = c % CH;
    const uint2 a = *reinterpret_cast<const uint2*>(lds + row * STAGE_ROW + ch * 16);
    const uint2 b = *reinterpret_cast<const uint2*>(lds + row * STAGE_ROW + ch * 16 + 8);
    *reinterpret_cast<uint4*>(dst + (row0 + row) * ld + ch * 8) = make_uint4(a.x, a.y, b.x, b.y);
  }
}
template <int D>
__device__ __forceinline__ void store_qrows(const f32x16 (&acc)[D / 32], float mul, uint8_t* lds,
                                           uint16_t* dst, int64_t ld, int64_t row0) {
  store_qrows_f<D>(acc, [mul](float x) { return x * mul; }, lds, dst, ld, row0);
}

// ---- forward ----------------------------------------------------------------
//
// A block of W waves owns 32 W queries of one query head (32 per wave, one
// MFMA column tile) and walks the key tiles up to its last query. K and V
// tiles move HBM -> LDS by direct loads, double buffered: tile t + 1 is in
// flight while tile t is computed, with one barrier per tile. V stays
// row-major in LDS; its transposed operand comes from the transposing read.
// A wave holds Q (D / 4 registers), O^T (D / 2) and one 64-key score tile
// (32), so two waves share each SIMD and one wave's softmax overlaps the
// other's MFMAs.
//
// The running row maximum m is raised only when a tile's maximum exceeds it
// by more than kRaise (log2 units) in some lane of the wave; until then the
// probabilities exp2(s - m) stay below 2^kRaise, far inside fp32 and bf16
// range. Output and log-sum-exp are relative to the same m, so the result is
// the exact softmax up to rounding; most tiles skip the O rescale.
constexpr float kRaise = 8.0f;

// Cross-half reductions: v_permlane32_swap exchanges the two 32-lane halves,
// leaving lane l's value and lane l ^ 32's in the two results.
__device__ __forceinline__ float xhalf_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// SPLIT: split precision (q, k and v each carried as bf16 hi and lo halves,
// from qkv and qkv_lo): S^T = K_hi Q_hi^T + K_lo Q_hi^T + K_hi Q_lo^T and
// O^T += V_hi^T P_hi^T + V_lo^T P_hi^T + V_hi^T P_lo^T with P = P_hi + P_lo,
// the low-by-low terms left out, so the scores, probabilities and output hold
// about 16 significant bits. The output is written split as well, row t of
// out_split holding [hi | hi | lo] of the Hq D outputs (the activation order
// of a split product over K' = 3 Hq D), and its hi half into out. Twice the
// LDS and three times the MFMAs; one wave per SIMD (W = 4), whose register
// file holds the extra fragments.
template <int D, int W, bool SPLIT = false>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(SPLIT ? 1 : 2))) void attn_fwd(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ qkv_lo, int64_t ld, int S, int Hq, int Hkv,
    float scale_log2, uint16_t* __restrict__ out, int64_t ldo, uint16_t* __restrict__ out_split,
    int64_t ld_split, float* __restrict__ lse) {
  constexpr int NS = D / 16, ND = D / 32;
  constexpr int TILE = KT * D * 2;
  constexpr int NT = SPLIT ? 8 : 4;     // LDS tiles: K, V of two stages (and their lo halves)
  constexpr int STAGE_ROW = 2 * D + 8;  // staged output row (bytes), 8-byte aligned
  constexpr int SMEM = NT * TILE > W * 32 * STAGE_ROW ? NT * TILE : W * 32 * STAGE_ROW;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];
  uint8_t* const K0 = smem;
  uint8_t* const V0 = smem + TILE;
  uint8_t* const K1 = smem + 2 * TILE;
  uint8_t* const V1 = smem + 3 * TILE;
  constexpr int LO = 4 * TILE;  // a stage tile's lo half sits this far behind it
  const int qb = gridDim.z - 1 - blockIdx.z;  // the longest blocks start first
  const int hq = blockIdx.x, b = blockIdx.y;
  const int g = hq / (Hq / Hkv);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
  const int q0 = qb * (32 * W) + wave * 32;
  const int qi = q0 + l32;
  const int64_t tok0 = static_cast<int64_t>(b) * S;
  const int kcol = (Hq + g) * D, vcol = (Hq + Hkv + g) * D;
  const int n_tiles = (qb + 1) * (32 * W) / KT;

  auto load_tiles = [&](int64_t r0, uint8_t* Kd, uint8_t* Vd) {
    dma_rowtile<D, W>(qkv, ld, r0, kcol, Kd);
    dma_rowtile<D, W>(qkv, ld, r0, vcol, Vd);
    if constexpr (SPLIT) {
      dma_rowtile<D, W>(qkv_lo, ld, r0, kcol, Kd + LO);
      dma_rowtile<D, W>(qkv_lo, ld, r0, vcol, Vd + LO);
    }
  };
  load_tiles(tok0, K0, V0);

  bf16x8 qf[NS], ql[SPLIT ? NS : 1];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    qf[s] = *reinterpret_cast<const bf16x8*>(qkv + (tok0 + qi) * ld + hq * D + s * 16 + h * 8);
    if constexpr (SPLIT)
      ql[s] = *reinterpret_cast<const bf16x8*>(qkv_lo + (tok0 + qi) * ld + hq * D + s * 16 + h * 8);
  }
  f32x16 o[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) o[dt] = f32x16{};
  float m = -INFINITY, l = 0.0f;

  auto step = [&](int t, const uint8_t* Kc, const uint8_t* Vc, uint8_t* Kn, uint8_t* Vn) {
    __builtin_amdgcn_s_waitcnt(0);  // this thread's loads of tile t have landed
    __syncthreads();                // everyone's have, and nobody still reads the other buffers
    if (t + 1 < n_tiles) load_tiles(tok0 + (t + 1) * KT, Kn, Vn);
    const int kv0 = t * KT;
    if (kv0 > q0 + 31) return;  // every key of the tile is after every query of the wave

    f32x16 st[2] = {f32x16{}, f32x16{}};
    bf16x8 kfr[2][2];  // K fragments, step s + 1 read while step s multiplies
    kfr[0][0] = frag_row<D>(Kc, l32, 0, h);
    kfr[0][1] = frag_row<D>(Kc, 32 + l32, 0, h);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (s + 1 < NS) {
        kfr[(s + 1) & 1][0] = frag_row<D>(Kc, l32, s + 1, h);
        kfr[(s + 1) & 1][1] = frag_row<D>(Kc, 32 + l32, s + 1, h);
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        st[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfr[s & 1][mt], qf[s], st[mt], 0, 0, 0);
        if constexpr (SPLIT) {
          st[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_row<D>(Kc + LO, mt * 32 + l32, s, h), qf[s],
                                                           st[mt], 0, 0, 0);
          st[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfr[s & 1][mt], ql[s], st[mt], 0, 0, 0);
        }
      }
    }
    if (kv0 + KT - 1 > q0) {  // the tile crosses the wave's diagonal
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kv0 + mt * 32 + acc_row(r, h) > qi) st[mt][r] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[mt][r]);
    const float mc = xhalf_max(mx) * scale_log2;
    if (__builtin_amdgcn_ballot_w64(mc > m + kRaise)) {
      const float m_new = fmaxf(m, mc);
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) o[dt] *= alpha;
      m = m_new;
    }
    float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // four short chains instead of one long one
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(st[mt][r], scale_log2, -m));
        st[mt][r] = pv;
        ps[r & 3] += pv;
      }
    l += xhalf_sum((ps[0] + ps[1]) + (ps[2] + ps[3]));
#pragma unroll
    for (int s = 0; s < KT / 16; ++s) {
      const bf16x8 pb = cvt8(st[s >> 1], 8 * (s & 1));
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) {
        const bf16x8 vt = frag_tr<D>(Vc, dt * 32, s, lane);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vt, pb, o[dt], 0, 0, 0);
        if constexpr (SPLIT) {
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_tr<D>(Vc + LO, dt * 32, s, lane), pb, o[dt],
                                                          0, 0, 0);
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vt, cvt8_lo(st[s >> 1], 8 * (s & 1)), o[dt], 0, 0, 0);
        }
      }
    }
  };

  int t = 0;
  for (; t + 1 < n_tiles; t += 2) {
    step(t, K0, V0, K1, V1);
    step(t + 1, K1, V1, K0, V0);
  }
  if (t < n_tiles) step(t, K0, V0, K1, V1);
  __syncthreads();  // all tiles read; the buffers now stage the output

  if (h == 0) lse[(static_cast<int64_t>(b) * Hq + hq) * S + qi] = (m + log2f(l)) * kLn2;
  uint8_t* const stage = smem + wave * 32 * STAGE_ROW;
  const float inv_l = 1.0f / l;
  store_qrows<D>(o, inv_l, stage, out + hq * D, ldo, tok0 + q0);
  if constexpr (SPLIT) {
    const auto hi = [inv_l](float x) { return x * inv_l; };
    const auto lo = [inv_l](float x) {
      const float y = x * inv_l;
      return y - bf16_to_f32(f32_to_bf16(y));
    };
    const int64_t seg = static_cast<int64_t>(Hq) * D;
    store_qrows_f<D>(o, hi, stage, out_split + hq * D, ld_split, tok0 + q0);
    store_qrows_f<D>(o, hi, stage, out_split + seg + hq * D, ld_split, tok0 + q0);
    store_qrows_f<D>(o, lo, stage, out_split + 2 * seg + hq * D, ld_split, tok0 + q0);
  }
}

// ---- backward ---------------------------------------------------------------

// D[b, h, q] = sum_d dO[q, h d] * O[q, h d]: D / 8 lanes per (token, head),
// each with one 16-byte load of dO and of O; the group's partial sums meet by
// lane exchanges inside the group.
template <int D>
__global__ __launch_bounds__(kThreads) void attn_bwd_dot(const uint16_t* __restrict__ dout,
                                                         const uint16_t* __restrict__ out,
                                                         int64_t ldo, int64_t T, int S, int Hq,
                                                         float* __restrict__ dsum) {
  constexpr int L = D / 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t pair = gid / L;
  const int sub = static_cast<int>(gid % L);
  const bool valid = pair < T * Hq;
  float acc = 0.0f;
  int64_t t = 0;
  int hq = 0;
  if (valid) {
    t = pair / Hq;
    hq = static_cast<int>(pair % Hq);
    const uint4 a = *reinterpret_cast<const uint4*>(dout + t * ldo + hq * D + sub * 8);
    const uint4 o = *reinterpret_cast<const uint4*>(out + t * ldo + hq * D + sub * 8);
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, ow[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      acc += __uint_as_float(aw[k] << 16) * __uint_as_float(ow[k] << 16);
      acc += __uint_as_float(aw[k] & 0xffff0000u) * __uint_as_float(ow[k] & 0xffff0000u);
    }
  }
#pragma unroll
  for (int off = L / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (valid && sub == 0) {
    const int64_t b = t / S, s = t % S;
    dsum[(b * Hq + hq) * S + s] = acc;
  }
}

// dK, dV: keys along lanes. A block owns 128 keys of one kv head (32 per
// wave) and walks, for every query head of the group, the 64-query tiles at
// or after its first key. Q and dO tiles arrive by direct loads, double
// buffered like the forward's K and V; their transposed operands (for
// dV = P^T dO and dK = dS^T Q) come from the transposing LDS read.
// D = 64 fits two waves per SIMD (254 registers, no spills): 7 % faster on
// the 0.5B shape (8 x 2048 tokens, 14 / 2 heads). D = 128 needs 486.
template <int D>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(D == 64 ? 2 : 1))) void attn_bwd_dkdv(
    const uint16_t* __restrict__ qkv, int64_t ld, const uint16_t* __restrict__ dout, int64_t ldo,
    const float* __restrict__ lse, const float* __restrict__ dsum, int S, int Hq, int Hkv,
    float scale, uint16_t* __restrict__ dqkv, int hsplit, float* __restrict__ part) {
  constexpr int NS = D / 16, ND = D / 32;
  constexpr int TILE = 64 * D * 2;
  __shared__ __attribute__((aligned(1024))) uint8_t Q0[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t O0[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t Q1[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t O1[TILE];
  __shared__ __attribute__((aligned(16))) float LD0[128];  // lse (log2 domain) then rowsum(dO O) of the tile's 64 queries
  __shared__ __attribute__((aligned(16))) float LD1[128];
  const int kb = blockIdx.z, g = blockIdx.x / hsplit, hs = blockIdx.x % hsplit, b = blockIdx.y;
  const int G = Hq / Hkv;
  // This block's query heads of the group: [h_lo, h_hi) (all of them unless split).
  const int h_lo = hs * G / hsplit, h_hi = (hs + 1) * G / hsplit;
  const int hq0 = g * G + h_lo;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
  const int k0w = kb * QB + wave * 32;
  const int kj = k0w + l32;  // this lane's key
  const int64_t tok0 = static_cast<int64_t>(b) * S;
  const int kcol = (Hq + g) * D, vcol = (Hq + Hkv + g) * D;
  const float scale_log2 = scale * kLog2e;
  const int first_q = kb * QB;
  const int nqt = (S - first_q) / 64;  // query tiles per head
  const int n_items = (h_hi - h_lo) * nqt;

  // item i: query head hq0 + i / nqt, query tile first_q + 64 (i % nqt)
  auto issue = [&](int i, uint8_t* Qd, uint8_t* Od) {
    const int hq = hq0 + i / nqt;
    const int64_t r0 = tok0 + first_q + (i % nqt) * 64;
    dma_rowtile<D>(qkv, ld, r0, hq * D, Qd);
    dma_rowtile<D>(dout, ldo, r0, hq * D, Od);
  };
  auto fetch_ld = [&](int i) -> float {  // threads 0..127: this item's lse / rowsum value
    const int hq = hq0 + i / nqt;
    const int q = first_q + (i % nqt) * 64 + (threadIdx.x & 63);
    const int64_t at = (static_cast<int64_t>(b) * Hq + hq) * S + q;
    return threadIdx.x < 64 ? lse[at] * kLog2e : dsum[at];
  };

  bf16x8 kf[NS], vf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    kf[s] = *reinterpret_cast<const bf16x8*>(qkv + (tok0 + kj) * ld + kcol + s * 16 + h * 8);
    vf[s] = *reinterpret_cast<const bf16x8*>(qkv + (tok0 + kj) * ld + vcol + s * 16 + h * 8);
  }
  f32x16 dk[ND], dv[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) {
    dk[dt] = f32x16{};
    dv[dt] = f32x16{};
  }

  issue(0, Q0, O0);
  if (threadIdx.x < 128) LD0[threadIdx.x] = fetch_ld(0);

  // One query tile (two 32-query halves) as a software pipeline. The S^T and
  // dP^T MFMAs of both halves go first (their LDS operands read one step
  // ahead), then each half's softmax and dS run while the MFMA pipe still
  // works on earlier products, and each half's dV, dK MFMAs take their
  // transposed operands one step ahead. sched_barrier pins the order the
  // compiler would otherwise collapse. The first two tiles of every head
  // cross the block's keys (DIAG): there P is zeroed for keys after the
  // query; a half entirely before the wave's keys contributes zeros.
  // Lane-dependent LDS offsets of the tile reads, computed once and hidden
  // from the optimizer, so that every read is its tile plus one of these
  // registers plus an immediate (32-row half, k16 step). Row reads: row l32
  // at chunk 2 s + h. Transposing reads: k-rows 4 h + i / 4 (+ 8), column
  // block dt; the swizzle of those rows does not depend on the k16 step.
  uint32_t row_off[NS], tr_off[2][ND];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    row_off[s] = rowtile_off<D>(l32, 2 * s + h);
    asm volatile("" : "+v"(row_off[s]));
  }
#pragma unroll
  for (int hv = 0; hv < 2; ++hv)
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
      const int q = (lane >> 4) & 1, li = lane & 15;
      tr_off[hv][dt] = rowtile_off<D>(4 * h + (li >> 2) + 8 * hv, (dt * 32 + q * 16) / 8 + ((li & 3) >> 1)) +
                       (li & 1) * 8;
      asm volatile("" : "+v"(tr_off[hv][dt]));
    }
  auto rd_row = [&](const uint8_t* t, int mq, int s) -> bf16x8 {
    return *(const lds_bf16x8_t*)((lds_cptr)t + row_off[s] + mq * 32 * (2 * D));
  };
  auto rd_tr = [&](const uint8_t* t, int dt, int s) -> bf16x8 {
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)((lds_cptr)t + tr_off[0][dt] + s * 16 * (2 * D)));
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)((lds_cptr)t + tr_off[1][dt] + s * 16 * (2 * D)));
    typedef short v8i16 __attribute__((ext_vector_type(8)));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  auto tile = [&](auto diagc, int qt0, const uint8_t* Qc, const uint8_t* Oc, const float* LDc) {
    constexpr bool DIAG = decltype(diagc)::value;
    f32x16 sacc[2] = {f32x16{}, f32x16{}}, dp[2] = {f32x16{}, f32x16{}};
    bf16x8 qa[2], oa[2];
    qa[0] = rd_row(Qc, 0, 0);
    oa[0] = rd_row(Oc, 0, 0);
    auto sdp = [&](auto idxc) {
      constexpr int idx = decltype(idxc)::value, mq = idx / NS, s = idx % NS;
      if constexpr (idx + 1 < 2 * NS) {
        constexpr int n = idx + 1;
        qa[n & 1] = rd_row(Qc, n / NS, n % NS);
        oa[n & 1] = rd_row(Oc, n / NS, n % NS);
      }
      __builtin_amdgcn_sched_barrier(0);
      sacc[mq] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[idx & 1], kf[s], sacc[mq], 0, 0, 0);
      dp[mq] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(oa[idx & 1], vf[s], dp[mq], 0, 0, 0);
    };
    StaticFor<0, 2 * NS>::run(sdp);
    auto half = [&](auto mqc) {
      constexpr int mq = decltype(mqc)::value;
      __builtin_amdgcn_sched_barrier(0);
      bf16x8 ta[2], tb[2];  // dO^T and Q^T operands, one step ahead
      ta[0] = rd_tr(Oc, 0, 2 * mq);
      tb[0] = rd_tr(Qc, 0, 2 * mq);
      const float4* l4 = reinterpret_cast<const float4*>(LDc + mq * 32 + 4 * h);
      const float4* d4 = reinterpret_cast<const float4*>(LDc + 64 + mq * 32 + 4 * h);
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {  // rows 8 gq + 4 h + 0..3 of the half: acc registers 4 gq..
        const float4 lv = l4[2 * gq], dv4 = d4[2 * gq];
        const float lq[4] = {lv.x, lv.y, lv.z, lv.w}, dq[4] = {dv4.x, dv4.y, dv4.z, dv4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * gq + j;
          float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[mq][r], scale_log2, -lq[j]));
          if (DIAG && kj > qt0 + mq * 32 + acc_row(r, h)) p = 0.0f;
          sacc[mq][r] = p;
          dp[mq][r] = p * (dp[mq][r] - dq[j]);
        }
      }
      const bf16x8 pa[2] = {cvt8(sacc[mq], 0), cvt8(sacc[mq], 8)};
      const bf16x8 da[2] = {cvt8(dp[mq], 0), cvt8(dp[mq], 8)};
      auto acc = [&](auto idxc) {
        constexpr int idx = decltype(idxc)::value, ss = idx / ND, dt = idx % ND;
        if constexpr (idx + 1 < 2 * ND) {
          constexpr int n = idx + 1;
          ta[n & 1] = rd_tr(Oc, n % ND, 2 * mq + n / ND);
          tb[n & 1] = rd_tr(Qc, n % ND, 2 * mq + n / ND);
        }
        __builtin_amdgcn_sched_barrier(0);
        dv[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[ss], ta[idx & 1], dv[dt], 0, 0, 0);
        dk[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(da[ss], tb[idx & 1], dk[dt], 0, 0, 0);
      };
      StaticFor<0, 2 * ND>::run(acc);
    };
    half(std::integral_constant<int, 0>{});
    half(std::integral_constant<int, 1>{});
  };

  auto step = [&](int i, const uint8_t* Qc, const uint8_t* Oc, const float* LDc, uint8_t* Qn,
                  uint8_t* On, float* LDn) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    float next_ld = 0.0f;
    const bool more = i + 1 < n_items;
    if (more) {
      issue(i + 1, Qn, On);
      if (threadIdx.x < 128) next_ld = fetch_ld(i + 1);
    }
    const int t = i % nqt;
    if (t < 2) tile(std::true_type{}, first_q + t * 64, Qc, Oc, LDc);
    else tile(std::false_type{}, first_q + t * 64, Qc, Oc, LDc);
    if (more && threadIdx.x < 128) LDn[threadIdx.x] = next_ld;
  };

  int i = 0;
  for (; i + 1 < n_items; i += 2) {
    step(i, Q0, O0, LD0, Q1, O1, LD1);
    step(i + 1, Q1, O1, LD1, Q0, O0, LD0);
  }
  if (i < n_items) step(i, Q0, O0, LD0, Q1, O1, LD1);

  // dk[dt][r]: key k0w + acc_row(r, h), d = dt * 32 + l32. Split blocks
  // write fp32 partials, [split][token][k heads | v heads][d], summed by
  // attn_bwd_kv_reduce in split order.
  if (part) {
    const int64_t W = 2 * static_cast<int64_t>(Hkv) * D;
    float* pb = part + static_cast<int64_t>(hs) * gridDim.y * S * W;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = tok0 + k0w + acc_row(r, h);
        pb[row * W + g * D + dt * 32 + l32] = dk[dt][r] * scale;
        pb[row * W + (Hkv + g) * D + dt * 32 + l32] = dv[dt][r];
      }
    return;
  }
#pragma unroll
  for (int dt = 0; dt < ND; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = tok0 + k0w + acc_row(r, h);
      dqkv[row * ld + kcol + dt * 32 + l32] = f32_to_bf16(dk[dt][r] * scale);
      dqkv[row * ld + vcol + dt * 32 + l32] = f32_to_bf16(dv[dt][r]);
    }
}

// dK, dV at D = 128 with each 32-key group's work split over two waves that
// share a SIMD (waves w and w + 4): the P wave (w < 4) holds K, forms
// S^T = K Q^T and the probabilities P and accumulates dV += P^T dO; the dS
// wave holds V, forms dP^T = V dO^T and, with P from LDS, dS = P (dP -
// rowsum(dO O)) and dK += dS^T Q. Each wave carries one operand and one
// accumulator set, about half of the single-wave kernel's registers, so two
// waves fit a SIMD and one's softmax or dS arithmetic runs under the other's
// MFMAs. P crosses in fp32 in the accumulator layout both waves share (no
// rounding, no shuffles): the products and their order are the single-wave
// kernel's. Two barriers per query tile: one for the tile (the P wave's Q
// and the dS wave's dO arrive by direct loads, double buffered), one for P.
template <int D>
__global__ __launch_bounds__(2 * kThreads) __attribute__((amdgpu_waves_per_eu(2))) void attn_bwd_dkdv_pair(
    const uint16_t* __restrict__ qkv, int64_t ld, const uint16_t* __restrict__ dout, int64_t ldo,
    const float* __restrict__ lse, const float* __restrict__ dsum, int S, int Hq, int Hkv,
    float scale, uint16_t* __restrict__ dqkv, int hsplit, float* __restrict__ part) {
  constexpr int NS = D / 16, ND = D / 32;
  constexpr int TILE = 64 * D * 2;
  __shared__ __attribute__((aligned(1024))) uint8_t Q0[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t O0[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t Q1[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t O1[TILE];
  __shared__ __attribute__((aligned(16))) float LD0[128];  // lse (log2 domain) then rowsum(dO O) of the tile's 64 queries
  __shared__ __attribute__((aligned(16))) float LD1[128];
  // P of each key group: [half][register group][lane] float4, as the P wave holds it.
  __shared__ __attribute__((aligned(16))) float Pb[4][2 * 4 * 64 * 4];
  const int kb = blockIdx.z, g = blockIdx.x / hsplit, hs = blockIdx.x % hsplit, b = blockIdx.y;
  const int G = Hq / Hkv;
  const int h_lo = hs * G / hsplit, h_hi = (hs + 1) * G / hsplit;
  const int hq0 = g * G + h_lo;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
  const bool pwave = wave < 4;
  const int kw = wave & 3;
  const int k0w = kb * QB + kw * 32;
  const int kj = k0w + l32;  // this lane's key
  const int64_t tok0 = static_cast<int64_t>(b) * S;
  const int kcol = (Hq + g) * D, vcol = (Hq + Hkv + g) * D;
  const float scale_log2 = scale * kLog2e;
  const int first_q = kb * QB;
  const int nqt = (S - first_q) / 64;
  const int n_items = (h_hi - h_lo) * nqt;
  float* const Pw = Pb[kw];

  // Item i: query head hq0 + i / nqt, query tile first_q + 64 (i % nqt). The
  // P waves bring Q, the dS waves dO.
  auto issue = [&](int i, uint8_t* Qd, uint8_t* Od) {
    const int hq = hq0 + i / nqt;
    const int64_t r0 = tok0 + first_q + (i % nqt) * 64;
    if (pwave) dma_rowtile<D>(qkv, ld, r0, hq * D, Qd, kw);
    else dma_rowtile<D>(dout, ldo, r0, hq * D, Od, kw);
  };
  auto fetch_ld = [&](int i) -> float {  // threads 0..127: this item's lse / rowsum value
    const int hq = hq0 + i / nqt;
    const int q = first_q + (i % nqt) * 64 + (threadIdx.x & 63);
    const int64_t at = (static_cast<int64_t>(b) * Hq + hq) * S + q;
    return threadIdx.x < 64 ? lse[at] * kLog2e : dsum[at];
  };

  uint32_t row_off[NS], tr_off[2][ND];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    row_off[s] = rowtile_off<D>(l32, 2 * s + h);
    asm volatile("" : "+v"(row_off[s]));
  }
#pragma unroll
  for (int hv = 0; hv < 2; ++hv)
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
      const int q = (lane >> 4) & 1, li = lane & 15;
      tr_off[hv][dt] = rowtile_off<D>(4 * h + (li >> 2) + 8 * hv, (dt * 32 + q * 16) / 8 + ((li & 3) >> 1)) +
                       (li & 1) * 8;
      asm volatile("" : "+v"(tr_off[hv][dt]));
    }
  auto rd_row = [&](const uint8_t* t, int mq, int s) -> bf16x8 {
    return *(const lds_bf16x8_t*)((lds_cptr)t + row_off[s] + mq * 32 * (2 * D));
  };
  auto rd_tr = [&](const uint8_t* t, int dt, int s) -> bf16x8 {
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)((lds_cptr)t + tr_off[0][dt] + s * 16 * (2 * D)));
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)((lds_cptr)t + tr_off[1][dt] + s * 16 * (2 * D)));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) f32x4 lds_f4;
  auto p_slot = [&](int mq, int rg) -> lds_f4* {
    return (lds_f4*)((__attribute__((address_space(3))) float*)Pw + ((mq * 4 + rg) * 64 + lane) * 4);
  };

  issue(0, Q0, O0);
  if (threadIdx.x < 128) LD0[threadIdx.x] = fetch_ld(0);

  // The loop both roles run: the same barriers in the same order.
  auto run = [&](auto& tile) {
    auto step = [&](int i, const uint8_t* Qc, const uint8_t* Oc, const float* LDc, uint8_t* Qn,
                    uint8_t* On, float* LDn) {
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      float next_ld = 0.0f;
      const bool more = i + 1 < n_items;
      if (more && threadIdx.x < 128) next_ld = fetch_ld(i + 1);
      // The next item's direct loads go out after the P barrier: issued with
      // the S^T / dP^T products they slowed those products' operand reads
      // (measured: 9 % of the kernel).
      auto issue_next = [&]() {
        if (more) issue(i + 1, Qn, On);
      };
      const int t = i % nqt;
      if (t < 2) tile(std::true_type{}, first_q + t * 64, Qc, Oc, LDc, issue_next);
      else tile(std::false_type{}, first_q + t * 64, Qc, Oc, LDc, issue_next);
      if (more && threadIdx.x < 128) LDn[threadIdx.x] = next_ld;
    };
    int i = 0;
    for (; i + 1 < n_items; i += 2) {
      step(i, Q0, O0, LD0, Q1, O1, LD1);
      step(i + 1, Q1, O1, LD1, Q0, O0, LD0);
    }
    if (i < n_items) step(i, Q0, O0, LD0, Q1, O1, LD1);
  };

  // dk or dv [dt][r]: key k0w + acc_row(r, h), d = dt * 32 + l32, to the
  // partials ([split][token][k heads | v heads][d]) or as bf16 into dqkv.
  auto write_out = [&](const f32x16 (&acc)[ND], int col_part, int col_out, float mul) {
    if (part) {
      const int64_t W = 2 * static_cast<int64_t>(Hkv) * D;
      float* pb = part + static_cast<int64_t>(hs) * gridDim.y * S * W;
#pragma unroll
      for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = tok0 + k0w + acc_row(r, h);
          pb[row * W + col_part + dt * 32 + l32] = acc[dt][r] * mul;
        }
      return;
    }
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = tok0 + k0w + acc_row(r, h);
        dqkv[row * ld + col_out + dt * 32 + l32] = f32_to_bf16(acc[dt][r] * mul);
      }
  };

  if (pwave) {
    bf16x8 kf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s)
      kf[s] = *reinterpret_cast<const bf16x8*>(qkv + (tok0 + kj) * ld + kcol + s * 16 + h * 8);
    f32x16 dv[ND];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) dv[dt] = f32x16{};
    auto tile = [&](auto diagc, int qt0, const uint8_t* Qc, const uint8_t* Oc, const float* LDc, auto& issue_next) {
      constexpr bool DIAG = decltype(diagc)::value;
      bf16x8 pa[2][2];  // P as the dV MFMA's bf16 operand, per half and k16 step
      {
        f32x16 sacc[2] = {f32x16{}, f32x16{}};
        bf16x8 qa[2];
        qa[0] = rd_row(Qc, 0, 0);
        // The two halves' products alternate, so that consecutive MFMAs do
        // not wait on each other's accumulator.
        auto sm = [&](auto idxc) {
          constexpr int idx = decltype(idxc)::value, mq = idx & 1, s = idx >> 1;
          if constexpr (idx + 1 < 2 * NS) qa[(idx + 1) & 1] = rd_row(Qc, (idx + 1) & 1, (idx + 1) >> 1);
          __builtin_amdgcn_sched_barrier(0);
          sacc[mq] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[idx & 1], kf[s], sacc[mq], 0, 0, 0);
        };
        StaticFor<0, 2 * NS>::run(sm);
#pragma unroll
        for (int mq = 0; mq < 2; ++mq) {
          const float4* l4 = reinterpret_cast<const float4*>(LDc + mq * 32 + 4 * h);
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {  // rows 8 gq + 4 h + 0..3 of the half: registers 4 gq..
            const float4 lv = l4[2 * gq];
            const float lq[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int r = 4 * gq + j;
              float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[mq][r], scale_log2, -lq[j]));
              if (DIAG && kj > qt0 + mq * 32 + acc_row(r, h)) p = 0.0f;
              sacc[mq][r] = p;
            }
            *p_slot(mq, gq) = f32x4{sacc[mq][4 * gq], sacc[mq][4 * gq + 1], sacc[mq][4 * gq + 2],
                                    sacc[mq][4 * gq + 3]};
          }
          pa[mq][0] = cvt8(sacc[mq], 0);
          pa[mq][1] = cvt8(sacc[mq], 8);
        }
      }
      __syncthreads();  // P to the dS waves
      issue_next();
      auto half = [&](auto mqc) {
        constexpr int mq = decltype(mqc)::value;
        // dO^T operands read kAhead MFMAs ahead through a ring of registers
        bf16x8 ta[kAhead + 1];
        auto pre = [&](auto xc) {
          constexpr int x = decltype(xc)::value;
          ta[x] = rd_tr(Oc, x % ND, 2 * mq + x / ND);
        };
        StaticFor<0, kAhead>::run(pre);
        auto acc = [&](auto idxc) {
          constexpr int idx = decltype(idxc)::value, ss = idx / ND, dt = idx % ND, nx = idx + kAhead;
          if constexpr (nx < 2 * ND) ta[nx % (kAhead + 1)] = rd_tr(Oc, nx % ND, 2 * mq + nx / ND);
          __builtin_amdgcn_sched_barrier(0);
          dv[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[mq][ss], ta[idx % (kAhead + 1)], dv[dt], 0, 0, 0);
        };
        StaticFor<0, 2 * ND>::run(acc);
      };
      half(std::integral_constant<int, 0>{});
      half(std::integral_constant<int, 1>{});
    };
    run(tile);
    write_out(dv, (Hkv + g) * D, vcol, 1.0f);
  } else {
    bf16x8 vf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s)
      vf[s] = *reinterpret_cast<const bf16x8*>(qkv + (tok0 + kj) * ld + vcol + s * 16 + h * 8);
    f32x16 dk[ND];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) dk[dt] = f32x16{};
    auto tile = [&](auto diagc, int qt0, const uint8_t* Qc, const uint8_t* Oc, const float* LDc, auto& issue_next) {
      f32x16 dp[2] = {f32x16{}, f32x16{}};
      {
        bf16x8 oa[2];
        oa[0] = rd_row(Oc, 0, 0);
        auto dm = [&](auto idxc) {
          constexpr int idx = decltype(idxc)::value, mq = idx & 1, s = idx >> 1;
          if constexpr (idx + 1 < 2 * NS) oa[(idx + 1) & 1] = rd_row(Oc, (idx + 1) & 1, (idx + 1) >> 1);
          __builtin_amdgcn_sched_barrier(0);
          dp[mq] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(oa[idx & 1], vf[s], dp[mq], 0, 0, 0);
        };
        StaticFor<0, 2 * NS>::run(dm);
      }
      __syncthreads();  // P from the P waves
      issue_next();
      auto half = [&](auto mqc) {
        constexpr int mq = decltype(mqc)::value;
        // Q^T operands read kAhead MFMAs ahead through a ring of registers;
        // the first ones go out before the dS arithmetic, which covers them
        bf16x8 tb[kAhead + 1];
        auto pre = [&](auto xc) {
          constexpr int x = decltype(xc)::value;
          tb[x] = rd_tr(Qc, x % ND, 2 * mq + x / ND);
        };
        StaticFor<0, kAhead>::run(pre);
        const float4* d4 = reinterpret_cast<const float4*>(LDc + 64 + mq * 32 + 4 * h);
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const f32x4 pv = *p_slot(mq, gq);
          const float4 dv4 = d4[2 * gq];
          const float pq[4] = {pv.x, pv.y, pv.z, pv.w}, dq[4] = {dv4.x, dv4.y, dv4.z, dv4.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) dp[mq][4 * gq + j] = pq[j] * (dp[mq][4 * gq + j] - dq[j]);
        }
        const bf16x8 da[2] = {cvt8(dp[mq], 0), cvt8(dp[mq], 8)};
        auto acc = [&](auto idxc) {
          constexpr int idx = decltype(idxc)::value, ss = idx / ND, dt = idx % ND, nx = idx + kAhead;
          if constexpr (nx < 2 * ND) tb[nx % (kAhead + 1)] = rd_tr(Qc, nx % ND, 2 * mq + nx / ND);
          __builtin_amdgcn_sched_barrier(0);
          dk[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(da[ss], tb[idx % (kAhead + 1)], dk[dt], 0, 0, 0);
        };
        StaticFor<0, 2 * ND>::run(acc);
      };
      half(std::integral_constant<int, 0>{});
      half(std::integral_constant<int, 1>{});
    };
    run(tile);
    write_out(dk, g * D, kcol, scale);
  }
}

// dK, dV at D = 128 with one wave per SIMD. A block of four waves owns 128
// keys of one kv head (32 per wave: K and V fragments in registers, dK and dV
// accumulators) and walks, for every query head of the group, the 32-query
// tiles at or after its first key ("items"), as a software pipeline over
// eight LDS stages of Q, dO and the items' lse and rowsum(dO O). Iteration i
// runs two MFMA phases: A, the dV and dK products of item i - 1; B, the S^T
// and dP^T products of item i + 1. Between those MFMAs run item i's
// probabilities, causal mask, dS and bf16 conversions, so that one wave's
// MFMA and VALU work overlap. (Two waves sharing a SIMD, one computing while
// the other multiplies, overlap poorly: a SIMD running an MFMA wave beside a
// VALU wave issued MFMAs at about a third of their rate.)
// One barrier per iteration, ahead of phase A's last two groups: before it
// each wave waits for its direct loads of item i + 1's stage; after it, item
// i - 1's stage is free and takes item i + 7's loads (six iterations to land).
// With one wave per SIMD every instruction takes an issue slot of about 4
// cycles, and an MFMA 32: the loop spends about 10 instructions per MFMA
// (operand reads, the arithmetic, scalar address updates), so it is bound by
// issue and, at the matrix cores' power draw, by the clock more than by the
// matrix cores themselves. Measured on the 7B launch: 12 % fewer cycles than
// attn_bwd_dkdv_pair, at a clock about as much lower, the same time.
// Edges without branches: item -1's stage is zeroed and its P and dS are
// zeros (its products add +0.0 to zeroed accumulators); items past the last
// reload the last one (finite data); the iterations past the last item (one
// to run its dV, dK products, then padding to a whole round of stages) mask
// every probability of theirs, so their P and dS are zeros.
// Every accumulator sums the products of attn_bwd_dkdv in the same order, so
// the results are the same bits.
template <int D>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void attn_bwd_dkdv_pipe(
    const uint16_t* __restrict__ qkv, int64_t ld, const uint16_t* __restrict__ dout, int64_t ldo,
    const float* __restrict__ lse, const float* __restrict__ dsum, int S, int Hq, int Hkv,
    float scale, uint16_t* __restrict__ dqkv, int hsplit, float* __restrict__ part) {
  static_assert(D == 128, "eight 17 KB stages, one wave per SIMD");
  constexpr int NS = D / 16, ND = D / 32;
  constexpr int IQ = 32;               // queries per item
  constexpr int TILE = IQ * D * 2;     // Q or dO rows of an item
  constexpr int LDW = 64 * 4;          // one wave's copy of the item's lse (32) and rowsum (32)
  constexpr int STAGE = 2 * TILE + 4 * LDW;
  constexpr int NST = 8;               // stages
  constexpr int AHEAD = NST - 1;       // iteration i loads item i + AHEAD
  constexpr int NLD = 5;               // direct loads per wave and item: 2 Q, 2 dO, 1 lse / rowsum
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  // One array per stage: reads of a stage wait only for direct loads into it.
  __shared__ __attribute__((aligned(1024))) uint8_t St0[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t St1[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t St2[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t St3[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t St4[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t St5[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t St6[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t St7[STAGE];
  const int kb = blockIdx.z, g = blockIdx.x / hsplit, hs = blockIdx.x % hsplit, b = blockIdx.y;
  const int G = Hq / Hkv;
  const int h_lo = hs * G / hsplit, h_hi = (hs + 1) * G / hsplit;
  const int hq0 = g * G + h_lo;
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int k0w = kb * QB + wave * 32;
  const int kj = k0w + l32;  // this lane's key
  const int64_t tok0 = static_cast<int64_t>(b) * S;
  const int kcol = (Hq + g) * D, vcol = (Hq + Hkv + g) * D;
  const float scale_log2 = scale * kLog2e;
  const int first_q = kb * QB;
  const int nqt = (S - first_q) / IQ;  // items per query head
  const int n_items = (h_hi - h_lo) * nqt;

  auto stage = [&](auto c) -> uint8_t* {
    constexpr int k = decltype(c)::value % NST;
    if constexpr (k == 0) return St0;
    else if constexpr (k == 1) return St1;
    else if constexpr (k == 2) return St2;
    else if constexpr (k == 3) return St3;
    else if constexpr (k == 4) return St4;
    else if constexpr (k == 5) return St5;
    else if constexpr (k == 6) return St6;
    else return St7;
  };

  // Direct loads of item i (clamped to the last) into a stage. Q and dO rows
  // as dma_rowtile: instruction k of this wave fills rows 16 k + 4 wave +
  // (0..3); lane l covers row 4 wave + l / 16 (mod 16) at physical chunk
  // l % 16, a byte offset within those rows that does not depend on k (the
  // swizzle repeats every 16 rows), so one register per source and a uniform
  // base. The lse and rowsum of the item's queries go to this wave's own copy.
  constexpr int CPR = D / 8;
  uint32_t dq_off, do_off;
  {
    const int sub = lane / CPR, row = 4 * wave + sub;
    const int c = (lane % CPR) ^ swz_bits<D>(row);
    dq_off = static_cast<uint32_t>(sub * ld * 2 + c * 16);
    do_off = static_cast<uint32_t>(sub * ldo * 2 + c * 16);
  }
  const float* const ld_src = h ? dsum : lse;
  // The item whose stage loads next, walked in item order and held at the
  // last one: its index, its query tile within its head, the byte addresses
  // of its first Q and dO rows (at the head's column) and the index of its
  // first lse / rowsum value. Advanced by scalar adds, so that each iteration
  // spends a few scalar instructions on its loads rather than the divisions
  // and 64-bit products of computing the addresses afresh.
  struct Cursor {
    int i, t;
    const char* q;
    const char* o;
    int64_t at;
  };
  const int64_t q_row = 2 * IQ * ld, o_row = 2 * IQ * ldo;                   // next tile
  const int64_t q_head = 2 * D - (nqt - 1) * q_row, o_head = 2 * D - (nqt - 1) * o_row;  // next head
  const int64_t at_head = S - (nqt - 1) * static_cast<int64_t>(IQ);
  Cursor cur{0, 0,
             reinterpret_cast<const char*>(qkv + (tok0 + first_q) * ld + static_cast<int64_t>(hq0) * D),
             reinterpret_cast<const char*>(dout + (tok0 + first_q) * ldo + static_cast<int64_t>(hq0) * D),
             (static_cast<int64_t>(b) * Hq + hq0) * S + first_q};
  auto advance = [&](Cursor& c) __attribute__((always_inline)) {
    const bool more = c.i < n_items - 1, wrap = c.t == nqt - 1;
    c.q += more ? (wrap ? q_head : q_row) : 0;
    c.o += more ? (wrap ? o_head : o_row) : 0;
    c.at += more ? (wrap ? at_head : IQ) : 0;
    c.t = more ? (wrap ? 0 : c.t + 1) : c.t;
    c.i += more ? 1 : 0;
  };
  // Q rows (k = 0, 1: rows 16 k + 4 wave + 0..3), dO rows (k = 2, 3), lse / rowsum (k = 4)
  const int64_t q_k[2] = {4 * wave * 2 * ld, (16 + 4 * wave) * 2 * ld};
  const int64_t o_k[2] = {4 * wave * 2 * ldo, (16 + 4 * wave) * 2 * ldo};
  auto dma = [&](const Cursor& c, uint8_t* st, int k) __attribute__((always_inline)) {
    if (k < 4) {
      const int rb = (4 * (k & 1) + wave) * 4;
      const char* base = k < 2 ? c.q + q_k[k & 1] : c.o + o_k[k & 1];
      __builtin_amdgcn_global_load_lds((const gbl_void_t*)(base + (k < 2 ? dq_off : do_off)),
                                       (lds_void_t*)(st + (k >> 1) * TILE + rb * (2 * D)), 16, 0, 0);
    } else {
      __builtin_amdgcn_global_load_lds((const gbl_void_t*)(ld_src + c.at + l32),
                                       (lds_void_t*)(st + 2 * TILE + wave * LDW), 4, 0, 0);
    }
  };

  // Lane offsets of the operand reads, as in attn_bwd_dkdv.
  uint32_t row_off[NS], tr_off[2][ND];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    row_off[s] = rowtile_off<D>(l32, 2 * s + h);
    asm volatile("" : "+v"(row_off[s]));
  }
#pragma unroll
  for (int hv = 0; hv < 2; ++hv)
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
      const int q = (lane >> 4) & 1, li = lane & 15;
      tr_off[hv][dt] = rowtile_off<D>(4 * h + (li >> 2) + 8 * hv, (dt * 32 + q * 16) / 8 + ((li & 3) >> 1)) +
                       (li & 1) * 8;
      asm volatile("" : "+v"(tr_off[hv][dt]));
    }
  auto rd_row = [&](const uint8_t* t, int s) -> bf16x8 {
    return *(const lds_bf16x8_t*)((lds_cptr)t + row_off[s]);
  };
  auto rd_tr = [&](const uint8_t* t, int dt, int s) -> bf16x8 {
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)((lds_cptr)t + tr_off[0][dt] + s * 16 * (2 * D)));
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)((lds_cptr)t + tr_off[1][dt] + s * 16 * (2 * D)));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  // prologue: K, V fragments; items 0 .. AHEAD - 1 to stages 0 .. AHEAD - 1;
  // item -1's stage (NST - 1) zeroed
  bf16x8 kf[NS], vf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    kf[s] = *reinterpret_cast<const bf16x8*>(qkv + (tok0 + kj) * ld + kcol + s * 16 + h * 8);
    vf[s] = *reinterpret_cast<const bf16x8*>(qkv + (tok0 + kj) * ld + vcol + s * 16 + h * 8);
  }
  // The prologue's loads stay in stage order (the waits below count them).
  __builtin_amdgcn_sched_barrier(0);
  // A direct load into the last stage's lse / rowsum copy first (item 0's:
  // never read), so that the compiler meets every stage's loads before the
  // loop; its waits for them then stay exact inside it.
  dma(cur, St7, NLD - 1);
  __builtin_amdgcn_sched_barrier(0);
  auto pro_load = [&](auto jc) __attribute__((always_inline)) {
    constexpr int j = decltype(jc)::value;
#pragma unroll
    for (int k = 0; k < NLD; ++k) dma(cur, stage(Ic<j>{}), k);
    advance(cur);
    __builtin_amdgcn_sched_barrier(0);
  };
  StaticFor<0, AHEAD>::run(pro_load);
  __builtin_amdgcn_sched_barrier(0);
  for (int c = threadIdx.x; c < 2 * TILE / 16; c += kThreads)
    reinterpret_cast<u32x4_t*>(St7)[c] = u32x4_t{0u, 0u, 0u, 0u};
  f32x16 dk[ND], dv[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) {
    dk[dt] = f32x16{};
    dv[dt] = f32x16{};
  }
  f32x16 sf[2], df[2];  // S^T and dP^T of an item: [set]
  // item 0 landed (the later stages may be in flight), the zeros written
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(NLD * (AHEAD - 1) + 1));
  __builtin_amdgcn_s_barrier();
  // S^T, dP^T of item 0 (set 0)
  sf[0] = f32x16{};
  df[0] = f32x16{};
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    sf[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(rd_row(St0, s), kf[s], sf[0], 0, 0, 0);
    df[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(rd_row(St0 + TILE, s), vf[s], df[0], 0, 0, 0);
  }
  // Operand reads run two groups ahead of their MFMAs (a ring of three):
  // one group (about 64 cycles) is shorter than an LDS read's latency with
  // four waves reading.
  bf16x8 ta[3], tb[3];   // dO^T and Q^T operands of phase A
  bf16x8 qa[3], oa[3];   // Q and dO row operands of phase B
  f32x4 lq4[2], dq4[2];  // lse (log2 domain) and rowsum of four queries, ahead of use
  ta[0] = rd_tr(St7 + TILE, 0, 0);
  tb[0] = rd_tr(St7, 0, 0);
  ta[1] = rd_tr(St7 + TILE, 1, 0);
  tb[1] = rd_tr(St7, 1, 0);
  const int lim0 = kj - 4 * h;

  // Item i's arithmetic as a three-stage pipeline over the iteration's 16
  // MFMA groups G (phase A: G = 0..7, phase B: G = 8..15): value v goes
  // through stage 1 (S scaled, minus lse) in group v + 2, stage 2 (exp2, dP
  // minus rowsum) in v + 3 and stage 3 (causal mask, dS, and with its odd
  // neighbour the bf16 pair) in v + 4; the last values finish in the next
  // iteration's first groups, ahead of the phase A products that read them.
  // Each group then runs three short independent chains (a dependent VALU
  // step waits about 8 cycles on the one before).
  // P and dS as bf16 operands, packed pairs: [set][k16 step of the item][pair]
  uint32_t pw[2][2][4], dw[2][2][4];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int w = 0; w < 4; ++w) pw[1][kk][w] = dw[1][kk][w] = 0u;  // item -1
  // (zeros before item 0: item -1's values finish in iteration 0 as zeros)
  float xs[16], es[16], ts[16], ps[16], dss[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) xs[v] = es[v] = ts[v] = ps[v] = dss[v] = 0.0f;
  int lim_p = 0x7fffffff;  // item -1: every value masked (its P, dS are zeros)
  int tc = 0;              // item i's query tile within its head
  sf[1] = f32x16{};
  df[1] = f32x16{};
  lq4[0] = lq4[1] = dq4[0] = dq4[1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  auto pack = [](float a, float b) -> uint32_t {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(mr_f32x2{a, b}, bf16x2_t));
  };
  auto st1 = [&](auto setc, auto vc) __attribute__((always_inline)) {
    constexpr int set = decltype(setc)::value, v = decltype(vc)::value;
    xs[v] = __builtin_fmaf(sf[set][v], scale_log2, -lq4[(v >> 2) & 1][v & 3]);
    asm volatile("" : "+v"(xs[v]));  // computed here, not sunk to its use
  };
  auto st2 = [&](auto setc, auto vc) __attribute__((always_inline)) {
    constexpr int set = decltype(setc)::value, v = decltype(vc)::value;
    es[v] = __builtin_amdgcn_exp2f(xs[v]);
    ts[v] = df[set][v] - dq4[(v >> 2) & 1][v & 3];
    asm volatile("" : "+v"(es[v]), "+v"(ts[v]));
  };
  auto st3 = [&](auto setc, auto vc, int lim) __attribute__((always_inline)) {
    constexpr int set = decltype(setc)::value, v = decltype(vc)::value;
    ps[v] = lim > 8 * (v >> 2) + (v & 3) ? 0.0f : es[v];
    dss[v] = ps[v] * ts[v];
    if constexpr (v & 1) {
      pw[set][v >> 3][(v & 7) >> 1] = pack(ps[v - 1], ps[v]);
      dw[set][v >> 3][(v & 7) >> 1] = pack(dss[v - 1], dss[v]);
      asm volatile("" : "+v"(pw[set][v >> 3][(v & 7) >> 1]), "+v"(dw[set][v >> 3][(v & 7) >> 1]));
    }
  };
  auto opnd = [](const uint32_t (&w)[4]) -> bf16x8 {
    return __builtin_bit_cast(bf16x8, u32x4_t{w[0], w[1], w[2], w[3]});
  };

  auto iter = [&](auto pc, int i) __attribute__((always_inline)) {
    constexpr int P = decltype(pc)::value;
    constexpr int C = P & 1, N = C ^ 1;  // sets of item i and of items i +- 1
    uint8_t* const Sp = stage(Ic<P + NST - 1>{});  // item i - 1; after the barrier, item i + AHEAD's loads
    uint8_t* const Sc = stage(Ic<P>{});             // item i
    uint8_t* const Sn = stage(Ic<P + 1>{});         // item i + 1
    const lds_cptr LDc = (lds_cptr)Sc + 2 * TILE + wave * LDW;
    // Value v of item i is masked iff key kj > query qt0 + acc_row(v, h),
    // i.e. iff lim > 8 (v / 4) + v % 4; every value of the padding items past
    // the last, so that their P and dS are zeros.
    // (branch-free: a branch here splits the loop body, and the compiler then
    // copies the accumulator sets between register files at the join)
    const int lim_c = lim0 - first_q - tc * IQ + (((n_items - 1 - i) >> 31) & (1 << 30));

    auto ldrd = [&](auto gqc) __attribute__((always_inline)) {  // queries 8 gq + 4 h + 0..3
      constexpr int gq = decltype(gqc)::value;
      typedef __attribute__((address_space(3))) f32x4 lds_f32x4_t;
      const lds_cptr l4 = LDc + (gq * 8 + 4 * h) * 4;
      lq4[gq & 1] = *(const lds_f32x4_t*)l4 * kLog2e;
      dq4[gq & 1] = *(const lds_f32x4_t*)(l4 + 32 * 4);
      asm volatile("" : "+v"(lq4[gq & 1]));
    };
    // the arithmetic of group G (see above)
    auto arith = [&](auto gc) __attribute__((always_inline)) {
      constexpr int G = decltype(gc)::value;
      if constexpr (G % 4 == 0) ldrd(Ic<G / 4>{});
      if constexpr (G >= 4) st3(Ic<C>{}, Ic<G - 4>{}, lim_c);
      else st3(Ic<N>{}, Ic<G + 12>{}, lim_p);
      if constexpr (G >= 3) st2(Ic<C>{}, Ic<G - 3>{});
      else st2(Ic<N>{}, Ic<G + 13>{});
      if constexpr (G >= 2) st1(Ic<C>{}, Ic<G - 2>{});
      else st1(Ic<N>{}, Ic<G + 14>{});
    };
    // phase A, group x: k16 step kk = x / ND of item i - 1, d tile dt = x % ND
    auto ga = [&](auto xc) __attribute__((always_inline)) {
      constexpr int x = decltype(xc)::value, kk = x / ND, dt = x % ND;
      if constexpr (x + 2 < 2 * ND) {
        ta[(x + 2) % 3] = rd_tr(Sp + TILE, (x + 2) % ND, (x + 2) / ND);
        tb[(x + 2) % 3] = rd_tr(Sp, (x + 2) % ND, (x + 2) / ND);
      }
      dv[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(opnd(pw[N][kk]), ta[x % 3], dv[dt], 0, 0, 0);
      dk[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(opnd(dw[N][kk]), tb[x % 3], dk[dt], 0, 0, 0);
      arith(Ic<x>{});
      __builtin_amdgcn_sched_barrier(0);
    };
    StaticFor<0, 2 * ND - 2>::run(ga);
    // item i + 1's stage landed (this wave's loads, then everyone's); every
    // wave is past its reads of item i - 1's stage
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(NLD * (AHEAD - 2)));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    qa[0] = rd_row(Sn, 0);
    oa[0] = rd_row(Sn + TILE, 0);
    qa[1] = rd_row(Sn, 1);
    oa[1] = rd_row(Sn + TILE, 1);
    ga(Ic<2 * ND - 2>{});
    ga(Ic<2 * ND - 1>{});
    // phase B, group x: k16 step s = x of item i + 1
    auto gb = [&](auto xc) __attribute__((always_inline)) {
      constexpr int x = decltype(xc)::value;
      if constexpr (x + 2 < NS) {
        qa[(x + 2) % 3] = rd_row(Sn, x + 2);
        oa[(x + 2) % 3] = rd_row(Sn + TILE, x + 2);
      } else {  // the next iteration's first phase A operands: item i's stage
        ta[x - (NS - 2)] = rd_tr(Sc + TILE, x - (NS - 2), 0);
        tb[x - (NS - 2)] = rd_tr(Sc, x - (NS - 2), 0);
      }
      if constexpr (x == 1) dma(cur, Sp, 0);
      if constexpr (x == 2) dma(cur, Sp, 2);
      if constexpr (x == 3) dma(cur, Sp, 1);
      if constexpr (x == 5) dma(cur, Sp, 3);
      if constexpr (x == 6) dma(cur, Sp, 4);
      sf[N] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[x % 3], kf[x], x == 0 ? f32x16{} : sf[N], 0, 0, 0);
      df[N] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(oa[x % 3], vf[x], x == 0 ? f32x16{} : df[N], 0, 0, 0);
      arith(Ic<2 * ND + x>{});
      __builtin_amdgcn_sched_barrier(0);
    };
    StaticFor<0, NS>::run(gb);
    lim_p = lim_c;
    advance(cur);
    tc = tc == nqt - 1 ? 0 : tc + 1;
  };

  // Whole rounds of NST iterations (compile-time stages): n_items + 1
  // iterations and up to NST - 1 padding ones, whose items add zeros.
  const int n_it = (n_items + NST) / NST * NST;
  for (int i = 0; i < n_it; i += NST) {
    iter(Ic<0>{}, i);
    iter(Ic<1>{}, i + 1);
    iter(Ic<2>{}, i + 2);
    iter(Ic<3>{}, i + 3);
    iter(Ic<4>{}, i + 4);
    iter(Ic<5>{}, i + 5);
    iter(Ic<6>{}, i + 6);
    iter(Ic<7>{}, i + 7);
  }
  __builtin_amdgcn_s_waitcnt(0);  // the last (repeated) direct loads

  // dk, dv [dt][r]: key k0w + acc_row(r, h), d = dt * 32 + l32, to the
  // partials ([split][token][k heads | v heads][d]) or as bf16 into dqkv.
  if (part) {
    const int64_t W = 2 * static_cast<int64_t>(Hkv) * D;
    float* pbase = part + static_cast<int64_t>(hs) * gridDim.y * S * W;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = tok0 + k0w + acc_row(r, h);
        pbase[row * W + g * D + dt * 32 + l32] = dk[dt][r] * scale;
        pbase[row * W + (Hkv + g) * D + dt * 32 + l32] = dv[dt][r];
      }
    return;
  }
#pragma unroll
  for (int dt = 0; dt < ND; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = tok0 + k0w + acc_row(r, h);
      dqkv[row * ld + kcol + dt * 32 + l32] = f32_to_bf16(dk[dt][r] * scale);
      dqkv[row * ld + vcol + dt * 32 + l32] = f32_to_bf16(dv[dt][r]);
    }
}

// dK, dV of head-split blocks: the sum of the partials in split order, as
// bf16 into the k and v columns of dqkv. One thread per 4 consecutive values.
__global__ __launch_bounds__(kThreads) void attn_bwd_kv_reduce(const float* __restrict__ part,
                                                              int hsplit, int64_t T, int64_t W,
                                                              int64_t col0, uint16_t* __restrict__ dqkv,
                                                              int64_t ld) {
  const int64_t e = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * 4;
  if (e >= T * W) return;
  float4 acc = *reinterpret_cast<const float4*>(part + e);
  for (int sp = 1; sp < hsplit; ++sp) {
    const float4 v = *reinterpret_cast<const float4*>(part + sp * T * W + e);
    acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
  }
  const int64_t row = e / W, c = e % W;
  const uint32_t lo = pack_bf16x2(acc.x, acc.y);
  const uint32_t hi = pack_bf16x2(acc.z, acc.w);
  *reinterpret_cast<uint2*>(dqkv + row * ld + col0 + c) = make_uint2(lo, hi);
}

// dQ: queries along lanes; a block owns 128 queries of one query head and
// walks the key tiles up to its last query, K and V arriving by direct loads,
// double buffered. dQ^T = K^T dS^T takes K^T from the transposing LDS read.
// With out non-null it also forms D = rowsum(dO O) of its queries (the bits
// attn_bwd_dot gives) and writes it to dsum for the dK/dV kernel that follows;
// else it reads dsum.
template <int D>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void attn_bwd_dq(
    const uint16_t* __restrict__ qkv, int64_t ld, const uint16_t* __restrict__ dout, int64_t ldo,
    const float* __restrict__ lse, float* __restrict__ dsum, int S, int Hq, int Hkv,
    float scale, uint16_t* __restrict__ dqkv, const uint16_t* __restrict__ out) {
  constexpr int NS = D / 16, ND = D / 32;
  constexpr int TILE = KT * D * 2;
  __shared__ __attribute__((aligned(1024))) uint8_t K0[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t V0[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t K1[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t V1[TILE];
  const int qb = gridDim.z - 1 - blockIdx.z;  // the longest blocks start first
  const int hq = blockIdx.x, b = blockIdx.y;
  const int g = hq / (Hq / Hkv);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
  const int q0 = qb * QB + wave * 32;
  const int qi = q0 + l32;
  const int64_t tok0 = static_cast<int64_t>(b) * S;
  const int kcol = (Hq + g) * D, vcol = (Hq + Hkv + g) * D;
  const float scale_log2 = scale * kLog2e;
  const int n_tiles = (qb + 1) * QB / KT;

  dma_rowtile<D>(qkv, ld, tok0, kcol, K0);
  dma_rowtile<D>(qkv, ld, tok0, vcol, V0);
  const float lse2 = lse[(static_cast<int64_t>(b) * Hq + hq) * S + qi] * kLog2e;
  bf16x8 qf[NS], of[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    qf[s] = *reinterpret_cast<const bf16x8*>(qkv + (tok0 + qi) * ld + hq * D + s * 16 + h * 8);
    of[s] = *reinterpret_cast<const bf16x8*>(dout + (tok0 + qi) * ldo + hq * D + s * 16 + h * 8);
  }
  float dq_sum;
  if (out) {
    // attn_bwd_dot's lane `sub` sums the 8 products of dO and O at d = 8 sub
    // .. 8 sub + 7 in order, then a butterfly over its D / 8 lanes adds the
    // pieces (sub ^ D/16, ..., sub ^ 1). Here piece sub = 2 s + h is piece s
    // of this lane: the same sums, the butterfly's steps over s in registers
    // and its last step (h) across the lane halves. Every lane of a butterfly
    // ends with the same bits (each pair is added the same way up to order).
    float pd[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
      const u32x4v a = __builtin_bit_cast(u32x4v, of[s]);
      const u32x4v o = *reinterpret_cast<const u32x4v*>(out + (tok0 + qi) * ldo + hq * D + s * 16 + h * 8);
      const uint32_t aw[4] = {a[0], a[1], a[2], a[3]}, ow[4] = {o[0], o[1], o[2], o[3]};
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc += __uint_as_float(aw[k] << 16) * __uint_as_float(ow[k] << 16);
        acc += __uint_as_float(aw[k] & 0xffff0000u) * __uint_as_float(ow[k] & 0xffff0000u);
      }
      pd[s] = acc;
    }
#pragma unroll
    for (int o = NS / 2; o >= 1; o >>= 1)
#pragma unroll
      for (int s = 0; s < o; ++s) pd[s] = pd[s] + pd[s + o];
    dq_sum = pd[0] + __shfl_xor(pd[0], 32, 64);
    if (h == 0) dsum[(static_cast<int64_t>(b) * Hq + hq) * S + qi] = dq_sum;
  } else {
    dq_sum = dsum[(static_cast<int64_t>(b) * Hq + hq) * S + qi];
  }
  f32x16 dq[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) dq[dt] = f32x16{};

  auto step = [&](int t, const uint8_t* Kc, const uint8_t* Vc, uint8_t* Kn, uint8_t* Vn) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t + 1 < n_tiles) {
      dma_rowtile<D>(qkv, ld, tok0 + (t + 1) * KT, kcol, Kn);
      dma_rowtile<D>(qkv, ld, tok0 + (t + 1) * KT, vcol, Vn);
    }
    const int kv0 = t * KT;
    if (kv0 > q0 + 31) return;
    const bool diag = kv0 + KT - 1 > q0;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {  // 32 keys at a time: S^T, dP^T, then their dQ share
      if (kv0 + mt * 32 > q0 + 31) break;
      f32x16 st = f32x16{}, dpt = f32x16{};
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_row<D>(Kc, mt * 32 + l32, s, h), qf[s], st,
                                                     0, 0, 0);
        dpt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_row<D>(Vc, mt * 32 + l32, s, h), of[s], dpt,
                                                      0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = __builtin_amdgcn_exp2f(__builtin_fmaf(st[r], scale_log2, -lse2));
        if (diag && kv0 + mt * 32 + acc_row(r, h) > qi) p = 0.0f;
        st[r] = p * (dpt[r] - dq_sum);  // dS^T
      }
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) {
        const bf16x8 db = cvt8(st, 8 * ss);
#pragma unroll
        for (int dt = 0; dt < ND; ++dt)
          dq[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_tr<D>(Kc, dt * 32, 2 * mt + ss, lane), db,
                                                           dq[dt], 0, 0, 0);
      }
    }
  };

  int t = 0;
  for (; t + 1 < n_tiles; t += 2) {
    step(t, K0, V0, K1, V1);
    step(t + 1, K1, V1, K0, V0);
  }
  if (t < n_tiles) step(t, K0, V0, K1, V1);
  __syncthreads();
  uint8_t* stage = wave == 0 ? K0 : wave == 1 ? V0 : wave == 2 ? K1 : V1;
  store_qrows<D>(dq, scale, stage, dqkv + hq * D, ld, tok0 + q0);
}

// Grids put the query (or key) block index in z, the slowest dimension:
// workgroups go to the 8 XCDs round-robin by linear id, so heads x batches
// (x, y) spread each causal length class evenly over the XCDs, and z in
// decreasing work order starts the longest blocks first.
template <int D>
int launch_fwd(const uint16_t* qkv, int64_t ld, int B, int S, int Hq, int Hkv, float scale,
               uint16_t* out, int64_t ldo, float* lse, hipStream_t s) {
  if (S % 256 == 0)
    hipLaunchKernelGGL((attn_fwd<D, 8>), dim3(Hq, B, S / 256), dim3(512), 0, s, qkv, nullptr, ld, S, Hq, Hkv,
                       scale * kLog2e, out, ldo, nullptr, 0, lse);
  else
    hipLaunchKernelGGL((attn_fwd<D, 4>), dim3(Hq, B, S / 128), dim3(256), 0, s, qkv, nullptr, ld, S, Hq, Hkv,
                       scale * kLog2e, out, ldo, nullptr, 0, lse);
  MR_LAUNCH_CHECK("mr_attn_fwd");
  return MR_OK;
}

template <int D>
int launch_fwd_split(const uint16_t* qkv, const uint16_t* qkv_lo, int64_t ld, int B, int S, int Hq, int Hkv,
                     float scale, uint16_t* out, int64_t ldo, uint16_t* out_split, int64_t ld_split, float* lse,
                     hipStream_t s) {
  hipLaunchKernelGGL((attn_fwd<D, 4, true>), dim3(Hq, B, S / 128), dim3(256), 0, s, qkv, qkv_lo, ld, S, Hq, Hkv,
                     scale * kLog2e, out, ldo, out_split, ld_split, lse);
  MR_LAUNCH_CHECK("mr_attn_fwd_split");
  return MR_OK;
}

// Grids of few key blocks (short sequences, few kv heads, small batches)
// leave CUs idle and put the long causal first blocks on the critical path:
// then each kv head's query heads are split over several blocks, up to
// kKvTargetBlocks blocks, whose fp32 dK/dV partials live in the caller's
// workspace. Measured: 1.3x on 8 x 2048 tokens with 2 kv heads, 3.4x on
// 2 x 1024; a grid already at 512 blocks (4 kv heads) loses to the partials'
// traffic.
constexpr int64_t kKvTargetBlocks = 512;
constexpr int64_t kKvPartCapBytes = 128ll << 20;

int64_t kv_part_bytes(int B, int S, int Hkv, int D, int hsplit) {
  return hsplit > 1 ? static_cast<int64_t>(hsplit) * B * S * 2 * Hkv * D * 4 : 0;
}

// The automatic split: the smallest that reaches kKvTargetBlocks blocks (or
// all G query heads), with its partials within cap bytes.
int auto_hsplit(int B, int S, int Hq, int Hkv, int D, int64_t cap) {
  const int G = Hq / Hkv;
  const int64_t blocks = static_cast<int64_t>(Hkv) * B * (S / QB);
  int hsplit = 1;
  while (hsplit < G && blocks * hsplit < kKvTargetBlocks && kv_part_bytes(B, S, Hkv, D, hsplit + 1) <= cap)
    ++hsplit;
  return hsplit;
}

// MR_ATTN_PAIR=1 in the environment runs dK, dV at D = 128 on
// attn_bwd_dkdv_pair instead of attn_bwd_dkdv_pipe (read at every launch;
// the two give the same bits, which the tests check).
bool use_pair_kernel() {
  const char* e = getenv("MR_ATTN_PAIR");
  return e && e[0] == '1';
}

template <int D>
int launch_bwd(const uint16_t* qkv, int64_t ld, const uint16_t* out, const uint16_t* dout,
               int64_t ldo, const float* lse, float* dsum, int B, int S, int Hq, int Hkv,
               float scale, uint16_t* dqkv, int hsplit, float* part, hipStream_t s) {
  const int64_t T = static_cast<int64_t>(B) * S;
  // The dQ kernel forms D = rowsum(dO O) and leaves it in dsum for the dK/dV
  // kernel, which therefore runs second. MR_ATTN_DOT=1: D by attn_bwd_dot
  // first and dQ last, as before (the same bits, for comparisons).
  const char* e = getenv("MR_ATTN_DOT");
  const bool dot_first = e && e[0] == '1';
  if (dot_first) {
    const int64_t lanes = T * Hq * (D / 8);
    hipLaunchKernelGGL(attn_bwd_dot<D>, dim3(static_cast<unsigned>((lanes + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, s, dout, out, ldo, T, S, Hq, dsum);
  } else {
    hipLaunchKernelGGL(attn_bwd_dq<D>, dim3(Hq, B, S / QB), dim3(kThreads), 0, s, qkv, ld, dout, ldo,
                       lse, dsum, S, Hq, Hkv, scale, dqkv, out);
  }
  const int64_t W = 2 * static_cast<int64_t>(Hkv) * D;
  if (hsplit == 1) part = nullptr;
  if constexpr (D == 128) {
    if (use_pair_kernel())
      hipLaunchKernelGGL(attn_bwd_dkdv_pair<D>, dim3(Hkv * hsplit, B, S / QB), dim3(2 * kThreads), 0, s, qkv,
                         ld, dout, ldo, lse, dsum, S, Hq, Hkv, scale, dqkv, hsplit, part);
    else
      hipLaunchKernelGGL(attn_bwd_dkdv_pipe<D>, dim3(Hkv * hsplit, B, S / QB), dim3(kThreads), 0, s, qkv,
                         ld, dout, ldo, lse, dsum, S, Hq, Hkv, scale, dqkv, hsplit, part);
  } else
    hipLaunchKernelGGL(attn_bwd_dkdv<D>, dim3(Hkv * hsplit, B, S / QB), dim3(kThreads), 0, s, qkv, ld,
                       dout, ldo, lse, dsum, S, Hq, Hkv, scale, dqkv, hsplit, part);
  if (part) {
    const int64_t threads = T * W / 4;
    hipLaunchKernelGGL(attn_bwd_kv_reduce, dim3(static_cast<unsigned>((threads + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, s, part, hsplit, T, W, static_cast<int64_t>(Hq) * D, dqkv, ld);
  }
  if (dot_first)
    hipLaunchKernelGGL(attn_bwd_dq<D>, dim3(Hq, B, S / QB), dim3(kThreads), 0, s, qkv, ld, dout, ldo,
                       lse, dsum, S, Hq, Hkv, scale, dqkv, static_cast<const uint16_t*>(nullptr));
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

// Byte span of `rows` rows of `width` bf16 values at leading dimension ld.
int64_t span(int64_t rows, int64_t ld, int64_t width) { return ((rows - 1) * ld + width) * 2; }

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
  const int64_t T = static_cast<int64_t>(B) * S;
  if (overlap(out, span(T, ldo, static_cast<int64_t>(Hq) * head_dim), qkv,
              span(T, ld, static_cast<int64_t>(Hq + 2 * Hkv) * head_dim)))
    return fail(MR_EINVAL, "mr_attn_fwd: out must not overlap qkv");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* q = static_cast<const uint16_t*>(qkv);
  uint16_t* o = static_cast<uint16_t*>(out);
  if (head_dim == 128) return launch_fwd<128>(q, ld, B, S, Hq, Hkv, scale, o, ldo, lse, s);
  return launch_fwd<64>(q, ld, B, S, Hq, Hkv, scale, o, ldo, lse, s);
}

int mr_attn_fwd_split(const void* qkv_hi, const void* qkv_lo, int64_t ld, int B, int S, int Hq, int Hkv,
                      int head_dim, float scale, void* out, int64_t ldo, void* out_split, int64_t ld_split,
                      float* lse, void* stream) {
  using namespace mr;
  clear_error();
  int rc = check("mr_attn_fwd_split", qkv_hi, ld, B, S, Hq, Hkv, head_dim, ldo);
  if (rc) return rc;
  if (!qkv_lo || !aligned16(qkv_lo)) return fail(MR_EINVAL, "mr_attn_fwd_split: qkv_lo must be 16-byte aligned");
  if (!out || !lse || !out_split || !aligned16(out) || !aligned16(out_split))
    return fail(MR_EINVAL, "mr_attn_fwd_split: bad output");
  if (ld_split < 3ll * Hq * head_dim || ld_split % 8)
    return fail(MR_EINVAL, "mr_attn_fwd_split: out_split rows must hold 3 Hq head_dim values (ld a multiple of 8)");
  {
    const int64_t T = static_cast<int64_t>(B) * S;
    const int64_t n_qkv = span(T, ld, static_cast<int64_t>(Hq + 2 * Hkv) * head_dim);
    const int64_t n_o = span(T, ldo, static_cast<int64_t>(Hq) * head_dim);
    const int64_t n_s = span(T, ld_split, 3ll * Hq * head_dim);
    if (overlap(out, n_o, qkv_hi, n_qkv) || overlap(out, n_o, qkv_lo, n_qkv) || overlap(out_split, n_s, qkv_hi, n_qkv) ||
        overlap(out_split, n_s, qkv_lo, n_qkv) || overlap(out, n_o, out_split, n_s))
      return fail(MR_EINVAL, "mr_attn_fwd_split: out and out_split must not overlap qkv or each other");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* qh = static_cast<const uint16_t*>(qkv_hi);
  const uint16_t* ql = static_cast<const uint16_t*>(qkv_lo);
  uint16_t* o = static_cast<uint16_t*>(out);
  uint16_t* os = static_cast<uint16_t*>(out_split);
  if (head_dim == 128) return launch_fwd_split<128>(qh, ql, ld, B, S, Hq, Hkv, scale, o, ldo, os, ld_split, lse, s);
  return launch_fwd_split<64>(qh, ql, ld, B, S, Hq, Hkv, scale, o, ldo, os, ld_split, lse, s);
}

size_t mr_attn_bwd_workspace_bytes(int B, int S, int Hq, int Hkv, int head_dim, int hsplit) {
  using namespace mr;
  if (B <= 0 || S <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || (head_dim != 64 && head_dim != 128))
    return 0;
  const int h = hsplit > 0 ? hsplit : auto_hsplit(B, S, Hq, Hkv, head_dim, kKvPartCapBytes);
  return static_cast<size_t>(kv_part_bytes(B, S, Hkv, head_dim, h));
}

int mr_attn_bwd(const void* qkv, int64_t ld, const void* out, const void* dout, int64_t ldo,
                const float* lse, float* dsum_ws, int B, int S, int Hq, int Hkv, int head_dim,
                float scale, void* dqkv, int hsplit, void* workspace, size_t workspace_bytes,
                void* stream) {
  using namespace mr;
  clear_error();
  int rc = check("mr_attn_bwd", qkv, ld, B, S, Hq, Hkv, head_dim, ldo);
  if (rc) return rc;
  if (!out || !dout || !lse || !dsum_ws || !dqkv || !aligned16(out) || !aligned16(dout) ||
      !aligned16(dqkv))
    return fail(MR_EINVAL, "mr_attn_bwd: bad argument");
  {
    // dQ is written while the dK/dV kernel, launched after it, still reads
    // q, k, v, O and dO, and the row sums while the dQ kernel reads them:
    // the outputs must not share memory with the inputs or each other
    const int64_t T = static_cast<int64_t>(B) * S;
    const int64_t n_qkv = span(T, ld, static_cast<int64_t>(Hq + 2 * Hkv) * head_dim);
    const int64_t n_o = span(T, ldo, static_cast<int64_t>(Hq) * head_dim);
    const int64_t n_sum = T * Hq * static_cast<int64_t>(sizeof(float));
    if (overlap(dqkv, n_qkv, qkv, n_qkv) || overlap(dqkv, n_qkv, out, n_o) || overlap(dqkv, n_qkv, dout, n_o) ||
        overlap(dsum_ws, n_sum, qkv, n_qkv) || overlap(dsum_ws, n_sum, out, n_o) ||
        overlap(dsum_ws, n_sum, dout, n_o) || overlap(dsum_ws, n_sum, dqkv, n_qkv))
      return fail(MR_EINVAL, "mr_attn_bwd: dqkv and dsum_ws must not overlap qkv, out, dout or each other");
  }
  const int G = Hq / Hkv;
  if (hsplit < 0 || hsplit > G)
    return fail(MR_EINVAL, "mr_attn_bwd: hsplit %d outside [0, %d] (0 = automatic)", hsplit, G);
  if (workspace && !aligned16(workspace))
    return fail(MR_EINVAL, "mr_attn_bwd: workspace must be 16-byte aligned");
  const int64_t have = workspace ? static_cast<int64_t>(workspace_bytes) : 0;
  if (hsplit == 0) {
    hsplit = auto_hsplit(B, S, Hq, Hkv, head_dim, have < kKvPartCapBytes ? have : kKvPartCapBytes);
  } else if (kv_part_bytes(B, S, Hkv, head_dim, hsplit) > have) {
    return fail(MR_EINVAL, "mr_attn_bwd: hsplit %d needs a %lld-byte workspace, %lld given", hsplit,
                static_cast<long long>(kv_part_bytes(B, S, Hkv, head_dim, hsplit)),
                static_cast<long long>(have));
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* q = static_cast<const uint16_t*>(qkv);
  const uint16_t* o = static_cast<const uint16_t*>(out);
  const uint16_t* dO = static_cast<const uint16_t*>(dout);
  uint16_t* dq = static_cast<uint16_t*>(dqkv);
  float* part = static_cast<float*>(workspace);
  if (head_dim == 128)
    return launch_bwd<128>(q, ld, o, dO, ldo, lse, dsum_ws, B, S, Hq, Hkv, scale, dq, hsplit, part, s);
  return launch_bwd<64>(q, ld, o, dO, ldo, lse, dsum_ws, B, S, Hq, Hkv, scale, dq, hsplit, part, s);
}

}  // extern "C"
