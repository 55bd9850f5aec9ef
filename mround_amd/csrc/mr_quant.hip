// Fake quantization (forward) and its straight-through backward fused with the
// sign-SGD step, for gfx950.
//
// Arithmetic follows the reference's float32 operation order exactly
// (mround/reference/quantize.py:156-319 forward, 370-522 backward; the
// round-to-nearest shortcut of mround/core/quantizer.py:269-284): correctly
// rounded quotients (IEEE division, or the exact reciprocal-and-correction
// forms of div_maxq() and quotients() where those are proven exact), round
// half to even (rintf), no contraction into fused multiply-adds (this file is
// built with -ffp-contract=off). Codes and reconstructions are therefore
// bit-identical to a float32 evaluation of the reference's formulas; only the
// per-group sums of the backward differ, by summation order.
//
// Two launch shapes:
//   fast    each lane owns 8 consecutive weights; a group of gs weights spans
//           gs/8 adjacent lanes (a power of two <= 64) and its min/max and
//           gradient sums are xor-butterfly reductions over those lanes, so
//           every lane of the group ends with bit-identical group values.
//           One wave streams 8 * 64 weights with 16-byte loads: W, v and the
//           outputs are read and written exactly once (HBM-bound).
//   generic one wave per group, strided over the group; covers per-channel
//           groups, padded last groups and fp16 inputs.
#include <cmath>

#include "mr_common.h"

namespace mr {
namespace {

constexpr int kBlock = 256;

// Row placement of the reconstruction (forward) or of the gradient (backward)
// inside a larger row-major buffer with the same column count: row r lives at
// (r / blk) * stride + off + r % blk; blk == 0 is the identity.
// n / d for 0 <= n < 2^31 and a divisor d >= 1 fixed per launch: with
// l = ceil(log2 d), p = 31 + l and m = ceil(2^p / d) < 2^32, floor(n * m / 2^p)
// equals floor(n / d), because n * m / 2^p exceeds n / d by less than
// 2^31 / 2^p = 2^-l <= 1 / d. One 32 x 32 -> 64-bit multiply and a shift
// instead of an integer division.
struct FastDiv {
  uint32_t m = 0;
  int p = 0;
  static FastDiv make(uint32_t d) {
    FastDiv f;
    int l = 0;
    while ((uint64_t{1} << l) < d) ++l;
    f.p = 31 + l;
    f.m = static_cast<uint32_t>(((uint64_t{1} << f.p) + d - 1) / d);
    return f;
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    return static_cast<uint32_t>((static_cast<uint64_t>(n) * m) >> p);
  }
};

struct RowMap {
  int64_t blk, stride, off;
  int cpr;              // 8-element chunks per row (fast kernels)
  FastDiv by_cpr, by_blk;  // set on the host by prepare() (fast kernels)
  __device__ __forceinline__ int64_t row(int64_t r) const {
    return blk ? (r / blk) * stride + off + r % blk : r;
  }
  // The fast kernels' constants for `cols` columns; mapped launches have
  // fewer than 2^31 chunks, so chunk and row indices fit 31 bits.
  void prepare(int64_t cols) {
    cpr = static_cast<int>(cols / 8);
    if (blk && cpr > 0) {  // (narrower rows take the generic kernels, which divide)
      by_cpr = FastDiv::make(static_cast<uint32_t>(cpr));
      by_blk = FastDiv::make(static_cast<uint32_t>(blk));
    }
  }
  // Element index of chunk `chunk` (8 elements) under the placement.
  __device__ __forceinline__ int64_t chunk_elem(int64_t chunk) const {
    if (!blk) return chunk * 8;
    const uint32_t c = static_cast<uint32_t>(chunk);
    const uint32_t r = by_cpr.div(c);
    const uint32_t col = c - r * static_cast<uint32_t>(cpr);
    const uint32_t rb = by_blk.div(r);
    const uint32_t rr = r - rb * static_cast<uint32_t>(blk);
    return ((static_cast<int64_t>(rb) * stride + off + rr) * cpr + col) * 8;
  }
};

struct Group {
  float s;         // scale (signed under the symmetric modes)
  float zp;        // zero point (asymmetric)
  float wmax_raw;  // max(max(W_g), 0)
  float wmin_raw;  // min(min(W_g), 0)
  float wmin;      // wmin_raw * beta
  float wmin_s;    // wmin / s (asymmetric)
  float base;      // searched scale
  bool pos_dom;    // symmetric: the positive extreme dominates
};

__device__ __forceinline__ float clamp_magnitude(float s, float eps) {
  float sg = signf(s);
  sg = (sg == 0.0f) ? 1.0f : sg;
  return sg * fmaxf(fabsf(s), eps);
}

// x / maxq, correctly rounded, from inv_maxq = RN(1/maxq): the fused
// correction of quotients() below. maxq is 2^b - 1 or 2^(b - 1), b in [2, 8],
// a divisor of at most 8 significant bits, and the identity holds for every
// float32 significand of x (checked exhaustively for each maxq by the test
// suite); x is zero or of magnitude in [2^-60, 2^60], otherwise it divides.
__device__ __forceinline__ float div_maxq(float x, float maxq, float inv_maxq) {
  const float ax = fabsf(x);
  if (ax == 0.0f || (ax >= 0x1p-60f && ax <= 0x1p60f)) {
    const float q0 = x * inv_maxq;
    const float r = fmaf(q0, maxq, -x);
    return fmaf(-r, inv_maxq, q0);
  }
  return x / maxq;
}

// Per-group scale and zero point: mround/reference/quantize.py:156-246.
template <int MODE>
__device__ __forceinline__ Group group_params(float mx, float mn, float a, float b, float base,
                                              float maxq, float inv_maxq, float eps) {
  Group p;
  p.base = base;
  p.zp = 0.0f;
  p.wmin_s = 0.0f;
  p.pos_dom = false;
  p.wmax_raw = fmaxf(mx, 0.0f);
  p.wmin_raw = fminf(mn, 0.0f);
  if constexpr (MODE == MR_SYM_SEARCHED) {
    p.wmin = 0.0f;
    p.s = clamp_magnitude(base * b, eps);
  } else {
    float wmax = p.wmax_raw * a;
    p.wmin = p.wmin_raw * b;
    if constexpr (MODE == MR_ASYM) {
      p.s = fmaxf(div_maxq(wmax - p.wmin, maxq, inv_maxq), eps);
      // -wmin / s rounds to -(wmin / s): one division serves both.
      p.wmin_s = p.wmin / p.s;
      p.zp = rintf(-p.wmin_s);
    } else {
      float pos_mag = wmax;
      float neg_mag = -p.wmin;
      p.pos_dom = pos_mag >= neg_mag;
      float dominant = p.pos_dom ? pos_mag : neg_mag;
      float signed_ = p.pos_dom ? -dominant : dominant;
      p.s = clamp_magnitude(div_maxq(signed_, maxq, inv_maxq), eps);
    }
  }
  return p;
}

// One weight from its quotient t = w / s: code (before narrowing), clamp mask,
// reconstruction.
template <int MODE, bool HAS_V>
__device__ __forceinline__ float quant_t(float t, float v, const Group& p, float qmin, float qmax,
                                         float& code, float& inside) {
  float x = t;
  if constexpr (HAS_V) x = x + v;
  float raw = rintf(x);
  if constexpr (MODE == MR_ASYM) raw = raw + p.zp;
  inside = (raw >= qmin && raw <= qmax) ? 1.0f : 0.0f;
  code = clampf(raw, qmin, qmax);
  if constexpr (MODE == MR_ASYM) return p.s * (code - p.zp);
  return p.s * code;
}

template <int MODE, bool HAS_V>
__device__ __forceinline__ float quant_one(float w, float v, const Group& p, float qmin, float qmax,
                                           float& code, float& inside) {
  return quant_t<MODE, HAS_V>(w / p.s, v, p, qmin, qmax, code, inside);
}

// Quotients w / s of a lane's weights by their group's scale.
//
// The reference divides in float32, so every quotient must be the correctly
// rounded one. An IEEE division costs about ten instructions and a hazard
// stall; the fast kernels divide each of a lane's bfloat16 weights by the one
// scale instead as
//   y = RN(1/s) (one IEEE division per lane),  q0 = RN(w * y),
//   r = RN(q0 * s - w) (fused),                 t = RN(q0 - r * y) (fused),
// a one-step Markstein correction. For a numerator of at most 8 significant
// bits (every bfloat16 value) and any float32 divisor t equals RN(w / s): the
// identity depends only on the two significands while every intermediate
// stays normal, and all 2^7 x 2^23 significand pairs are checked exhaustively
// by the test suite. The lane takes this path only when each weight is zero
// or has magnitude in [2^-60, 2^60] and so does the scale (then q0, r and t
// are normal); otherwise, and for float32 weights, it divides. With s > 0
// this form also gives the quotient of a signed zero its IEEE sign; a
// negative symmetric scale divides -w by -s.
constexpr float kQuotLo = 0x1p-60f, kQuotHi = 0x1p60f;
// Smallest admissible (bits << 1) - 2 of a nonzero weight; both zeros wrap
// above every key.
constexpr uint32_t kQuotKeyLo = ((127u - 60u) << 24) - 2u;

template <int WT, int N>
__device__ __forceinline__ bool lane_quotients_fast(const float (&x)[N], float mx, float mn) {
  if constexpr (WT != MR_BF16) {
    return false;
  } else {
    uint32_t kmin = 0xffffffffu;
#pragma unroll
    for (int k = 0; k < N; ++k) kmin = min(kmin, (__float_as_uint(x[k]) << 1) - 2u);
    return kmin >= kQuotKeyLo && fmaxf(mx, -mn) <= kQuotHi;
  }
}

template <int WT, int MODE, int N>
__device__ __forceinline__ void quotients(const float (&x)[N], float s, bool lane_fast,
                                          float (&t)[N]) {
  if constexpr (WT == MR_BF16) {
    // The asymmetric scale is positive; should it not be, the lane divides.
    const float sa = MODE == MR_ASYM ? s : fabsf(s);
    if (lane_fast && sa >= kQuotLo && sa <= kQuotHi) {
      const float y = 1.0f / sa;
      const uint32_t sgn = MODE == MR_ASYM ? 0u : (__float_as_uint(s) & 0x80000000u);
#pragma unroll
      for (int k = 0; k < N; ++k) {
        const float w = __uint_as_float(__float_as_uint(x[k]) ^ sgn);
        const float q0 = w * y;
        const float r = fmaf(q0, sa, -w);
        t[k] = fmaf(-r, y, q0);
      }
      return;
    }
  }
#pragma unroll
  for (int k = 0; k < N; ++k) t[k] = x[k] / s;
}

__device__ __forceinline__ float group_max(float x, int tpg) {
  for (int off = tpg >> 1; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, tpg));
  return x;
}
__device__ __forceinline__ float group_min(float x, int tpg) {
  for (int off = tpg >> 1; off > 0; off >>= 1) x = fminf(x, __shfl_xor(x, off, tpg));
  return x;
}
__device__ __forceinline__ float group_sum(float x, int tpg) {
  for (int off = tpg >> 1; off > 0; off >>= 1) x = x + __shfl_xor(x, off, tpg);
  return x;
}
// Compile-time-width butterflies: xor partners below 32 lanes come from
// ds_swizzle in bit mode (lane ^ OFF within each 32-lane half, no address
// arithmetic); only the 32-lane step needs a permute.
template <int OFF>
__device__ __forceinline__ float xor_lane(float x) {
  if constexpr (OFF < 32) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x1f | (OFF << 10)));
  } else {
    return __shfl_xor(x, OFF, 64);
  }
}
template <int OFF>
__device__ __forceinline__ float bfly_max(float x) {
  if constexpr (OFF >= 1) return bfly_max<OFF / 2>(fmaxf(x, xor_lane<OFF>(x)));
  return x;
}
template <int OFF>
__device__ __forceinline__ float bfly_min(float x) {
  if constexpr (OFF >= 1) return bfly_min<OFF / 2>(fminf(x, xor_lane<OFF>(x)));
  return x;
}
template <int OFF>
__device__ __forceinline__ float bfly_sum(float x) {
  if constexpr (OFF >= 1) return bfly_sum<OFF / 2>(x + xor_lane<OFF>(x));
  return x;
}
// TPG > 0: width known at compile time; TPG == 0: runtime width `tpg`.
template <int TPG>
__device__ __forceinline__ float gmax(float x, int tpg) {
  if constexpr (TPG > 0) return bfly_max<TPG / 2>(x);
  return group_max(x, tpg);
}
template <int TPG>
__device__ __forceinline__ float gmin(float x, int tpg) {
  if constexpr (TPG > 0) return bfly_min<TPG / 2>(x);
  return group_min(x, tpg);
}
template <int TPG>
__device__ __forceinline__ float gsum(float x, int tpg) {
  if constexpr (TPG > 0) return bfly_sum<TPG / 2>(x);
  return group_sum(x, tpg);
}

__device__ __forceinline__ float wave_max(float x) { return group_max(x, 64); }
__device__ __forceinline__ float wave_min(float x) { return group_min(x, 64); }
__device__ __forceinline__ float wave_sum(float x) { return group_sum(x, 64); }

// ---------------------------------------------------------------- forward --

template <int WT, int OT, int MODE, bool HAS_V, int TPG>
__global__ __launch_bounds__(kBlock) void fq_fwd_fast(
    const void* __restrict__ w, const float* __restrict__ v, const float* __restrict__ alpha,
    const float* __restrict__ beta, const float* __restrict__ init_scale, void* __restrict__ wq,
    uint8_t* __restrict__ codes, float* __restrict__ scale_out, float* __restrict__ zp_out,
    int64_t n_chunks, int tpg, int tpg_shift, float maxq, float inv_maxq, float qmin, float qmax, float eps,
    RowMap map) {
  int64_t chunk = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const bool active = chunk < n_chunks;
  // Inactive lanes form whole groups (n_chunks % tpg == 0); they stay for the
  // shuffles on a valid address and store nothing.
  if (!active) chunk = n_chunks - 1;
  const int64_t grp = chunk >> tpg_shift;
  const int64_t e = chunk * 8;

  float x[8];
  load8<WT>(w, e, x);
  float mx = x[0], mn = x[0];
#pragma unroll
  for (int k = 1; k < 8; ++k) {
    mx = fmaxf(mx, x[k]);
    mn = fminf(mn, x[k]);
  }
  if constexpr (MODE != MR_SYM_SEARCHED) {
    mx = gmax<TPG>(mx, tpg);
    mn = gmin<TPG>(mn, tpg);
  }
  float a = 1.0f, b = 1.0f, base = 0.0f;
  if constexpr (HAS_V) {
    a = alpha[grp];
    b = beta[grp];
  }
  if constexpr (MODE == MR_SYM_SEARCHED) base = init_scale[grp];
  const Group p = group_params<MODE>(mx, mn, a, b, base, maxq, inv_maxq, eps);

  float vv[8];
  if constexpr (HAS_V) {
    load8_f32_cached(v, e, vv);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) vv[k] = 0.0f;
  }
  float t[8];
  quotients<WT, MODE>(x, p.s, lane_quotients_fast<WT>(x, mx, mn), t);
  float q[8], c[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float in;
    q[k] = quant_t<MODE, HAS_V>(t[k], vv[k], p, qmin, qmax, c[k], in);
  }
  if (!active) return;
  if (wq) store8<OT>(wq, map.chunk_elem(chunk), q);
  if (codes) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      lo |= (static_cast<uint32_t>(static_cast<int>(c[k])) & 0xffu) << (8 * k);
      hi |= (static_cast<uint32_t>(static_cast<int>(c[k + 4])) & 0xffu) << (8 * k);
    }
    *reinterpret_cast<uint2*>(codes + e) = make_uint2(lo, hi);
  }
  if ((chunk & (tpg - 1)) == 0) {
    if (scale_out) scale_out[grp] = p.s;
    if (zp_out) zp_out[grp] = p.zp;
  }
}

// Quantize and pack in one pass: the forward's codes go straight into MLX
// uint32 words (element 0 in the low bits; 3/5/6/7-bit codes straddle words),
// with the group's MLX scale and bias (scales = out(s), biases =
// out(-scales * out(zp)), zp = 2^(bits-1) for the symmetric modes) from the
// group leader. Four consecutive lanes hold 32 codes, which fill exactly
// `bits` words: each lane shifts its 8 codes (8 * bits stream bits, at most 64)
// into place in every word they touch, the four lanes OR their words together
// by two xor-shuffles, and lane r of the four stores words r and r + 4.
// Needs cols % 32 == 0 (every 32-code run lies in one row and one group).
// Lane exchanges within each quad of lanes by DPP quad permutations (VALU,
// no LDS): the value of lane l ^ 1 and of lane l ^ 2.
__device__ __forceinline__ uint32_t quad_xor1(uint32_t x) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ uint32_t quad_xor2(uint32_t x) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x4E, 0xF, 0xF, false));
}
// The value of the next lane of the quad (the last lane keeps its own).
__device__ __forceinline__ uint32_t quad_next(uint32_t x) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0xF9, 0xF, 0xF, false));
}

// PB: the code width when it is 2, 3, 4 or 8 (a lane's 8 codes then fill half a
// word, three quarters of one, one word or two words, in its quad's word
// order), 0 for any width (5, 6, 7: codes straddle words).
template <int WT, int OT, int MODE, bool HAS_V, int TPG, int PB>
__global__ __launch_bounds__(kBlock) void fq_pack_fast(
    const void* __restrict__ w, const float* __restrict__ v, const float* __restrict__ alpha,
    const float* __restrict__ beta, const float* __restrict__ init_scale, uint32_t* __restrict__ packed,
    void* __restrict__ scales, void* __restrict__ biases, int64_t n_chunks, int tpg, int tpg_shift,
    int bits, float maxq, float inv_maxq, float qmin, float qmax, float eps) {
  int64_t chunk = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const bool active = chunk < n_chunks;
  if (!active) chunk = n_chunks - 1;  // whole groups of inactive lanes stay for the shuffles
  const int64_t grp = chunk >> tpg_shift;
  const int64_t e = chunk * 8;

  float x[8];
  load8<WT>(w, e, x);
  float mx = x[0], mn = x[0];
#pragma unroll
  for (int k = 1; k < 8; ++k) {
    mx = fmaxf(mx, x[k]);
    mn = fminf(mn, x[k]);
  }
  if constexpr (MODE != MR_SYM_SEARCHED) {
    mx = gmax<TPG>(mx, tpg);
    mn = gmin<TPG>(mn, tpg);
  }
  float a = 1.0f, b = 1.0f, base = 0.0f;
  if constexpr (HAS_V) {
    a = alpha[grp];
    b = beta[grp];
  }
  if constexpr (MODE == MR_SYM_SEARCHED) base = init_scale[grp];
  const Group p = group_params<MODE>(mx, mn, a, b, base, maxq, inv_maxq, eps);
  float vv[8];
  if constexpr (HAS_V) {
    load8_f32_cached(v, e, vv);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) vv[k] = 0.0f;
  }
  // stored (unsigned) codes: the symmetric ones offset by 2^(bits-1)
  const uint32_t off = MODE == MR_ASYM ? 0u : static_cast<uint32_t>(maxq);
  float t[8];
  quotients<WT, MODE>(x, p.s, lane_quotients_fast<WT>(x, mx, mn), t);
  uint32_t u[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float c, in;
    quant_t<MODE, HAS_V>(t[k], vv[k], p, qmin, qmax, c, in);
    u[k] = static_cast<uint32_t>(static_cast<int>(c) + static_cast<int>(off));
  }
  // Four consecutive lanes hold the 32 codes of a `bits`-word run; lane r's
  // codes are stream bits [8 r bits, 8 (r + 1) bits).
  const int r = static_cast<int>(chunk & 3);
  uint32_t* dst = packed + (e >> 5) * bits;
  if constexpr (PB == 2 || PB == 4) {
    uint32_t st = 0;  // the lane's 8 codes: 16 or 32 bits
#pragma unroll
    for (int k = 0; k < 8; ++k) st |= u[k] << (k * PB);
    if constexpr (PB == 2) {
      const uint32_t odd = quad_xor1(st);  // lanes 2j and 2j + 1 make word j
      if (!active) return;
      if (!(r & 1)) dst[r >> 1] = st | (odd << 16);
    } else {
      if (!active) return;
      dst[r] = st;
    }
  } else if constexpr (PB == 3) {
    // 24 stream bits per lane: word r (r < 3) is bits 32 r .. 32 r + 31 of the
    // run, the top 24 - 8 r bits of lane r's codes and the low 8 + 8 r bits
    // of lane r + 1's.
    uint32_t st = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) st |= u[k] << (3 * k);
    const uint32_t nx = quad_next(st);
    if (!active) return;
    if (r < 3) dst[r] = (st >> (8 * r)) | (nx << (24 - 8 * r));
  } else if constexpr (PB == 8) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      lo |= u[k] << (8 * k);
      hi |= u[k + 4] << (8 * k);
    }
    if (!active) return;
    dst[2 * r] = lo;  // (the words are only 4-byte aligned)
    dst[2 * r + 1] = hi;
  } else {
    uint64_t stream = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) stream |= static_cast<uint64_t>(u[k]) << (k * bits);
    const int start = 8 * r * bits;  // this lane's first bit in the 32-code run
    uint32_t word[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int sh = start - 32 * q;  // where the lane's bits start relative to word q
      uint32_t part = 0;
      if (q < bits) {
        if (sh >= 0) part = sh < 32 ? static_cast<uint32_t>(stream << sh) : 0u;
        else part = -sh < 64 ? static_cast<uint32_t>(stream >> (-sh)) : 0u;
      }
      part |= quad_xor1(part);
      part |= quad_xor2(part);
      word[q] = part;
    }
    if (!active) return;
    if (r < bits) dst[r] = word[r];
    if (r + 4 < bits) dst[r + 4] = word[r + 4];
  }
  if ((chunk & (tpg - 1)) == 0) {
    // scales = out(s), biases = out(-scales * out(zp)): the narrowed values
    // are formed in registers, not read back from memory.
    const float sq = round_to<OT>(p.s);
    float z = maxq;  // symmetric: the stored code offset
    if constexpr (MODE == MR_ASYM) z = round_to<OT>(p.zp);
    store_elem<OT>(scales, grp, sq);
    store_elem<OT>(biases, grp, -sq * z);
  }
}

__device__ __forceinline__ float load_any(const void* p, int dt, int64_t i) {
  if (dt == MR_F32) return load_elem<MR_F32>(p, i);
  if (dt == MR_BF16) return load_elem<MR_BF16>(p, i);
  return load_elem<MR_F16>(p, i);
}
__device__ __forceinline__ void store_any(void* p, int dt, int64_t i, float x) {
  if (dt == MR_F32) store_elem<MR_F32>(p, i, x);
  else if (dt == MR_BF16) store_elem<MR_BF16>(p, i, x);
  else store_elem<MR_F16>(p, i, x);
}

// One wave per group; v and codes use the padded grouped layout (stride gs).
template <int MODE, bool HAS_V>
__global__ __launch_bounds__(kBlock) void fq_fwd_generic(
    const void* __restrict__ w, int wt, const float* __restrict__ v,
    const float* __restrict__ alpha, const float* __restrict__ beta,
    const float* __restrict__ init_scale, void* __restrict__ wq, int ot,
    uint8_t* __restrict__ codes, float* __restrict__ scale_out, float* __restrict__ zp_out,
    int64_t rows, int64_t cols, int gs, int64_t ng, float maxq, float inv_maxq, float qmin, float qmax,
    float eps, RowMap map) {
  const int64_t grp = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (grp >= rows * ng) return;  // uniform across the wave
  const int64_t r = grp / ng;
  const int64_t c0 = (grp % ng) * gs;
  float mx = 0.0f, mn = 0.0f;  // padding zeros and the forced zero coincide
  if constexpr (MODE != MR_SYM_SEARCHED) {
    for (int t = lane; t < gs; t += 64) {
      int64_t c = c0 + t;
      float x = c < cols ? load_any(w, wt, r * cols + c) : 0.0f;
      mx = fmaxf(mx, x);
      mn = fminf(mn, x);
    }
    mx = wave_max(mx);
    mn = wave_min(mn);
  }
  float a = 1.0f, b = 1.0f, base = 0.0f;
  if constexpr (HAS_V) {
    a = alpha[grp];
    b = beta[grp];
  }
  if constexpr (MODE == MR_SYM_SEARCHED) base = init_scale[grp];
  const Group p = group_params<MODE>(mx, mn, a, b, base, maxq, inv_maxq, eps);
  for (int t = lane; t < gs; t += 64) {
    int64_t c = c0 + t;
    float x = c < cols ? load_any(w, wt, r * cols + c) : 0.0f;
    float vv = 0.0f;
    if constexpr (HAS_V) vv = v[grp * gs + t];
    float code, in;
    float q = quant_one<MODE, HAS_V>(x, vv, p, qmin, qmax, code, in);
    if (wq && c < cols) store_any(wq, ot, map.row(r) * cols + c, q);
    if (codes) codes[grp * gs + t] = static_cast<uint8_t>(static_cast<int>(code) & 0xff);
  }
  if (lane == 0) {
    if (scale_out) scale_out[grp] = p.s;
    if (zp_out) zp_out[grp] = p.zp;
  }
}

// --------------------------------------------------------------- backward --

// Per-element backward terms: mround/reference/quantize.py:464-520.
//
// The reference writes d(qdq)/ds for the asymmetric mode as
//   (c - zp) + s * (inside * (-w/s^2 + wmin/s^2) - wmin/s^2),
// which is (c - zp) - w/s inside the clamp and (c - zp) - wmin/s outside it;
// for the symmetric modes it is c - inside * w / s. Both are evaluated here
// from t = w/s, the quotient the rounding already needs, and the per-group
// wmin/s, so the backward costs one division per weight like the forward.
// grad_v = g * s * inside is formed exactly as the reference forms it; only
// the summands of the per-group sums are rounded differently.
template <int MODE>
struct BwdTerms {
  float gv, ts, td;
};

template <int MODE>
__device__ __forceinline__ BwdTerms<MODE> bwd_one(float t, float vv, float g, const Group& p,
                                                  float wmin_over_s, float qmin, float qmax) {
  float raw = rintf(t + vv);
  if constexpr (MODE == MR_ASYM) raw = raw + p.zp;
  const bool in = raw >= qmin && raw <= qmax;
  const float inside = in ? 1.0f : 0.0f;
  const float code = clampf(raw, qmin, qmax);
  BwdTerms<MODE> r;
  r.gv = g * p.s * inside;
  if constexpr (MODE == MR_ASYM) {
    const float dq = (code - p.zp) - (in ? t : wmin_over_s);
    r.ts = g * dq;
    r.td = g * (1.0f - inside) * p.wmin_raw;
  } else {
    const float dq = code - (in ? t : 0.0f);
    r.ts = g * dq;
    r.td = 0.0f;
  }
  return r;
}

// dL/dalpha, dL/dbeta from the group sums: mround/reference/quantize.py:388-396,
// 480-487, 506-520.
template <int MODE>
__device__ __forceinline__ void coef_grads(const Group& p, float sum_s, float sum_d, float maxq,
                                           float& ga, float& gb) {
  if constexpr (MODE == MR_ASYM) {
    ga = sum_s * (p.wmax_raw / maxq);
    gb = sum_s * (-p.wmin_raw / maxq) + sum_d;
  } else if constexpr (MODE == MR_SYM) {
    float da = p.pos_dom ? -p.wmax_raw / maxq : 0.0f;
    float db = p.pos_dom ? 0.0f : -p.wmin_raw / maxq;
    ga = sum_s * da;
    gb = sum_s * db;
  } else {
    ga = 0.0f;
    gb = sum_s * p.base;
  }
}

struct StepArgs {
  float lr, lo, hi, vb;
  void* wq;   // if non-null: W' of the updated parameters, through the placement
  int wq_dt;  // its dtype
  // If non-null, the rate is lr_tab[clamp(*step, 0, lr_len - 1)] (a schedule
  // in device memory, for launches recorded once and replayed every step).
  const float* lr_tab;
  const int* step;
  int lr_len;
  __device__ __forceinline__ float rate() const {
    if (!lr_tab) return lr;
    const int i = min(max(*step, 0), lr_len - 1);
    return lr_tab[i];
  }
};

// Each lane owns one 8-weight chunk. (Two consecutive chunks a lane, which
// halves the per-group work per weight, measured 30 % slower: each 16-byte
// access of the wave then covers every other 16 bytes.)
template <int WT, int GT, int MODE, bool UPDATE, int TPG>
__global__ __launch_bounds__(kBlock) void fq_bwd_fast(
    const void* __restrict__ w, float* __restrict__ v, float* __restrict__ alpha,
    float* __restrict__ beta, const float* __restrict__ init_scale, const void* __restrict__ g,
    int64_t n_chunks, int tpg, int tpg_shift, float maxq, float inv_maxq, float qmin, float qmax, float eps,
    StepArgs st, float* __restrict__ gv_out, float* __restrict__ ga_out,
    float* __restrict__ gb_out, RowMap map) {
  constexpr int N = 8;
  if constexpr (UPDATE) st.lr = st.rate();
  int64_t chunk = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const bool active = chunk < n_chunks;
  if (!active) chunk = n_chunks - 1;
  const int64_t grp = chunk >> tpg_shift;
  const int64_t e = chunk * 8;

  float x[N], vv[N], gg[N];
  load8<WT>(w, e, x);
  load8_f32_cached(v, e, vv);
  load8<GT>(g, map.chunk_elem(chunk), gg);
  float mx = x[0], mn = x[0];
#pragma unroll
  for (int k = 1; k < N; ++k) {
    mx = fmaxf(mx, x[k]);
    mn = fminf(mn, x[k]);
  }
  if constexpr (MODE != MR_SYM_SEARCHED) {
    mx = gmax<TPG>(mx, tpg);
    mn = gmin<TPG>(mn, tpg);
  }
  const float a = alpha[grp];
  const float b = beta[grp];
  float base = 0.0f;
  if constexpr (MODE == MR_SYM_SEARCHED) base = init_scale[grp];
  const Group p = group_params<MODE>(mx, mn, a, b, base, maxq, inv_maxq, eps);
  const float wmin_over_s = p.wmin_s;
  const bool lane_fast = lane_quotients_fast<WT>(x, mx, mn);
  float tq[N];
  quotients<WT, MODE>(x, p.s, lane_fast, tq);

  float sum_s = 0.0f, sum_d = 0.0f;
  float gv[N];
#pragma unroll
  for (int k = 0; k < N; ++k) {
    BwdTerms<MODE> t = bwd_one<MODE>(tq[k], vv[k], gg[k], p, wmin_over_s, qmin, qmax);
    gv[k] = t.gv;
    sum_s = sum_s + t.ts;
    if constexpr (MODE == MR_ASYM) sum_d = sum_d + t.td;
  }
  sum_s = gsum<TPG>(sum_s, tpg);
  if constexpr (MODE == MR_ASYM) sum_d = gsum<TPG>(sum_d, tpg);
  float ga, gb;
  coef_grads<MODE>(p, sum_s, sum_d, maxq, ga, gb);

  if (!active) return;
  if (gv_out) store8_f32(gv_out, e, gv);
  const bool leader = (chunk & (tpg - 1)) == 0;
  if (leader) {
    if (ga_out) ga_out[grp] = ga;
    if (gb_out) gb_out[grp] = gb;
  }
  if constexpr (UPDATE) {
    float nv[N];
#pragma unroll
    for (int k = 0; k < N; ++k) nv[k] = clampf(vv[k] - st.lr * signf(gv[k]), -st.vb, st.vb);
    store8_f32_cached(v, e, nv);
    // Every lane of the group holds the group sums, so each forms the new
    // coefficients itself (the leader stores them).
    const float na = clampf(a - st.lr * signf(ga), st.lo, st.hi);
    const float nb = clampf(b - st.lr * signf(gb), st.lo, st.hi);
    if (leader) {
      alpha[grp] = na;
      beta[grp] = nb;
    }
    if (st.wq) {
      // The next step's W': the forward's arithmetic on the same group
      // extremes and the parameters just written.
      const Group p2 = group_params<MODE>(mx, mn, na, nb, base, maxq, inv_maxq, eps);
      quotients<WT, MODE>(x, p2.s, lane_fast, tq);
      float q[N];
#pragma unroll
      for (int k = 0; k < N; ++k) {
        float code, in;
        q[k] = quant_t<MODE, true>(tq[k], nv[k], p2, qmin, qmax, code, in);
      }
      const int64_t o = map.chunk_elem(chunk);
      if (st.wq_dt == MR_BF16) store8<MR_BF16>(st.wq, o, q);
      else if (st.wq_dt == MR_F16) store8<MR_F16>(st.wq, o, q);
      else store8<MR_F32>(st.wq, o, q);
    }
  }
}

template <int MODE, bool UPDATE>
__global__ __launch_bounds__(kBlock) void fq_bwd_generic(
    const void* __restrict__ w, int wt, float* __restrict__ v, float* __restrict__ alpha,
    float* __restrict__ beta, const float* __restrict__ init_scale, const void* __restrict__ g,
    int gt, int64_t rows, int64_t cols, int gs, int64_t ng, float maxq, float inv_maxq, float qmin, float qmax,
    float eps, StepArgs st, float* __restrict__ gv_out, float* __restrict__ ga_out,
    float* __restrict__ gb_out, RowMap map) {
  if constexpr (UPDATE) st.lr = st.rate();
  const int64_t grp = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (grp >= rows * ng) return;
  const int64_t r = grp / ng;
  const int64_t c0 = (grp % ng) * gs;
  float mx = 0.0f, mn = 0.0f;
  if constexpr (MODE != MR_SYM_SEARCHED) {
    for (int t = lane; t < gs; t += 64) {
      int64_t c = c0 + t;
      float x = c < cols ? load_any(w, wt, r * cols + c) : 0.0f;
      mx = fmaxf(mx, x);
      mn = fminf(mn, x);
    }
    mx = wave_max(mx);
    mn = wave_min(mn);
  }
  const float a = alpha[grp];
  const float b = beta[grp];
  float base = 0.0f;
  if constexpr (MODE == MR_SYM_SEARCHED) base = init_scale[grp];
  const Group p = group_params<MODE>(mx, mn, a, b, base, maxq, inv_maxq, eps);
  const float wmin_over_s = p.wmin_s;
  float sum_s = 0.0f, sum_d = 0.0f;
  for (int t = lane; t < gs; t += 64) {
    int64_t c = c0 + t;
    bool real = c < cols;
    float x = real ? load_any(w, wt, r * cols + c) : 0.0f;
    float gg = real ? load_any(g, gt, map.row(r) * cols + c) : 0.0f;
    float vv = v[grp * gs + t];
    BwdTerms<MODE> tm = bwd_one<MODE>(x / p.s, vv, gg, p, wmin_over_s, qmin, qmax);
    sum_s = sum_s + tm.ts;
    if constexpr (MODE == MR_ASYM) sum_d = sum_d + tm.td;
    if (gv_out) gv_out[grp * gs + t] = tm.gv;
    if constexpr (UPDATE) v[grp * gs + t] = clampf(vv - st.lr * signf(tm.gv), -st.vb, st.vb);
  }
  sum_s = wave_sum(sum_s);
  if constexpr (MODE == MR_ASYM) sum_d = wave_sum(sum_d);
  float ga, gb;
  coef_grads<MODE>(p, sum_s, sum_d, maxq, ga, gb);
  if (lane == 0) {
    if (ga_out) ga_out[grp] = ga;
    if (gb_out) gb_out[grp] = gb;
    if constexpr (UPDATE) {
      alpha[grp] = clampf(a - st.lr * signf(ga), st.lo, st.hi);
      beta[grp] = clampf(b - st.lr * signf(gb), st.lo, st.hi);
    }
  }
  if constexpr (UPDATE) {
    if (st.wq) {
      // The next step's W' from the parameters just written (each lane
      // rereads the v entries it wrote itself).
      const float na = clampf(a - st.lr * signf(ga), st.lo, st.hi);
      const float nb = clampf(b - st.lr * signf(gb), st.lo, st.hi);
      const Group p2 = group_params<MODE>(mx, mn, na, nb, base, maxq, inv_maxq, eps);
      for (int t = lane; t < gs; t += 64) {
        const int64_t c = c0 + t;
        if (c >= cols) continue;
        const float x = load_any(w, wt, r * cols + c);
        float code, in;
        const float q = quant_one<MODE, true>(x, v[grp * gs + t], p2, qmin, qmax, code, in);
        store_any(st.wq, st.wq_dt, map.row(r) * cols + c, q);
      }
    }
  }
}

// ------------------------------------------------------------ host side --

struct Shape {
  int64_t rows, cols, ng, n_groups;
  int gs, tpg, tpg_shift;
  bool fast;
  float maxq, inv_maxq, qmin, qmax;  // inv_maxq = RN(1 / maxq)
};

int check_common(const char* fn, const void* w, int w_dtype, int64_t rows, int64_t cols,
                 int group_size, int bits, int mode, const float* init_scale, Shape& sh) {
  if (!w && rows > 0 && cols > 0) return fail(MR_EINVAL, "%s: weight pointer is null", fn);
  if (!valid_dtype(w_dtype)) return fail(MR_EINVAL, "%s: unknown weight dtype %d", fn, w_dtype);
  if (rows < 0 || cols < 0) return fail(MR_EINVAL, "%s: negative shape", fn);
  if (bits < 2 || bits > 8) return fail(MR_EINVAL, "%s: bits must be in [2, 8], got %d", fn, bits);
  if (mode != MR_ASYM && mode != MR_SYM && mode != MR_SYM_SEARCHED)
    return fail(MR_EINVAL, "%s: unknown mode %d", fn, mode);
  if (group_size != -1 && group_size <= 0)
    return fail(MR_EINVAL, "%s: group_size must be positive or -1, got %d", fn, group_size);
  if ((mode == MR_SYM_SEARCHED) != (init_scale != nullptr) && rows > 0 && cols > 0)
    return fail(MR_EINVAL, "%s: init_scale is required by, and only by, the searched mode", fn);
  sh.rows = rows;
  sh.cols = cols;
  int64_t gs = group_size == -1 ? cols : group_size;
  if (gs > (int64_t{1} << 30)) return fail(MR_EINVAL, "%s: group too large", fn);
  sh.gs = static_cast<int>(gs);
  sh.ng = (group_size == -1) ? 1 : (cols + gs - 1) / gs;
  sh.n_groups = rows * sh.ng;
  int tpg = sh.gs / 8;
  bool pow2 = tpg > 0 && (tpg & (tpg - 1)) == 0 && tpg <= 64;
  sh.tpg = tpg;
  sh.tpg_shift = 0;
  while (pow2 && (1 << sh.tpg_shift) < tpg) ++sh.tpg_shift;
  sh.fast = (sh.gs % 8 == 0) && pow2 && gs > 0 && (cols % gs == 0);
  if (mode == MR_ASYM) {
    sh.maxq = static_cast<float>((1 << bits) - 1);
    sh.qmin = 0.0f;
    sh.qmax = sh.maxq;
  } else {
    sh.maxq = static_cast<float>(1 << (bits - 1));
    sh.qmin = -sh.maxq;
    sh.qmax = sh.maxq - 1.0f;
  }
  sh.inv_maxq = 1.0f / sh.maxq;
  return MR_OK;
}

template <int MODE, bool HAS_V>
int launch_fwd(const Shape& sh, const void* w, int wt, const float* v, const float* alpha,
               const float* beta, const float* init_scale, void* wq, int ot, uint8_t* codes,
               float* scale_out, float* zp_out, float eps, RowMap map, hipStream_t stream) {
  map.prepare(sh.cols);
  const bool fast_types = (wt == MR_F32 || wt == MR_BF16) && (!wq || ot == MR_F32 || ot == MR_BF16);
  const bool fast_align = aligned16(w) && (!HAS_V || aligned16(v)) && (!wq || aligned16(wq)) &&
                          (!codes || (reinterpret_cast<uintptr_t>(codes) & 7u) == 0);
  if (sh.fast && fast_types && fast_align) {
    const int64_t n_chunks = sh.rows * sh.cols / 8;
    const int64_t blocks = (n_chunks + kBlock - 1) / kBlock;
    if (blocks > 0x7fffffff) return fail(MR_EINVAL, "mr_fq_forward: tensor too large");
#define MR_FWD_FAST_T(WT_, OT_, T_)                                                        \
  hipLaunchKernelGGL((fq_fwd_fast<WT_, OT_, MODE, HAS_V, T_>),                             \
                     dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, stream, w, v, alpha, \
                     beta, init_scale, wq, codes, scale_out, zp_out, n_chunks, sh.tpg,       \
                     sh.tpg_shift, sh.maxq, sh.inv_maxq, sh.qmin, sh.qmax, eps, map)
#define MR_FWD_FAST(WT_, OT_)                                               \
  do {                                                                      \
    if (sh.tpg == 8) MR_FWD_FAST_T(WT_, OT_, 8);                            \
    else if (sh.tpg == 4) MR_FWD_FAST_T(WT_, OT_, 4);                       \
    else if (sh.tpg == 16) MR_FWD_FAST_T(WT_, OT_, 16);                     \
    else MR_FWD_FAST_T(WT_, OT_, 0);                                        \
  } while (0)
    const int o = wq ? ot : MR_F32;
    if (wt == MR_BF16 && o == MR_BF16) MR_FWD_FAST(MR_BF16, MR_BF16);
    else if (wt == MR_BF16) MR_FWD_FAST(MR_BF16, MR_F32);
    else if (o == MR_BF16) MR_FWD_FAST(MR_F32, MR_BF16);
    else MR_FWD_FAST(MR_F32, MR_F32);
#undef MR_FWD_FAST_T
#undef MR_FWD_FAST
  } else {
    const int64_t blocks = (sh.n_groups + 3) / 4;
    if (blocks > 0x7fffffff) return fail(MR_EINVAL, "mr_fq_forward: tensor too large");
    hipLaunchKernelGGL((fq_fwd_generic<MODE, HAS_V>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kBlock), 0, stream, w, wt, v, alpha, beta, init_scale, wq, ot, codes,
                       scale_out, zp_out, sh.rows, sh.cols, sh.gs, sh.ng, sh.maxq, sh.inv_maxq, sh.qmin,
                       sh.qmax, eps, map);
  }
  MR_LAUNCH_CHECK("mr_fq_forward");
  return MR_OK;
}

template <int MODE, bool UPDATE>
int launch_bwd(const Shape& sh, const void* w, int wt, float* v, float* alpha, float* beta,
               const float* init_scale, const void* g, int gt, float eps, StepArgs st,
               float* gv_out, float* ga_out, float* gb_out, RowMap map, hipStream_t stream) {
  map.prepare(sh.cols);
  const bool fast_types = (wt == MR_F32 || wt == MR_BF16) && (gt == MR_F32 || gt == MR_BF16);
  const bool fast_align = aligned16(w) && aligned16(v) && aligned16(g) && (!gv_out || aligned16(gv_out));
  if (sh.fast && fast_types && fast_align) {
    const int64_t n_chunks = sh.rows * sh.cols / 8;
    const int64_t blocks = (n_chunks + kBlock - 1) / kBlock;
    if (blocks > 0x7fffffff) return fail(MR_EINVAL, "mr_fq_backward_signsgd: tensor too large");
#define MR_BWD_FAST_T(WT_, GT_, T_)                                                         \
  hipLaunchKernelGGL((fq_bwd_fast<WT_, GT_, MODE, UPDATE, T_>),                             \
                     dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, stream, w, v, alpha, \
                     beta, init_scale, g, n_chunks, sh.tpg, sh.tpg_shift, sh.maxq, sh.inv_maxq,  \
                     sh.qmin, sh.qmax, eps, st, gv_out, ga_out, gb_out, map)
#define MR_BWD_FAST(WT_, GT_)                                               \
  do {                                                                      \
    if (sh.tpg == 8) MR_BWD_FAST_T(WT_, GT_, 8);                            \
    else if (sh.tpg == 4) MR_BWD_FAST_T(WT_, GT_, 4);                       \
    else if (sh.tpg == 16) MR_BWD_FAST_T(WT_, GT_, 16);                     \
    else MR_BWD_FAST_T(WT_, GT_, 0);                                        \
  } while (0)
    if (wt == MR_BF16 && gt == MR_F32) MR_BWD_FAST(MR_BF16, MR_F32);
    else if (wt == MR_BF16) MR_BWD_FAST(MR_BF16, MR_BF16);
    else if (gt == MR_F32) MR_BWD_FAST(MR_F32, MR_F32);
    else MR_BWD_FAST(MR_F32, MR_BF16);
#undef MR_BWD_FAST_T
#undef MR_BWD_FAST
  } else {
    const int64_t blocks = (sh.n_groups + 3) / 4;
    if (blocks > 0x7fffffff) return fail(MR_EINVAL, "mr_fq_backward_signsgd: tensor too large");
    hipLaunchKernelGGL((fq_bwd_generic<MODE, UPDATE>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kBlock), 0, stream, w, wt, v, alpha, beta, init_scale, g, gt, sh.rows,
                       sh.cols, sh.gs, sh.ng, sh.maxq, sh.inv_maxq, sh.qmin, sh.qmax, eps, st, gv_out, ga_out,
                       gb_out, map);
  }
  MR_LAUNCH_CHECK("mr_fq_backward_signsgd");
  return MR_OK;
}

template <int MODE, bool HAS_V>
int launch_pack(const Shape& sh, const void* w, int wt, const float* v, const float* alpha,
                const float* beta, const float* init_scale, uint32_t* packed, void* scales, void* biases,
                int ot, int bits, float eps, hipStream_t stream) {
  const int64_t n_chunks = sh.rows * sh.cols / 8;
  const int64_t blocks = (n_chunks + kBlock - 1) / kBlock;
  if (blocks > 0x7fffffff) return fail(MR_EINVAL, "mr_quantize_pack: tensor too large");
#define MR_PACK_TB(WT_, OT_, T_, PB_)                                                                    \
  hipLaunchKernelGGL((fq_pack_fast<WT_, OT_, MODE, HAS_V, T_, PB_>), dim3(static_cast<unsigned>(blocks)), \
                     dim3(kBlock), 0, stream, w, v, alpha, beta, init_scale, packed, scales, biases,   \
                     n_chunks, sh.tpg, sh.tpg_shift, bits, sh.maxq, sh.inv_maxq, sh.qmin, sh.qmax, eps)
#define MR_PACK_T(WT_, OT_, T_)                         \
  do {                                                  \
    if (bits == 2) MR_PACK_TB(WT_, OT_, T_, 2);         \
    else if (bits == 3) MR_PACK_TB(WT_, OT_, T_, 3);    \
    else if (bits == 4) MR_PACK_TB(WT_, OT_, T_, 4);    \
    else if (bits == 8) MR_PACK_TB(WT_, OT_, T_, 8);    \
    else MR_PACK_TB(WT_, OT_, T_, 0);                   \
  } while (0)
#define MR_PACK_W(WT_, OT_)                             \
  do {                                                  \
    if (sh.tpg == 8) MR_PACK_T(WT_, OT_, 8);            \
    else if (sh.tpg == 4) MR_PACK_T(WT_, OT_, 4);       \
    else if (sh.tpg == 16) MR_PACK_T(WT_, OT_, 16);     \
    else MR_PACK_T(WT_, OT_, 0);                        \
  } while (0)
#define MR_PACK_O(WT_)                                   \
  do {                                                   \
    if (ot == MR_BF16) MR_PACK_W(WT_, MR_BF16);          \
    else if (ot == MR_F16) MR_PACK_W(WT_, MR_F16);       \
    else MR_PACK_W(WT_, MR_F32);                         \
  } while (0)
  if (wt == MR_BF16) MR_PACK_O(MR_BF16);
  else MR_PACK_O(MR_F32);
#undef MR_PACK_O
#undef MR_PACK_W
#undef MR_PACK_T
#undef MR_PACK_TB
  MR_LAUNCH_CHECK("mr_quantize_pack");
  return MR_OK;
}

}  // namespace
}  // namespace mr

extern "C" {

int mr_quantize_pack(const void* w, int w_dtype, const float* v, const float* alpha, const float* beta,
                     const float* init_scale, int64_t rows, int64_t cols, int group_size, int bits,
                     int mode, float eps, uint32_t* packed_out, void* scales_out, void* biases_out,
                     int out_dtype, void* stream) {
  using namespace mr;
  const char* fn = "mr_quantize_pack";
  clear_error();
  Shape sh;
  int rc = check_common(fn, w, w_dtype, rows, cols, group_size, bits, mode, init_scale, sh);
  if (rc) return rc;
  if (rows == 0 || cols == 0) return MR_OK;
  const bool any_v = v || alpha || beta;
  if (any_v && !(v && alpha && beta))
    return fail(MR_EINVAL, "%s: v, alpha and beta are given together or not at all", fn);
  if (!packed_out || !scales_out || !biases_out) return fail(MR_EINVAL, "%s: null output", fn);
  if (!valid_dtype(out_dtype)) return fail(MR_EINVAL, "%s: unknown output dtype %d", fn, out_dtype);
  if (w_dtype != MR_BF16 && w_dtype != MR_F32) return fail(MR_EINVAL, "%s: the weight must be bf16 or fp32", fn);
  if (group_size < 32 || !sh.fast || cols % 32)
    return fail(MR_EINVAL, "%s: needs a power-of-two group size of at least 32 dividing the row, and rows "
                "of whole 32-code runs (got group_size %d, cols %lld)", fn, group_size,
                static_cast<long long>(cols));
  if (!aligned16(w) || (v && !aligned16(v)) || (reinterpret_cast<uintptr_t>(packed_out) & 3u))
    return fail(MR_EINVAL, "%s: the weight and v must be 16-byte aligned and the words 4-byte aligned", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* pk = packed_out;
  if (mode == MR_ASYM)
    return any_v ? launch_pack<MR_ASYM, true>(sh, w, w_dtype, v, alpha, beta, init_scale, pk, scales_out,
                                              biases_out, out_dtype, bits, eps, s)
                 : launch_pack<MR_ASYM, false>(sh, w, w_dtype, v, alpha, beta, init_scale, pk, scales_out,
                                               biases_out, out_dtype, bits, eps, s);
  if (mode == MR_SYM)
    return any_v ? launch_pack<MR_SYM, true>(sh, w, w_dtype, v, alpha, beta, init_scale, pk, scales_out,
                                             biases_out, out_dtype, bits, eps, s)
                 : launch_pack<MR_SYM, false>(sh, w, w_dtype, v, alpha, beta, init_scale, pk, scales_out,
                                              biases_out, out_dtype, bits, eps, s);
  return any_v ? launch_pack<MR_SYM_SEARCHED, true>(sh, w, w_dtype, v, alpha, beta, init_scale, pk,
                                                    scales_out, biases_out, out_dtype, bits, eps, s)
               : launch_pack<MR_SYM_SEARCHED, false>(sh, w, w_dtype, v, alpha, beta, init_scale, pk,
                                                     scales_out, biases_out, out_dtype, bits, eps, s);
}

static int fq_forward_impl(const char* fn, const void* w, int w_dtype, const float* v,
                           const float* alpha, const float* beta, const float* init_scale,
                           int64_t rows, int64_t cols, int group_size, int bits, int mode, float eps,
                           void* wq_out, int wq_dtype, void* codes_out, float* scale_out,
                           float* zp_out, mr::RowMap map, void* stream) {
  using namespace mr;
  clear_error();
  Shape sh;
  int rc = check_common(fn, w, w_dtype, rows, cols, group_size, bits, mode, init_scale, sh);
  if (rc) return rc;
  if (rows == 0 || cols == 0) return MR_OK;
  const bool any_v = v || alpha || beta;
  if (any_v && !(v && alpha && beta))
    return fail(MR_EINVAL, "%s: v, alpha and beta are given together or not at all", fn);
  if (!wq_out && !codes_out && !scale_out && !zp_out)
    return fail(MR_EINVAL, "%s: no output requested", fn);
  if (wq_out && !valid_dtype(wq_dtype))
    return fail(MR_EINVAL, "%s: unknown output dtype %d", fn, wq_dtype);
  if (zp_out && mode != MR_ASYM)
    return fail(MR_EINVAL, "%s: a zero point exists only in the asymmetric mode", fn);
  if (map.blk < 0 || map.stride < 0 || map.off < 0)
    return fail(MR_EINVAL, "%s: negative row placement", fn);
  if (map.blk && (rows * cols / 8 > 0x7fffffffLL || map.blk > 0x7fffffffLL))
    return fail(MR_EINVAL, "%s: placed tensor too large", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* codes = static_cast<uint8_t*>(codes_out);
#define MR_FWD(MODE_)                                                                     \
  return any_v ? launch_fwd<MODE_, true>(sh, w, w_dtype, v, alpha, beta, init_scale, wq_out, \
                                         wq_dtype, codes, scale_out, zp_out, eps, map, s)  \
               : launch_fwd<MODE_, false>(sh, w, w_dtype, v, alpha, beta, init_scale, wq_out, \
                                          wq_dtype, codes, scale_out, zp_out, eps, map, s)
  if (mode == MR_ASYM) MR_FWD(MR_ASYM);
  if (mode == MR_SYM) MR_FWD(MR_SYM);
  MR_FWD(MR_SYM_SEARCHED);
#undef MR_FWD
}

int mr_fq_forward(const void* w, int w_dtype, const float* v, const float* alpha,
                  const float* beta, const float* init_scale, int64_t rows, int64_t cols,
                  int group_size, int bits, int mode, float eps, void* wq_out, int wq_dtype,
                  void* codes_out, float* scale_out, float* zp_out, void* stream) {
  return fq_forward_impl("mr_fq_forward", w, w_dtype, v, alpha, beta, init_scale, rows, cols,
                         group_size, bits, mode, eps, wq_out, wq_dtype, codes_out, scale_out, zp_out,
                         mr::RowMap{0, 0, 0, 0, {}, {}}, stream);
}

int mr_fq_forward_mapped(const void* w, int w_dtype, const float* v, const float* alpha,
                         const float* beta, const float* init_scale, int64_t rows, int64_t cols,
                         int group_size, int bits, int mode, float eps, void* wq_out, int wq_dtype,
                         int64_t row_block, int64_t row_stride, int64_t row_offset, void* stream) {
  if (!wq_out) return mr::fail(MR_EINVAL, "mr_fq_forward_mapped: no output");
  return fq_forward_impl("mr_fq_forward_mapped", w, w_dtype, v, alpha, beta, init_scale, rows,
                         cols, group_size, bits, mode, eps, wq_out, wq_dtype, nullptr, nullptr,
                         nullptr, mr::RowMap{row_block, row_stride, row_offset, 0, {}, {}}, stream);
}

static int fq_backward_impl(const char* fn, const void* w, int w_dtype, float* v, float* alpha,
                            float* beta, const float* init_scale, const void* g, int g_dtype,
                            int64_t rows, int64_t cols, int group_size, int bits, int mode,
                            float eps, int update, float lr, float coef_lo, float coef_hi,
                            float v_bound, float* grad_v_out, float* grad_alpha_out,
                            float* grad_beta_out, mr::RowMap map, void* stream,
                            void* wq_out = nullptr, int wq_dtype = 0,
                            const float* lr_tab = nullptr, const int* step = nullptr,
                            int lr_len = 0) {
  using namespace mr;
  clear_error();
  Shape sh;
  int rc = check_common(fn, w, w_dtype, rows, cols, group_size, bits, mode, init_scale, sh);
  if (rc) return rc;
  if (rows == 0 || cols == 0) return MR_OK;
  if (!v || !alpha || !beta) return fail(MR_EINVAL, "%s: v, alpha and beta are required", fn);
  if (!g) return fail(MR_EINVAL, "%s: gradient pointer is null", fn);
  if (!valid_dtype(g_dtype)) return fail(MR_EINVAL, "%s: unknown gradient dtype %d", fn, g_dtype);
  if (!update && !grad_v_out && !grad_alpha_out && !grad_beta_out)
    return fail(MR_EINVAL, "%s: nothing to do (no update, no gradient output)", fn);
  if (update && !(coef_lo <= coef_hi && v_bound >= 0.0f)) return fail(MR_EINVAL, "%s: bad bounds", fn);
  if (map.blk < 0 || map.stride < 0 || map.off < 0)
    return fail(MR_EINVAL, "%s: negative row placement", fn);
  if (map.blk && (rows * cols / 8 > 0x7fffffffLL || map.blk > 0x7fffffffLL))
    return fail(MR_EINVAL, "%s: placed tensor too large", fn);
  if (wq_out && !update) return fail(MR_EINVAL, "%s: W' is written only with the update", fn);
  if (lr_tab && (!step || lr_len < 1 || !update))
    return fail(MR_EINVAL, "%s: a rate schedule needs the step counter, its length and the update", fn);
  if (wq_out && !valid_dtype(wq_dtype)) return fail(MR_EINVAL, "%s: unknown W' dtype %d", fn, wq_dtype);
  if (wq_out && !aligned16(wq_out)) return fail(MR_EINVAL, "%s: W' must be 16-byte aligned", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  StepArgs st{lr, coef_lo, coef_hi, v_bound, wq_out, wq_dtype, lr_tab, step, lr_len};
#define MR_BWD(MODE_)                                                                       \
  return update ? launch_bwd<MODE_, true>(sh, w, w_dtype, v, alpha, beta, init_scale, g,     \
                                          g_dtype, eps, st, grad_v_out, grad_alpha_out,      \
                                          grad_beta_out, map, s)                             \
                : launch_bwd<MODE_, false>(sh, w, w_dtype, v, alpha, beta, init_scale, g,    \
                                           g_dtype, eps, st, grad_v_out, grad_alpha_out,     \
                                           grad_beta_out, map, s)
  if (mode == MR_ASYM) MR_BWD(MR_ASYM);
  if (mode == MR_SYM) MR_BWD(MR_SYM);
  MR_BWD(MR_SYM_SEARCHED);
#undef MR_BWD
}

int mr_fq_backward_signsgd(const void* w, int w_dtype, float* v, float* alpha, float* beta,
                           const float* init_scale, const void* g, int g_dtype, int64_t rows,
                           int64_t cols, int group_size, int bits, int mode, float eps,
                           int update, float lr, float coef_lo, float coef_hi, float v_bound,
                           float* grad_v_out, float* grad_alpha_out, float* grad_beta_out,
                           void* stream) {
  return fq_backward_impl("mr_fq_backward_signsgd", w, w_dtype, v, alpha, beta, init_scale, g,
                          g_dtype, rows, cols, group_size, bits, mode, eps, update, lr, coef_lo,
                          coef_hi, v_bound, grad_v_out, grad_alpha_out, grad_beta_out,
                          mr::RowMap{0, 0, 0, 0, {}, {}}, stream);
}

int mr_fq_backward_signsgd_mapped(const void* w, int w_dtype, float* v, float* alpha, float* beta,
                                  const float* init_scale, const void* g, int g_dtype,
                                  int64_t rows, int64_t cols, int group_size, int bits, int mode,
                                  float eps, float lr, float coef_lo, float coef_hi, float v_bound,
                                  int64_t row_block, int64_t row_stride, int64_t row_offset,
                                  void* stream) {
  return fq_backward_impl("mr_fq_backward_signsgd_mapped", w, w_dtype, v, alpha, beta, init_scale,
                          g, g_dtype, rows, cols, group_size, bits, mode, eps, 1, lr, coef_lo,
                          coef_hi, v_bound, nullptr, nullptr, nullptr,
                          mr::RowMap{row_block, row_stride, row_offset, 0, {}, {}}, stream);
}

int mr_fq_step_requant_mapped(const void* w, int w_dtype, float* v, float* alpha, float* beta,
                              const float* init_scale, const void* g, int g_dtype, int64_t rows,
                              int64_t cols, int group_size, int bits, int mode, float eps, float lr,
                              float coef_lo, float coef_hi, float v_bound, int64_t row_block,
                              int64_t row_stride, int64_t row_offset, void* wq_out, int wq_dtype,
                              void* stream) {
  if (!wq_out) {
    mr::clear_error();
    return mr::fail(MR_EINVAL, "mr_fq_step_requant_mapped: W' output is null");
  }
  return fq_backward_impl("mr_fq_step_requant_mapped", w, w_dtype, v, alpha, beta, init_scale, g,
                          g_dtype, rows, cols, group_size, bits, mode, eps, 1, lr, coef_lo, coef_hi,
                          v_bound, nullptr, nullptr, nullptr,
                          mr::RowMap{row_block, row_stride, row_offset, 0, {}, {}}, stream, wq_out, wq_dtype);
}

int mr_fq_step_requant_mapped_sched(const void* w, int w_dtype, float* v, float* alpha, float* beta,
                                    const float* init_scale, const void* g, int g_dtype,
                                    int64_t rows, int64_t cols, int group_size, int bits, int mode,
                                    float eps, const float* lr_table, int lr_len, const int* step,
                                    float coef_lo, float coef_hi, float v_bound, int64_t row_block,
                                    int64_t row_stride, int64_t row_offset, void* wq_out,
                                    int wq_dtype, void* stream) {
  if (!wq_out || !lr_table || !step) {
    mr::clear_error();
    return mr::fail(MR_EINVAL, "mr_fq_step_requant_mapped_sched: null W', schedule or step");
  }
  return fq_backward_impl("mr_fq_step_requant_mapped_sched", w, w_dtype, v, alpha, beta, init_scale,
                          g, g_dtype, rows, cols, group_size, bits, mode, eps, 1, 0.0f, coef_lo,
                          coef_hi, v_bound, nullptr, nullptr, nullptr,
                          mr::RowMap{row_block, row_stride, row_offset, 0, {}, {}}, stream, wq_out, wq_dtype,
                          lr_table, step, lr_len);
}

}  // extern "C"
