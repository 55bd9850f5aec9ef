// DeltaLoss accumulation for mixed-precision scoring, for gfx950.
//
// For one layer and a list of candidate widths, adds sum |g * (rtn_b(W) - W)|
// to each width's score, where rtn_b is round-to-nearest fake quantization at
// width b (mround/pipeline/scoring.py:213-221 and 262; oracle
// mround/planner/sensitivity.py:190-229). W and G are streamed once for all
// widths: the group extremes are shared, each width adds one division, one
// rounding and the product. Terms are formed in fp32 as the reference forms
// them; every term is added in fp64, per thread and across a fixed grid, so the
// result is deterministic and independent of the fp32 partial order.
//
// The gradient may be read through a row placement (the fused operands of the
// block GEMMs), and a searched symmetric scheme takes each width's scale grid
// instead of the observed range (mround/pipeline/scoring.py:196-221).
#include "mr_common.h"

namespace mr {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxWidths = 8;
constexpr int kBlocks = 1024;

struct DeltaWs {
  double partial[kMaxWidths][kBlocks];
};

struct Widths {
  int n;
  float maxq[kMaxWidths], qmin[kMaxWidths], qmax[kMaxWidths];
  const float* grid[kMaxWidths];  // searched scales (rows, n_groups), MR_SYM_SEARCHED only
};

// Gradient row r lives at row (r / blk) * stride + off + r % blk; blk == 0 is
// the identity.
struct GradMap {
  int64_t blk, stride, off, cpr;  // cpr: 8-element chunks per row
  __device__ __forceinline__ int64_t elem(int64_t chunk) const {
    if (!blk) return chunk * 8;
    const int64_t r = chunk / cpr;
    const int64_t pr = (r / blk) * stride + off + r % blk;
    return (pr * cpr + (chunk - r * cpr)) * 8;
  }
};

template <int WT, int MODE>
__global__ __launch_bounds__(kBlock) void delta_kernel(const void* __restrict__ w,
                                                       const float* __restrict__ g,
                                                       int64_t n_chunks, int tpg, int64_t gs,
                                                       Widths wd, GradMap gm, float eps,
                                                       DeltaWs* __restrict__ ws) {
  __shared__ double smem[kMaxWidths][kBlock / 64];
  double acc[kMaxWidths];
#pragma unroll
  for (int i = 0; i < kMaxWidths; ++i) acc[i] = 0.0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  // The stride is a multiple of 256, so the lanes of one group stay together.
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kBlock; base < n_chunks; base += stride) {
    int64_t chunk = base + threadIdx.x;
    const bool active = chunk < n_chunks;
    if (!active) chunk = n_chunks - 1;
    const int64_t e = chunk * 8;
    float x[8], gg[8];
    load8<WT>(w, e, x);
    load8_f32(g, gm.elem(chunk), gg);
    float mx = x[0], mn = x[0];
    if constexpr (MODE != MR_SYM_SEARCHED) {
#pragma unroll
      for (int k = 1; k < 8; ++k) {
        mx = fmaxf(mx, x[k]);
        mn = fminf(mn, x[k]);
      }
      for (int off = tpg >> 1; off > 0; off >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, off, tpg));
        mn = fminf(mn, __shfl_xor(mn, off, tpg));
      }
    }
    const float wmax = fmaxf(mx, 0.0f);
    const float wmin = fminf(mn, 0.0f);
    const int64_t grp = e / gs;
#pragma unroll
    for (int i = 0; i < kMaxWidths; ++i) {
      if (i >= wd.n) break;
      float s, zp = 0.0f;
      if constexpr (MODE == MR_ASYM) {
        s = fmaxf((wmax - wmin) / wd.maxq[i], eps);
        zp = rintf(-wmin / s);
      } else if constexpr (MODE == MR_SYM_SEARCHED) {
        const float base = wd.grid[i][grp];
        float sg = signf(base);
        sg = (sg == 0.0f) ? 1.0f : sg;
        s = sg * fmaxf(fabsf(base), eps);
      } else {
        const bool pos = wmax >= -wmin;
        const float dom = pos ? wmax : -wmin;
        const float sg0 = (pos ? -dom : dom) / wd.maxq[i];
        float sg = signf(sg0);
        sg = (sg == 0.0f) ? 1.0f : sg;
        s = sg * fmaxf(fabsf(sg0), eps);
      }
      double part = 0.0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        float raw = rintf(x[k] / s);
        float q;
        if constexpr (MODE == MR_ASYM) {
          raw = raw + zp;
          q = s * (clampf(raw, wd.qmin[i], wd.qmax[i]) - zp);
        } else {
          q = s * clampf(raw, wd.qmin[i], wd.qmax[i]);
        }
        part += static_cast<double>(fabsf(gg[k] * (q - x[k])));
      }
      if (active) acc[i] += part;
    }
  }
  const int wave = threadIdx.x / 64;
#pragma unroll
  for (int i = 0; i < kMaxWidths; ++i) {
    if (i >= wd.n) break;
    double v = acc[i];
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x % 64) == 0) smem[i][wave] = v;
  }
  __syncthreads();
  if (threadIdx.x < wd.n) {
    double t = 0.0;
    for (int j = 0; j < kBlock / 64; ++j) t += smem[threadIdx.x][j];
    ws->partial[threadIdx.x][blockIdx.x] = t;
  }
}

__global__ __launch_bounds__(kBlock) void delta_finalize(const DeltaWs* __restrict__ ws, int nparts,
                                                         int nw, double* __restrict__ scores) {
  __shared__ double smem[kBlock / 64];
  for (int i = 0; i < nw; ++i) {
    double acc = 0.0;
    for (int j = threadIdx.x; j < nparts; j += kBlock) acc += ws->partial[i][j];
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((threadIdx.x % 64) == 0) smem[threadIdx.x / 64] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
      double t = 0.0;
      for (int j = 0; j < kBlock / 64; ++j) t += smem[j];
      scores[i] += t;
    }
    __syncthreads();
  }
}

}  // namespace
}  // namespace mr

extern "C" {

size_t mr_delta_loss_workspace_bytes(int64_t rows, int64_t cols, int n_bits) {
  (void)rows;
  (void)cols;
  (void)n_bits;
  return sizeof(mr::DeltaWs);
}

int mr_delta_loss_mapped(const void* w, int w_dtype, const float* g, int64_t rows, int64_t cols,
                         int group_size, const int* bits_list, int n_bits, int mode, float eps,
                         const float* const* init_scales, int64_t g_row_block,
                         int64_t g_row_stride, int64_t g_row_offset, double* scores_out,
                         void* workspace, void* stream) {
  using namespace mr;
  clear_error();
  if (!w || !g || !bits_list || !scores_out || !workspace)
    return fail(MR_EINVAL, "mr_delta_loss: null pointer");
  if (n_bits < 1 || n_bits > kMaxWidths)
    return fail(MR_EINVAL, "mr_delta_loss: between 1 and %d widths, got %d", kMaxWidths, n_bits);
  if (mode != MR_ASYM && mode != MR_SYM && mode != MR_SYM_SEARCHED)
    return fail(MR_EINVAL, "mr_delta_loss: unknown mode %d", mode);
  if (w_dtype != MR_F32 && w_dtype != MR_BF16)
    return fail(MR_EINVAL, "mr_delta_loss: weights must be fp32 or bf16");
  const int64_t gs = group_size == -1 ? cols : group_size;
  const int64_t tpg = gs / 8;
  if (rows <= 0 || cols <= 0) return MR_OK;
  if (gs <= 0 || gs % 8 || cols % gs || tpg > 64 || (tpg & (tpg - 1)))
    return fail(MR_EINVAL,
                "mr_delta_loss: the group size must be 8 * 2^k <= 512 and divide the row (%lld, %lld)",
                static_cast<long long>(cols), static_cast<long long>(gs));
  if (!aligned16(w) || !aligned16(g)) return fail(MR_EINVAL, "mr_delta_loss: unaligned input");
  if (g_row_block < 0 || (g_row_block && (g_row_stride < g_row_block || g_row_offset < 0)))
    return fail(MR_EINVAL, "mr_delta_loss: bad gradient placement (block %lld, stride %lld, offset %lld)",
                static_cast<long long>(g_row_block), static_cast<long long>(g_row_stride),
                static_cast<long long>(g_row_offset));
  if (g_row_block && rows % g_row_block)
    return fail(MR_EINVAL, "mr_delta_loss: %lld rows do not split into placement blocks of %lld",
                static_cast<long long>(rows), static_cast<long long>(g_row_block));
  Widths wd{};
  wd.n = n_bits;
  for (int i = 0; i < n_bits; ++i) {
    int b = bits_list[i];
    if (b < 2 || b > 8) return fail(MR_EINVAL, "mr_delta_loss: bad width %d", b);
    if (mode == MR_ASYM) {
      wd.maxq[i] = static_cast<float>((1 << b) - 1);
      wd.qmin[i] = 0.0f;
      wd.qmax[i] = wd.maxq[i];
    } else {
      wd.maxq[i] = static_cast<float>(1 << (b - 1));
      wd.qmin[i] = -wd.maxq[i];
      wd.qmax[i] = wd.maxq[i] - 1.0f;
    }
    if (mode == MR_SYM_SEARCHED) {
      if (!init_scales || !init_scales[i])
        return fail(MR_EINVAL, "mr_delta_loss: the searched mode needs a scale grid per width");
      wd.grid[i] = init_scales[i];
    }
  }
  GradMap gm{g_row_block, g_row_stride, g_row_offset, cols / 8};
  const int64_t n_chunks = rows * cols / 8;
  int64_t want = (n_chunks + kBlock - 1) / kBlock;
  const int grid = static_cast<int>(want < kBlocks ? want : kBlocks);
  hipStream_t s = static_cast<hipStream_t>(stream);
  DeltaWs* ws = static_cast<DeltaWs*>(workspace);
  const int t = static_cast<int>(tpg);
#define MR_DELTA(WT, MODE) \
  hipLaunchKernelGGL((delta_kernel<WT, MODE>), dim3(grid), dim3(kBlock), 0, s, w, g, n_chunks, t, gs, wd, gm, eps, ws)
  if (w_dtype == MR_BF16) {
    if (mode == MR_ASYM) MR_DELTA(MR_BF16, MR_ASYM);
    else if (mode == MR_SYM) MR_DELTA(MR_BF16, MR_SYM);
    else MR_DELTA(MR_BF16, MR_SYM_SEARCHED);
  } else {
    if (mode == MR_ASYM) MR_DELTA(MR_F32, MR_ASYM);
    else if (mode == MR_SYM) MR_DELTA(MR_F32, MR_SYM);
    else MR_DELTA(MR_F32, MR_SYM_SEARCHED);
  }
#undef MR_DELTA
  hipLaunchKernelGGL(delta_finalize, dim3(1), dim3(kBlock), 0, s, ws, grid, n_bits, scores_out);
  MR_LAUNCH_CHECK("mr_delta_loss");
  return MR_OK;
}

int mr_delta_loss(const void* w, int w_dtype, const float* g, int64_t rows, int64_t cols,
                  int group_size, const int* bits_list, int n_bits, int mode, float eps,
                  double* scores_out, void* workspace, void* stream) {
  if (mode == MR_SYM_SEARCHED) {
    mr::clear_error();
    return mr::fail(MR_EINVAL, "mr_delta_loss: the searched mode takes scale grids "
                    "(mr_delta_loss_mapped)");
  }
  return mr_delta_loss_mapped(w, w_dtype, g, rows, cols, group_size, bits_list, n_bits, mode, eps,
                              nullptr, 0, 0, 0, scores_out, workspace, stream);
}

}  // extern "C"
