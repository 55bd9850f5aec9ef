// fp32 GEMMs on the MFMA cores of gfx950 (v_mfma_f32_32x32x2_f32): fp32
// operands, fp32 products and accumulation, for the products that must keep
// float32 precision: the single-layer tuning loop's layer residual
// x (W' - W)^T and weight gradient (dL/dr)^T x, which the reference forms in
// float32 (mround/core/tuning.py:140-190).
//
// C[M, N] = sum_k A(m, k) * (B(n, k) - B2(n, k)) (B2 optional), with each
// operand K-major (k contiguous) or MN-major (k the row index), as mr_gemm's
// layouts. Any sizes: tiles at the edges load zeros past the operand.
//
// A block of 256 threads (4 waves, 2 x 2) owns a 128 x 128 tile of C; each
// wave owns 64 x 64 as 2 x 2 accumulators of 32 x 32. Operand tiles of 32 k
// are staged through LDS by the whole block (each thread moves 16 values of
// each operand through registers, so B - B2 is formed on the way), stored
// k-major ([k][m]) so that an MFMA operand, 32 consecutive m (or n) at one k
// per lane half, is one conflict-free 4-byte read per lane. Operand loads of
// the next tile are issued before the MFMAs of the current one.
#include "mr_common.h"

namespace mr {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int TM = 128, TN = 128, TK = 32;
constexpr int kThreads = 256;
constexpr int PER = TM * TK / kThreads;  // operand values each thread moves per tile
constexpr int PAD = 4;                   // LDS row padding (floats)

// Value (r, k) of a K-major (x[r * ld + k]) or MN-major (x[k * ld + r])
// operand, zero outside rows x K.
template <bool KMAJOR>
__device__ __forceinline__ float at(const float* __restrict__ x, int64_t ld, int r, int k, int rows, int K) {
  if (r >= rows || k >= K) return 0.0f;
  return KMAJOR ? x[static_cast<int64_t>(r) * ld + k] : x[static_cast<int64_t>(k) * ld + r];
}

// Tile slot i of this thread: (r, k) within the 128 x 32 tile. K-major
// operands walk k fastest (consecutive threads read consecutive k of a row),
// MN-major ones r fastest (consecutive threads read consecutive r of a k-row).
template <bool KMAJOR>
__device__ __forceinline__ void slot(int i, int& r, int& k) {
  const int idx = i * kThreads + static_cast<int>(threadIdx.x);
  if constexpr (KMAJOR) {
    r = idx / TK;
    k = idx % TK;
  } else {
    k = idx / TM;
    r = idx % TM;
  }
}

template <bool A_KMAJOR, bool B_KMAJOR>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(int M, int N, int K, const float* __restrict__ A,
                                                            int64_t lda, const float* __restrict__ B,
                                                            const float* __restrict__ B2, int64_t ldb,
                                                            float* __restrict__ C, int64_t ldc) {
  __shared__ float As[TK][TM + PAD];
  __shared__ float Bs[TK][TN + PAD];
  const int m0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, kh = lane >> 5;

  float ra[PER], rb[PER];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int r, k;
      slot<A_KMAJOR>(i, r, k);
      ra[i] = at<A_KMAJOR>(A, lda, m0 + r, k0 + k, M, K);
      slot<B_KMAJOR>(i, r, k);
      const float b = at<B_KMAJOR>(B, ldb, n0 + r, k0 + k, N, K);
      rb[i] = B2 ? b - at<B_KMAJOR>(B2, ldb, n0 + r, k0 + k, N, K) : b;
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int r, k;
      slot<A_KMAJOR>(i, r, k);
      As[k][r] = ra[i];
      slot<B_KMAJOR>(i, r, k);
      Bs[k][r] = rb[i];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  load(0);
  for (int k0 = 0; k0 < K; k0 += TK) {
    __syncthreads();  // every read of the previous tile is done
    stash();
    __syncthreads();
    if (k0 + TK < K) load(k0 + TK);  // in flight during this tile's MFMAs
#pragma unroll
    for (int kk = 0; kk < TK; kk += 2) {
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = As[kk + kh][wm * 64 + i * 32 + l32];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = Bs[kk + kh][wn * 64 + j * 32 + l32];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[j], a[i], acc[i][j], 0, 0, 0);
    }
  }
  // B is the first MFMA operand, so accumulator register r of lane l holds
  // C[row m = l % 32][column n = (r / 4) * 8 + (l / 32) * 4 + r % 4] of its
  // 32 x 32 block: four consecutive columns per register group.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m = m0 + wm * 64 + i * 32 + l32;
      if (m >= M) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = n0 + wn * 64 + j * 32 + (r >> 2) * 8 + kh * 4 + (r & 3);
        if (n < N) C[static_cast<int64_t>(m) * ldc + n] = acc[i][j][r];
      }
    }
}

}  // namespace
}  // namespace mr

extern "C" {

int mr_gemm_f32(int layout, int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B,
                const float* B2, int64_t ldb, float* C, int64_t ldc, void* stream) {
  using namespace mr;
  clear_error();
  if (M < 0 || N < 0 || K < 0) return fail(MR_EINVAL, "mr_gemm_f32: negative size");
  if (M == 0 || N == 0) return MR_OK;
  if (!A || !B || !C) return fail(MR_EINVAL, "mr_gemm_f32: null operand");
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return fail(MR_EINVAL, "mr_gemm_f32: too large");
  if (layout < 0 || layout > 2) return fail(MR_EINVAL, "mr_gemm_f32: unknown layout %d", layout);
  const bool a_kmajor = layout != 2, b_kmajor = layout == 0;
  if (lda < (a_kmajor ? K : M) || ldb < (b_kmajor ? K : N) || ldc < N)
    return fail(MR_EINVAL, "mr_gemm_f32: a leading dimension is smaller than its row");
  if ((M + TM - 1) / TM > 65535) return fail(MR_EINVAL, "mr_gemm_f32: M above %d", 65535 * TM);
  const dim3 grid(static_cast<unsigned>((N + TN - 1) / TN), static_cast<unsigned>((M + TM - 1) / TM));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  switch (layout) {
    case 0:
      hipLaunchKernelGGL((gemm_f32_kernel<true, true>), grid, dim3(kThreads), 0, s, m, n, k, A, lda, B, B2, ldb, C,
                         ldc);
      break;
    case 1:
      hipLaunchKernelGGL((gemm_f32_kernel<true, false>), grid, dim3(kThreads), 0, s, m, n, k, A, lda, B, B2, ldb,
                         C, ldc);
      break;
    default:
      hipLaunchKernelGGL((gemm_f32_kernel<false, false>), grid, dim3(kThreads), 0, s, m, n, k, A, lda, B, B2, ldb,
                         C, ldc);
      break;
  }
  MR_LAUNCH_CHECK("mr_gemm_f32");
  return MR_OK;
}

}  // extern "C"
