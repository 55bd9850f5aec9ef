// bf16 GEMMs on the MFMA cores of gfx950, fp32 accumulation.
//
// C[M, N] = sum_k A(m, k) * B(n, k), with each operand stored either K-major
// (row-major with k contiguous: activations X[t, k], weights W[n, k]) or
// MN-major (k is the row index: dY[t, n] used as A(n, t) for dW = dY^T X, and
// W[k, n] used as B(n, k) for dX = dY W). The three products of a linear
// layer's forward and backward are therefore one kernel:
//   forward  Y  = X  W^T   A = X  (K-major)  B = W  (K-major)
//   input    dX = dY W     A = dY (K-major)  B = W  (MN-major)
//   weight   dW = dY^T X   A = dY (MN-major) B = X  (MN-major)
//
// Tiling: a block of 512 threads (8 waves of 64, 4 x 2) owns a BM x BN tile
// of C; each wave owns (BM/4) x (BN/2) as a grid of 32 x 32 accumulators fed by
// v_mfma_f32_32x32x16_bf16 (lane l: first operand row l%32, second operand
// row l%32, k half l/32; accumulator register r: first-operand index
// (r/4)*8 + (l/32)*4 + r%4, second-operand index l%32; the epilogues that
// stage their tile through LDS pass B first, so a lane holds one row of C and
// runs of 4 consecutive columns). Every
// operand tile moves HBM -> LDS by direct buffer loads (buffer_load ... lds,
// no registers) in the layout it has in memory: a K-major tile as rows of 64
// k, whose MFMA operand is one 16-byte LDS read; an MN-major tile as rows of
// one k, whose operand comes from two transposing LDS reads
// (ds_read_b64_tr_b16). Each lane's load offsets are fixed for the whole k
// loop (one 32-bit register per load); the k advance is in the scalar buffer
// base. The k loop is double-buffered in LDS with the next tile's loads in
// flight during the current tile's MFMAs, and within a tile the operands of
// the next k16 step are read while the current step's MFMAs run.
//
// Blocks are renumbered so that each XCD (blocks are dealt to the 8 XCDs
// round-robin) receives a contiguous run of tiles, grouped along M so that a
// run shares B panels in that XCD's L2.
#include <type_traits>

#include "mr_common.h"

namespace mr {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// 8 waves (two per SIMD) in a 4 x 2 grid: a 256 x 256 tile gives each wave
// 64 x 128 (128 accumulator registers), which leaves room for double-buffered
// operands and lets the two waves of a SIMD hide each other's LDS and
// barrier waits. A wave's columns start on a multiple of 64, which the SwiGLU
// epilogue's gate/up pairing needs.
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
// Waves 0-3 (one on each SIMD: the waves of a block are dealt to the four
// SIMDs so that waves w and w + 4 share one) issue every operand load of a
// tile, 16 each, right after the barrier; waves 4-7 go straight to their
// fragment reads and MFMAs. A wave stalls while the CU's load path takes its
// burst of direct loads, so this keeps one wave per SIMD issuing MFMAs at
// the start of every tile: measured 3-5 % faster on the 7B block's shapes
// than all eight waves loading (two loaders: 0-30 % slower).
constexpr int kLoaders = 4;
constexpr int kWaveRows = 4;  // waves along M
constexpr int BK = 64;
// LDS tiles are K-major rows of 64 bf16 (128 bytes, 8 chunks of 16 bytes)
// with no padding; chunk c of row r is stored at position c ^ ((r >> 1) & 7)
// (swz below), so the 16 rows one LDS cycle serves cover all 64 banks once.
constexpr int ROW_BYTES = BK * 2;

enum Epi : int {
  EPI_STORE = 0,   // C = acc (+ bias[n])
  EPI_RESID = 1,   // C = resid[m, n] + acc (+ bias[n]), fp32
  EPI_SWIGLU = 2,  // act = silu(g) * u from row-interleaved gate/up weights
  EPI_SWIGLU_BWD = 3,  // dgu (interleaved) from dact = acc and the saved gate/up
};

struct GemmParams {
  int M, N, K;
  const uint16_t* A;
  int64_t lda;
  const uint16_t* B;
  int64_t ldb;
  int n_out;           // SWIGLU: columns of act (B has 2 * n_out interleaved rows)
  void* C;
  int64_t ldc;
  const float* bias;
  const float* resid;
  int64_t ldr;
  uint16_t* gu;        // SWIGLU: gate/up copy, [M, 2 * n_out] bf16, interleaved like B
  int64_t ldgu;        // (SWIGLU_BWD reads the saved gate/up from gu and writes dgu to C)
  int grid_m, grid_n;
  // Tiles of this launch: logical tiles tile0 .. tile0 + n_tiles - 1 of the
  // grouped order. ksplit > 1: each tile's k steps are cut into ksplit runs
  // of kt_per steps (one block each), whose raw fp32 accumulators go to
  // ws[(tile - tile0) * ksplit + split] as BM x BN row-major partial tiles.
  int tile0, n_tiles, ksplit, kt_per;
  // sub = 1: this launch's tiles are the four quarters of each of the
  // (2 BM) x (2 BN) tiles tile0 .. of the grid_m x grid_n grid (see launch).
  int sub;
  float* ws;         // k-split partials (caller's workspace), or null: no split
  int64_t ws_bytes;
};

// Logical tile -> (tile row, tile column): groups of 8 tile rows, column by
// column within a group, so that consecutive tiles share B panels.
__device__ __forceinline__ void tile_coords(int lt, int grid_m, int grid_n, int& bm, int& bn) {
  constexpr int GROUP_M = 8;
  const int per_group = GROUP_M * grid_n;
  const int group = lt / per_group;
  const int first_m = group * GROUP_M;
  const int gm = min(grid_m - first_m, GROUP_M);
  bm = first_m + (lt % per_group) % gm;
  bn = (lt % per_group) / gm;
}

typedef __attribute__((address_space(3))) void lds_void_t;

// The wave's index in its block as a scalar, so that what derives from it
// (the direct loads' LDS addresses, the wave's tile offsets) stays in scalar
// registers.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }


// 16 lanes are served per LDS cycle: their 16 rows must cover the 64 banks.
// A row is 128 bytes (half the banks), so even and odd rows take the two
// halves and (row >> 1) & 7 spreads the 8 rows of each half over its 8
// 16-byte positions.
__device__ __forceinline__ int swz_bits(int row) { return (row >> 1) & 7; }

// ---- K-major operand: global -> LDS directly (global_load_lds, 16 B/lane) --
//
// One wave instruction moves 64 chunks = 8 rows; lane l covers row 8q + l/8
// and LDS position l % 8, i.e. global chunk (l % 8) ^ swz_bits(row). Rows past the
// valid range are clamped to the last valid row: they only feed accumulator
// rows or columns that are never stored.
// Buffer resource over `bytes` bytes from `base`. Every offset the loads use
// is already clamped inside the operand (see the loaders), so the resource
// bound is only a second fence.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcFlags = 0x00020000;  // raw 32-bit dwords, no swizzle
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                           static_cast<int>(bytes < 0x7fffffff ? bytes : 0x7fffffff),
                                           kRsrcFlags);
}

// 16 bytes per lane from the buffer into LDS at lds + 16 * lane. (Kept out of
// the templates: the host pass of hipcc drops the launch stubs of kernels
// whose templates call this builtin directly.)
__device__ __forceinline__ void load_lds16(rsrc_t r, uint8_t* lds, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, voff, 0, 0, 0);
}

template <int ROWS>
struct KMajorDirect {
  static constexpr int INSTR = ROWS * 8 / 64 / kLoaders;  // instructions per loading wave
  static_assert(INSTR * kLoaders * 64 == ROWS * 8, "the loading waves must cover every chunk of the tile");
  int voff[INSTR];
  __device__ __forceinline__ void init(int64_t ld, int row0, int rows_valid) {
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int sub = lane >> 3;
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      const int q = i * kLoaders + wave % kLoaders;
      const int row = q * 8 + sub;
      const int chunk = (lane & 7) ^ swz_bits(row);
      const int g = min(row0 + row, rows_valid - 1);
      voff[i] = static_cast<int>(((g - row0) * ld + chunk * 8) * 2);
    }
  }
  // The buffer over the operand from row row0, k0 on; then load i of this wave's INSTR into a stage.
  __device__ __forceinline__ static rsrc_t at(const uint16_t* base, int64_t ld, int row0, int rows_valid, int k0) {
    return make_rsrc(base + row0 * ld + k0, (static_cast<int64_t>(rows_valid - row0) * ld - k0) * 2);
  }
  __device__ __forceinline__ void issue_one(rsrc_t r, int i, uint8_t* lds) const {
    load_lds16(r, lds + (i * kLoaders + wave_id() % kLoaders) * 8 * ROW_BYTES, voff[i]);
  }
  __device__ __forceinline__ void issue(const uint16_t* base, int64_t ld, int row0, int rows_valid,
                                        int k0, uint8_t* lds) const {
    const uint16_t* b = base + row0 * ld + k0;
    const rsrc_t r = make_rsrc(b, (static_cast<int64_t>(rows_valid - row0) * ld - k0) * 2);
    const int wave = wave_id();
    if (wave >= kLoaders) return;
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      const int q = i * kLoaders + wave % kLoaders;
      load_lds16(r, lds + q * 8 * ROW_BYTES, voff[i]);
    }
  }
};

// ---- MN-major operand: element (row, k) at base[k * ld + row] -------------
//
// Staged as it lies in memory: BK rows (one per k) of ROWS bf16, moved
// HBM -> LDS by direct loads like the K-major tiles, no registers and no
// shuffles. Chunk c of k-row r sits at position c ^ (4 (r & 3)), so the four
// k-rows one transposing read touches land on distinct banks. The MFMA
// operand (8 consecutive k of one m) comes from two ds_read_b64_tr_b16: in
// each 16-lane group, lane i receives element i % 4 of the 8 bytes addressed
// by lane 4 j + i / 4 (j = 0..3); with source lane s addressing k-row
// k0 + s / 4 at column c0 + 4 (s % 4), lane i gets k0..k0+3 of column c0 + i.
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef short v8i16 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16_t;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8_t;

template <int ROWS>
struct MNMajorDirect {
  static constexpr int CPR = ROWS / 8;         // 16-byte chunks per k-row
  static constexpr int RPI = 64 / CPR;         // k-rows per wave instruction
  static constexpr int INSTR = BK / RPI / kLoaders;   // instructions per loading wave
  static_assert(INSTR * kLoaders * RPI == BK, "the loading waves must cover every k-row of the tile");
  static constexpr int ROWB = ROWS * 2;        // bytes per k-row
  int voff[INSTR];
  __device__ __forceinline__ void init(int64_t ld, int row0, int rows_valid) {
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int sub = lane / CPR, pchunk = lane % CPR;
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      const int kb = (i * kLoaders + wave % kLoaders) * RPI;
      const int kr = kb + sub;
      const int c = pchunk ^ (4 * (kr & 3));
      const int col = min(row0 + c * 8, rows_valid - 8);
      voff[i] = static_cast<int>((kr * ld + (col - row0)) * 2);
    }
  }
  __device__ __forceinline__ static rsrc_t at(const uint16_t* base, int64_t ld, int row0, int K, int k0) {
    return make_rsrc(base + static_cast<int64_t>(k0) * ld + row0, (static_cast<int64_t>(K - k0) * ld - row0) * 2);
  }
  __device__ __forceinline__ void issue_one(rsrc_t r, int i, uint8_t* lds) const {
    load_lds16(r, lds + (i * kLoaders + wave_id() % kLoaders) * RPI * ROWB, voff[i]);
  }
  __device__ __forceinline__ void issue(const uint16_t* base, int64_t ld, int row0, int K, int k0,
                                        uint8_t* lds) const {
    const uint16_t* b = base + static_cast<int64_t>(k0) * ld + row0;
    const rsrc_t r = make_rsrc(b, (static_cast<int64_t>(K - k0) * ld - row0) * 2);
    const int wave = wave_id();
    if (wave >= kLoaders) return;
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      const int kb = (i * kLoaders + wave % kLoaders) * RPI;
      load_lds16(r, lds + kb * ROWB, voff[i]);
    }
  }
  // Lane-dependent byte offset of the k16-step-0 operand for rows rbase.. of
  // a stage (the low 8 bytes; the high 8 are 4 k-rows further, step kk is
  // 16 kk k-rows further).
  __device__ __forceinline__ static uint32_t frag_off(int rbase, int lane) {
    const int h = lane >> 5, q = (lane >> 4) & 1, i = lane & 15;
    const int c = (rbase + q * 16) / 8 + ((i & 3) >> 1);
    return (8 * h + (i >> 2)) * ROWB + ((c ^ (4 * (i >> 2))) << 4) + (i & 1) * 8;
  }
};

// An epilogue's 16-byte global store; NT marks it non-temporal. Measured on
// the 7B block: the plain-store epilogues (the gradients, q/k/v) run 1-2 %
// faster with it, the SwiGLU backward the same, and the SwiGLU forward and
// the in-place residual add 0.7 and 1.5 % slower, so those keep plain stores.
template <bool NT, typename T>
__device__ __forceinline__ void store16(T* p, T v) {
  static_assert(sizeof(T) == 16, "16-byte stores only");
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// The epilogues of a wave's WM x WN share of a tile from its transposed
// accumulators (see SWAP in the kernels), staged through the wave's REGION
// bytes of LDS at `region` (free once the k loop has ended).
template <int WM, int WN, int REGION, int EPI, bool OUT_BF16, int TM, int TN>
__device__ __forceinline__ void store_tile(const GemmParams& p, f32x16 (&acc)[TM][TN], int m0, int n0, int wm,
                                           int wn, int lane, uint8_t* region) {
  const int lrow = (lane >> 5) * 4;
  const int lcol = lane & 31;
  if constexpr (EPI == EPI_SWIGLU) {
    // B rows interleave 32 gate rows and 32 up rows, and a wave's column
    // range starts on a multiple of 64: block j = 2q holds gate columns and
    // j = 2q + 1 the up columns of the same 32 act columns (accumulators are
    // transposed, see SWAP). Each 32-row slice of the wave's accumulators (JH
    // column blocks at a time, gate and up pairs whole) is staged as fp32 in
    // the wave's LDS share; then a lane takes 8 consecutive act columns of one
    // row, reads their gate and up values, and writes act and the bf16 gate
    // and up copies as one 16-byte store each: whole cache lines instead of
    // 64-byte row pieces. (Computing act while staging made the compiler read
    // the accumulators out of the AGPRs ahead of the silu chains and spill.)
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
    // Rows are not padded (32 rows of two blocks fill the 8-wave 128 x 128
    // kernel's 8 KB share); instead the 16-byte chunk c of row r sits at
    // chunk c ^ (r % 16), which spreads a write's 32 rows over all banks.
    constexpr int JH = (32 * TN * 32 * 4 <= REGION) ? TN : 2;
    constexpr int PITCH = JH * 32 * 4;
    constexpr int CH = JH * 16 / 8;  // 8-column act pieces per staged row
    constexpr int NIT = 32 * CH / 64;
    static_assert(32 * PITCH <= REGION && TN % JH == 0 && JH % 2 == 0 && NIT * 64 == 32 * CH,
                  "SwiGLU staging does not fit the wave's LDS share");
    auto at = [](int r, int c) __attribute__((always_inline)) { return r * PITCH + ((c ^ (r & 15)) << 4); };
    lds_u8* st = (lds_u8*)region;
    uint16_t* act = static_cast<uint16_t*>(p.C);
    const bool has_gu = p.gu != nullptr;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int jb = 0; jb < TN / JH; ++jb) {
#pragma unroll
        for (int jj = 0; jj < JH; ++jj) {
          const int j = jb * JH + jj;
#pragma unroll
          for (int gi = 0; gi < 4; ++gi)
            *(lds_f32x4*)(st + at(lcol, jj * 8 + gi * 2 + lrow / 4)) =
                f32x4{acc[i][j][4 * gi], acc[i][j][4 * gi + 1], acc[i][j][4 * gi + 2], acc[i][j][4 * gi + 3]};
        }
        // The same wave reads back what it wrote (LDS keeps a wave's accesses
        // in order), then the next slice overwrites the region.
        const int row0 = m0 + wm * WM + i * 32;
        const int col0 = n0 + wn * WN + jb * JH * 32;  // gate/up column, a multiple of 64
        // uniform bases of the slice; lane offsets stay 32-bit (ld < 2^22, 32 rows)
        uint16_t* const act_s = act + static_cast<int64_t>(row0) * p.ldc + col0 / 2;
        uint16_t* const gu_s = p.gu + static_cast<int64_t>(row0) * p.ldgu + col0;
        // (a slice wholly inside the outputs stores without per-lane guards,
        // as in the plain epilogue; N is a multiple of 32, so an act piece and
        // its gate and up pieces lie inside or past the edge together)
        auto out = [&](auto guardc, auto guc) __attribute__((always_inline)) {
          constexpr bool GUARD = decltype(guardc)::value, GU = decltype(guc)::value;
#pragma unroll
          for (int it = 0; it < NIT; ++it) {
            const int idx = it * 64 + lane, r = idx / CH, ch = idx % CH;
            const int gc = (ch >> 2) * 64 + (ch & 3) * 8;  // staged gate column; up 32 further
            const f32x4 g0 = *(const lds_f32x4*)(st + at(r, gc / 4)), g1 = *(const lds_f32x4*)(st + at(r, gc / 4 + 1));
            const f32x4 u0 = *(const lds_f32x4*)(st + at(r, gc / 4 + 8)), u1 = *(const lds_f32x4*)(st + at(r, gc / 4 + 9));
            if (!GUARD || (row0 + r < p.M && col0 / 2 + ch * 8 < p.n_out)) {
              float a[8];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                a[e] = silu(g0[e]) * u0[e];
                a[e + 4] = silu(g1[e]) * u1[e];
              }
              store16<false>(reinterpret_cast<u32x4*>(act_s + static_cast<uint32_t>(r * static_cast<int>(p.ldc) + ch * 8)),
                      u32x4{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(a[4], a[5]),
                            pack_bf16x2(a[6], a[7])});
              if constexpr (GU) {
                uint16_t* const o = gu_s + static_cast<uint32_t>(r * static_cast<int>(p.ldgu) + gc);
                store16<false>(reinterpret_cast<u32x4*>(o), u32x4{pack_bf16x2(g0[0], g0[1]), pack_bf16x2(g0[2], g0[3]),
                                                           pack_bf16x2(g1[0], g1[1]), pack_bf16x2(g1[2], g1[3])});
                store16<false>(reinterpret_cast<u32x4*>(o + 32), u32x4{pack_bf16x2(u0[0], u0[1]), pack_bf16x2(u0[2], u0[3]),
                                                                pack_bf16x2(u1[0], u1[1]), pack_bf16x2(u1[2], u1[3])});
              }
            }
          }
        };
        const bool full = row0 + 32 <= p.M && col0 / 2 + JH * 16 <= p.n_out;
        if (has_gu) {
          if (full) out(std::false_type{}, std::true_type{});
          else out(std::true_type{}, std::true_type{});
        } else {
          if (full) out(std::false_type{}, std::false_type{});
          else out(std::true_type{}, std::false_type{});
        }
      }
    }
  } else if constexpr (EPI == EPI_SWIGLU_BWD) {
    // acc is dact transposed (SWAP): lane l holds row l % 32 of block (i, j)
    // and, in register group gi, act columns j 32 + 8 gi + 4 (l / 32) .. + 3.
    // Each 32-row slice of the wave's dact (JH column blocks at a time) is
    // staged as fp32 in the wave's LDS share; then a lane takes 8 consecutive
    // act columns of one row: their gate and up values are one 16-byte load
    // each from the saved interleaved gate/up (gate of act column c at
    // (c / 32) 64 + c % 32, up 32 further), all of a slice's loads in flight
    // before any is used, and dgate and dup leave as one 16-byte store each
    // at the same places.
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    constexpr int JH = (32 * (TN * 32 * 4 + 16) <= REGION) ? TN : (32 * (2 * 32 * 4 + 16) <= REGION ? 2 : 1);
    constexpr int PITCH = JH * 32 * 4 + 16;
    constexpr int CH = JH * 32 / 8;  // 8-column pieces per staged row
    constexpr int NIT = 32 * CH / 64;
    static_assert(32 * PITCH <= REGION && TN % JH == 0 && NIT * 64 == 32 * CH, "staging does not fit");
    lds_u8* st = (lds_u8*)region;
    uint16_t* dgu = static_cast<uint16_t*>(p.C);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int jb = 0; jb < TN / JH; ++jb) {
#pragma unroll
        for (int jj = 0; jj < JH; ++jj) {
          const int j = jb * JH + jj;
#pragma unroll
          for (int gi = 0; gi < 4; ++gi)
            *(__attribute__((address_space(3))) f32x4*)(st + lcol * PITCH + (jj * 32 + gi * 8 + lrow) * 4) =
                f32x4{acc[i][j][4 * gi], acc[i][j][4 * gi + 1], acc[i][j][4 * gi + 2], acc[i][j][4 * gi + 3]};
        }
        // The same wave reads back what it wrote (LDS keeps a wave's accesses
        // in order). Loads go to clamped (always valid) places; only the
        // stores are guarded.
        const int row0 = m0 + wm * WM + i * 32;
        const int col0 = n0 + wn * WN + jb * JH * 32;
        const uint16_t* const gu_s = p.gu + static_cast<int64_t>(row0) * p.ldgu;
        uint16_t* const dgu_s = dgu + static_cast<int64_t>(row0) * p.ldc;
        u32x4 gv[NIT], uv[NIT];
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
          const int idx = it * 64 + lane, r = idx / CH, ch = idx % CH;
          const int row = min(row0 + r, p.M - 1), col = min(col0 + ch * 8, p.N - 8);
          // signed: a slice wholly past the edge clamps to row M - 1, below row0
          const int o = (row - row0) * static_cast<int>(p.ldgu) + (col >> 5) * 64 + (col & 31);
          gv[it] = *reinterpret_cast<const u32x4*>(gu_s + o);
          uv[it] = *reinterpret_cast<const u32x4*>(gu_s + o + 32);
        }
        auto out = [&](auto guardc) __attribute__((always_inline)) {  // (guards as in the plain epilogue)
          constexpr bool GUARD = decltype(guardc)::value;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
          const int idx = it * 64 + lane, r = idx / CH, ch = idx % CH;
          const int row = row0 + r, col = col0 + ch * 8;
          const f32x4 d0 = *(__attribute__((address_space(3))) f32x4*)(st + r * PITCH + ch * 32);
          const f32x4 d1 = *(__attribute__((address_space(3))) f32x4*)(st + r * PITCH + ch * 32 + 16);
          const float da[8] = {d0[0], d0[1], d0[2], d0[3], d1[0], d1[1], d1[2], d1[3]};
          float dg[8], du[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t gw = gv[it][e >> 1], uw = uv[it][e >> 1];
            const float g = __uint_as_float((e & 1) ? (gw & 0xffff0000u) : (gw << 16));
            const float u = __uint_as_float((e & 1) ? (uw & 0xffff0000u) : (uw << 16));
            const float sg = sigmoid(g);
            const float dsilu = sg * (1.0f + g * (1.0f - sg));
            dg[e] = da[e] * u * dsilu;
            du[e] = da[e] * g * sg;
          }
          if (!GUARD || (row < p.M && col < p.N)) {
            const uint32_t od = static_cast<uint32_t>(r * static_cast<int>(p.ldc) + (col >> 5) * 64 + (col & 31));
            store16<true>(reinterpret_cast<u32x4*>(dgu_s + od), u32x4{pack_bf16x2(dg[0], dg[1]), pack_bf16x2(dg[2], dg[3]),
                                                              pack_bf16x2(dg[4], dg[5]), pack_bf16x2(dg[6], dg[7])});
            store16<true>(reinterpret_cast<u32x4*>(dgu_s + od + 32), u32x4{pack_bf16x2(du[0], du[1]), pack_bf16x2(du[2], du[3]),
                                                                   pack_bf16x2(du[4], du[5]), pack_bf16x2(du[6], du[7])});
          }
        }
        };
        if (row0 + 32 <= p.M && col0 + JH * 32 <= p.N) out(std::false_type{});
        else out(std::true_type{});
      }
    }
  } else {  // EPI_STORE, EPI_RESID
    // The transposed accumulators are staged in fp32 per 32-row slice and JH
    // column blocks in the wave's LDS share, then leave as 16-byte row pieces
    // (bias, residual and the bf16 rounding applied on the way): whole cache
    // lines instead of 64-byte (bf16) row pieces, and a quarter of the store
    // instructions. Measured on the 7B block: q/k/v projection 9 %,
    // attention-output input gradient 10 %, fp32 outputs 1-4 % faster. (With
    // the bias added while staging, its branch made the compiler read every
    // accumulator out of the AGPRs ahead of it, 256 values, and spill.)
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
    constexpr int JH = (32 * (TN * 32 * 4 + 16) <= REGION) ? TN : (32 * (2 * 32 * 4 + 16) <= REGION ? 2 : 1);
    constexpr int PITCH = JH * 32 * 4 + 16;
    constexpr int OPC = OUT_BF16 ? 8 : 4;   // output columns per 16-byte store
    constexpr int CH = JH * 32 / OPC;       // stores per staged row
    constexpr int NIT = 32 * CH / 64;
    static_assert(32 * PITCH <= REGION && TN % JH == 0 && NIT * 64 == 32 * CH, "staging does not fit");
    static_assert(EPI == EPI_STORE || !OUT_BF16, "the residual epilogue writes fp32");
    lds_u8* st = (lds_u8*)region;
    const bool has_bias = p.bias != nullptr;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int jb = 0; jb < TN / JH; ++jb) {
#pragma unroll
        for (int jj = 0; jj < JH; ++jj) {
          const int j = jb * JH + jj;
#pragma unroll
          for (int gi = 0; gi < 4; ++gi)
            *(lds_f32x4*)(st + lcol * PITCH + (jj * 32 + gi * 8 + lrow) * 4) =
                f32x4{acc[i][j][4 * gi], acc[i][j][4 * gi + 1], acc[i][j][4 * gi + 2], acc[i][j][4 * gi + 3]};
        }
        const int row0 = m0 + wm * WM + i * 32;
        const int col0 = n0 + wn * WN + jb * JH * 32;
        // uniform bases of the slice; lane offsets stay 32-bit (ld < 2^22, 32 rows)
        const int64_t cbase = static_cast<int64_t>(row0) * p.ldc + col0;
        uint16_t* const cb16 = static_cast<uint16_t*>(p.C) + cbase;
        float* const cb32 = static_cast<float*>(p.C) + cbase;
        f32x4 res[EPI == EPI_RESID ? NIT : 1];
        if constexpr (EPI == EPI_RESID) {
          // every residual piece of the slice in flight before any store
          // (the output may be the residual itself, so stores cannot move ahead)
          const float* const rs = p.resid + static_cast<int64_t>(row0) * p.ldr;
#pragma unroll
          for (int it = 0; it < NIT; ++it) {
            const int idx = it * 64 + lane, r = idx / CH, ch = idx % CH;
            const int row = min(row0 + r, p.M - 1), col = min(col0 + ch * 4, p.N - 4);
            // signed: a slice wholly past the edge clamps to row M - 1, below row0
            res[it] = *reinterpret_cast<const f32x4*>(rs + ((row - row0) * static_cast<int>(p.ldr) + col));
          }
        }
        // A slice wholly inside the output stores without per-lane guards:
        // guarded stores each become a branch region of their own, and the
        // LDS reads then wait one by one instead of being in flight together.
        auto out = [&](auto biasc, auto guardc) __attribute__((always_inline)) {
          constexpr bool BIAS = decltype(biasc)::value, GUARD = decltype(guardc)::value;
#pragma unroll
          for (int it = 0; it < NIT; ++it) {
            const int idx = it * 64 + lane, r = idx / CH, ch = idx % CH;
            const int row = row0 + r, col = col0 + ch * OPC;
            const uint32_t oc = static_cast<uint32_t>(r * static_cast<int>(p.ldc) + ch * OPC);
            if (!GUARD || (row < p.M && col < p.N)) {
              // N is a multiple of 8: a store's columns lie wholly inside or past the edge
              const int cb = GUARD ? min(col, p.N - OPC) : col;
              f32x4 w = *(lds_f32x4*)(st + r * PITCH + ch * OPC * 4);
              if constexpr (BIAS) w += f32x4{p.bias[cb], p.bias[cb + 1], p.bias[cb + 2], p.bias[cb + 3]};
              if constexpr (OUT_BF16) {
                typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                f32x4 w2 = *(lds_f32x4*)(st + r * PITCH + ch * OPC * 4 + 16);
                if constexpr (BIAS)
                  w2 += f32x4{p.bias[cb + 4], p.bias[cb + 5], p.bias[cb + 6], p.bias[cb + 7]};
                store16<true>(reinterpret_cast<u32x4*>(cb16 + oc),
                        u32x4{pack_bf16x2(w[0], w[1]), pack_bf16x2(w[2], w[3]), pack_bf16x2(w2[0], w2[1]),
                              pack_bf16x2(w2[2], w2[3])});
              } else {
                if constexpr (EPI == EPI_RESID) w = res[it] + w;
                store16<EPI == EPI_STORE>(reinterpret_cast<f32x4*>(cb32 + oc), w);
              }
            }
          }
        };
        const bool full = row0 + 32 <= p.M && col0 + JH * 32 <= p.N;
        if (has_bias) {
          if (full) out(std::true_type{}, std::false_type{});
          else out(std::true_type{}, std::true_type{});
        } else {
          if (full) out(std::false_type{}, std::false_type{});
          else out(std::false_type{}, std::true_type{});
        }
      }
    }
  }
}

template <int BM, int BN, bool A_KMAJOR, bool B_KMAJOR, int EPI, bool OUT_BF16>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GemmParams p) {
  constexpr int WM = BM / kWaveRows, WN = BN / (kWaves / kWaveRows);
  constexpr int TM = WM / 32, TN = WN / 32;
  // Every epilogue feeds the MFMA with B as the first operand and A as the
  // second, so that each accumulator holds C transposed: lane l then owns row
  // l % 32 of its 32 x 32 block and, in register group gi, the 4 consecutive
  // columns 8 gi + 4 (l / 32) .. + 3, which the epilogue writes to LDS as one
  // 8- or 16-byte piece. (Every output element is the same k-ordered sum
  // either way.)
  constexpr bool SWAP = true;
  // Two LDS stages as four distinct arrays, indexed only with compile-time
  // stage numbers (the k loop below is unrolled by two), so that the waits
  // for the direct-to-LDS loads into one stage are not placed in front of the
  // operand reads of the other.
  __shared__ __attribute__((aligned(1024))) uint8_t As0[BM * ROW_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t As1[BM * ROW_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t Bs0[BN * ROW_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t Bs1[BN * ROW_BYTES];

  // XCD-aware renumbering (each XCD gets a contiguous run of the launch's
  // tiles), then the grouped order along M. Split launches take the splits
  // of one tile as consecutive blocks.
  int bid = blockIdx.x, split = 0;
  if (p.ksplit > 1) {
    split = bid % p.ksplit;
    bid /= p.ksplit;
  } else if ((p.n_tiles & 7) == 0) {
    bid = (bid & 7) * (p.n_tiles >> 3) + (bid >> 3);
  }
  int bm, bn;
  if (p.sub) {
    tile_coords(p.tile0 + (bid >> 2), p.grid_m, p.grid_n, bm, bn);
    bm = 2 * bm + ((bid >> 1) & 1);
    bn = 2 * bn + (bid & 1);
  } else {
    tile_coords(p.tile0 + bid, p.grid_m, p.grid_n, bm, bn);
  }
  const int m0 = bm * BM;
  const int n0 = bn * BN;
  if (m0 >= p.M || n0 >= p.N) return;  // a quarter wholly past the edge (the whole block leaves)

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int wm = wave / (kWaves / kWaveRows), wn = wave % (kWaves / kWaveRows);

  // Global loads of tile kt, straight into the given LDS stage.
  std::conditional_t<A_KMAJOR, KMajorDirect<BM>, MNMajorDirect<BM>> ld_a;
  std::conditional_t<B_KMAJOR, KMajorDirect<BN>, MNMajorDirect<BN>> ld_b;
  ld_a.init(p.lda, m0, p.M);
  ld_b.init(p.ldb, n0, p.N);
  auto issue_loads = [&](int kt, uint8_t* as_dst, uint8_t* bs_dst) {
    const int k0 = kt * BK;
    if constexpr (A_KMAJOR) ld_a.issue(p.A, p.lda, m0, p.M, k0, as_dst);
    else ld_a.issue(p.A, p.lda, m0, p.K, k0, as_dst);
    if constexpr (B_KMAJOR) ld_b.issue(p.B, p.ldb, n0, p.N, k0, bs_dst);
    else ld_b.issue(p.B, p.ldb, n0, p.K, k0, bs_dst);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16{};

  // MFMAs over one LDS stage, with the operands of the next k16 step read
  // while the current step's MFMAs run.
  // Every k step, fragment slot and accumulator is visited with compile-time
  // indices (StaticFor): left to the loop unroller, a body this large can
  // stay rolled, and a runtime index would move acc and the fragments to
  // scratch memory.
  // LDS operand addresses: the lane-dependent parts are computed once and
  // hidden from the optimizer, so that every operand read is its stage
  // array plus one of these registers plus an immediate (tile, k step). Left
  // alone, the compiler folds the tile and step offsets into a separate
  // register per read and runs out of room for the next step's operands.
  // The reads keep naming their stage array so that the waits for the
  // direct loads into one stage are not put in front of reads of the other.
  constexpr int NA = A_KMAJOR ? BK / 16 : TM, NB = B_KMAJOR ? BK / 16 : TN;
  uint32_t a_reg[NA], b_reg[NB];
  {
    const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int x = 0; x < NA; ++x) {
      if constexpr (A_KMAJOR)
        a_reg[x] = (wm * WM + l32) * ROW_BYTES + (((2 * x + h) ^ swz_bits(l32)) << 4);
      else
        a_reg[x] = MNMajorDirect<BM>::frag_off(wm * WM + x * 32, lane);
      asm volatile("" : "+v"(a_reg[x]));
    }
#pragma unroll
    for (int x = 0; x < NB; ++x) {
      if constexpr (B_KMAJOR)
        b_reg[x] = (wn * WN + l32) * ROW_BYTES + (((2 * x + h) ^ swz_bits(l32)) << 4);
      else
        b_reg[x] = MNMajorDirect<BN>::frag_off(wn * WN + x * 32, lane);
      asm volatile("" : "+v"(b_reg[x]));
    }
  }
  typedef const __attribute__((address_space(3))) uint8_t* lds_ptr;

  // MFMAs over one LDS stage, with the operands of the next k16 step read
  // while the current step's MFMAs run.
  // Every k step, fragment slot and accumulator is visited with compile-time
  // indices (StaticFor): left to the loop unroller, a body this large can
  // stay rolled, and a runtime index would move acc and the fragments to
  // scratch memory.
  auto compute = [&](auto stagec) {
    constexpr int st = decltype(stagec)::value;
    const lds_ptr la = (lds_ptr)(st ? As1 : As0);
    const lds_ptr lb = (lds_ptr)(st ? Bs1 : Bs0);
    bf16x8 af[2][TM], bfr[2][TN];
    auto read_frags = [&](auto kkc, auto slotc) {
      constexpr int kk = decltype(kkc)::value, slot = decltype(slotc)::value;
      auto ra = [&](auto ic) {
        constexpr int i = decltype(ic)::value;
        if constexpr (A_KMAJOR) {
          af[slot][i] = *(const lds_bf16x8_t*)(la + a_reg[kk] + i * 32 * ROW_BYTES);
        } else {
          constexpr uint32_t R = MNMajorDirect<BM>::ROWB;
          const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(la + a_reg[i] + kk * 16 * R));
          const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(la + a_reg[i] + kk * 16 * R + 4 * R));
          af[slot][i] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
      };
      auto rb = [&](auto jc) {
        constexpr int j = decltype(jc)::value;
        if constexpr (B_KMAJOR) {
          bfr[slot][j] = *(const lds_bf16x8_t*)(lb + b_reg[kk] + j * 32 * ROW_BYTES);
        } else {
          constexpr uint32_t R = MNMajorDirect<BN>::ROWB;
          const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(lb + b_reg[j] + kk * 16 * R));
          const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(lb + b_reg[j] + kk * 16 * R + 4 * R));
          bfr[slot][j] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
      };
      StaticFor<0, TM>::run(ra);
      StaticFor<0, TN>::run(rb);
    };
    read_frags(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    auto kstep = [&](auto kkc) {
      constexpr int kk = decltype(kkc)::value, cur = kk & 1;
      if constexpr (kk + 1 < BK / 16)
        read_frags(std::integral_constant<int, kk + 1>{}, std::integral_constant<int, cur ^ 1>{});
      // The next step's reads stay in front of this step's MFMAs (otherwise
      // the scheduler moves them behind and reuses the same registers).
      __builtin_amdgcn_sched_barrier(0);
      auto mm = [&](auto ijc) {
        constexpr int i = decltype(ijc)::value / TN, j = decltype(ijc)::value % TN;
        if constexpr (SWAP)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[cur][j], af[cur][i], acc[i][j], 0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[cur][i], bfr[cur][j], acc[i][j], 0, 0, 0);
      };
      StaticFor<0, TM * TN>::run(mm);
    };
    StaticFor<0, BK / 16>::run(kstep);
  };

  // One pipeline step: compute on stage `cur` while tile kt + 1 moves into
  // the other stage, then a barrier.
  auto step = [&](int kt, int KT, auto curc) {
    constexpr int cur = decltype(curc)::value;
    if (kt + 1 < KT) issue_loads(kt + 1, cur ? As0 : As1, cur ? Bs0 : Bs1);
    // Keep the loads of the next tile ahead of this tile's MFMAs: left to
    // itself the scheduler sinks them to the end of the step, right in front
    // of the wait for them, and the whole memory latency is exposed.
    __builtin_amdgcn_sched_barrier(0);
    compute(curc);
    // The direct loads of the next tile and every read of this one are done
    // before any wave moves on.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };

  const int kt_begin = split * p.kt_per;
  const int KT = min(p.K / BK, kt_begin + p.kt_per);
  if (kt_begin < KT) {
    issue_loads(kt_begin, As0, Bs0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int kt = kt_begin;
    for (; kt + 1 < KT; kt += 2) {
      step(kt, KT, std::integral_constant<int, 0>{});
      step(kt + 1, KT, std::integral_constant<int, 1>{});
    }
    if (kt < KT) step(kt, KT, std::integral_constant<int, 0>{});
  }

  // ---- epilogue ----
  const int lrow = (lane >> 5) * 4;
  const int lcol = lane & 31;
  if (p.ksplit > 1) {  // raw partial tile; the reduce kernel applies the epilogue
    float* out = p.ws + (static_cast<int64_t>(bid) * p.ksplit + split) * (BM * BN);
    auto tile = [&](auto ij) {
      constexpr int i = decltype(ij)::value / TN, j = decltype(ij)::value % TN;
      if constexpr (SWAP) {
#pragma unroll
        for (int gi = 0; gi < 4; ++gi)
          *reinterpret_cast<float4*>(out + (wm * WM + i * 32 + lcol) * BN + wn * WN + j * 32 + gi * 8 + lrow) =
              make_float4(acc[i][j][4 * gi], acc[i][j][4 * gi + 1], acc[i][j][4 * gi + 2], acc[i][j][4 * gi + 3]);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          out[(wm * WM + i * 32 + (r >> 2) * 8 + lrow + (r & 3)) * BN + wn * WN + j * 32 + lcol] =
              acc[i][j][r];
      }
    };
    StaticFor<0, TM * TN>::run(tile);
    return;
  }
  {
    constexpr int REGION = (BM + BN) * ROW_BYTES * 2 / kWaves;  // bytes of LDS per wave
    static_assert(2 * REGION == BM * ROW_BYTES && 2 * REGION == BN * ROW_BYTES, "two waves per LDS array");
    uint8_t* arr = wave < 2 ? As0 : wave < 4 ? As1 : wave < 6 ? Bs0 : Bs1;
    store_tile<WM, WN, REGION, EPI, OUT_BF16>(p, acc, m0, n0, wm, wn, lane, arr + (wave & 1) * REGION);
  }
}


// ---- 4-wave kernel for 256 x 256 tiles ---------------------------------------
//
// One wave per SIMD, each owning 128 x 128 of the tile (256 accumulator
// registers, held in AGPRs): half the LDS operand reads per MFMA of the 8-wave
// kernel (4 A and 4 B fragments feed 16 MFMAs per k16 step). A has three LDS
// stages and B two (160 KB), so that a k-tile's A loads go out a whole k-tile
// before they are needed; every wave issues 16 loads per k-tile, spread over
// the k16 steps between its MFMAs (4 per step: B of the next k-tile in step 0,
// A of the one after in steps 1 and 2, B of that one in step 3), which keeps
// the CU's load path at about half its rate instead of in bursts. Per k-tile
// there is one barrier, ahead of its last k16 step: every wave has read the
// stage in full, its own loads of the next k-tile have landed (the A loads of
// the k-tile after may still be in flight), and the next k-tile's first
// fragments are read while the last step's MFMAs run. The stage pattern
// repeats every 6 k-tiles (A stage u % 3, B stage u % 2, all compile-time);
// a K of KT k-tiles enters the first group of 6 at position (6 - KT % 6) % 6.
// Loads past the last k-tile repeat it into a stage nobody reads again.
// Measured on the 7B block's plain products: 3-11 % faster than the 8-wave
// kernel (gate/up 16384 x 37888 x 3584: 1340 against 1220 TFLOP/s).
constexpr int kWaves4 = 4;
template <bool A_KMAJOR, bool B_KMAJOR, int EPI, bool OUT_BF16>
__global__ __launch_bounds__(64 * kWaves4) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm4_kernel(GemmParams p) {
  constexpr int BM = 256, BN = 256, WM = 128, WN = 128, TM = WM / 32, TN = WN / 32;
  constexpr int STAGE = 256 * ROW_BYTES;  // bytes of one operand stage (either layout)
  static_assert(STAGE == MNMajorDirect<256>::ROWB * BK, "both layouts stage 32 KB");
  __shared__ __attribute__((aligned(1024))) uint8_t As0[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t As1[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t As2[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t Bs0[STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t Bs1[STAGE];

  // A k-split launch takes the splits of one tile as consecutive blocks, each
  // over kt_per k-tiles (the last over what remains).
  int bid = blockIdx.x, split = 0;
  if (p.ksplit > 1) {
    split = bid % p.ksplit;
    bid /= p.ksplit;
  } else if ((p.n_tiles & 7) == 0) {
    bid = (bid & 7) * (p.n_tiles >> 3) + (bid >> 3);
  }
  int bm, bn;
  tile_coords(p.tile0 + bid, p.grid_m, p.grid_n, bm, bn);
  const int m0 = bm * BM, n0 = bn * BN;
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;

  std::conditional_t<A_KMAJOR, KMajorDirect<BM>, MNMajorDirect<BM>> ld_a;
  std::conditional_t<B_KMAJOR, KMajorDirect<BN>, MNMajorDirect<BN>> ld_b;
  ld_a.init(p.lda, m0, p.M);
  ld_b.init(p.ldb, n0, p.N);
  const int kt0 = split * p.kt_per;
  const int KT = min(p.K / BK - kt0, p.kt_per);  // this block's k-tiles: kt0 .. kt0 + KT - 1
  auto tk = [&](int u) { return kt0 + min(u, KT - 1); };
  auto ra_at = [&](int kt) { return ld_a.at(p.A, p.lda, m0, A_KMAJOR ? p.M : p.K, kt * BK); };
  auto rb_at = [&](int kt) { return ld_b.at(p.B, p.ldb, n0, B_KMAJOR ? p.N : p.K, kt * BK); };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16{};

  // fragment addresses, as in the 8-wave kernel
  constexpr int NA = A_KMAJOR ? BK / 16 : TM, NB = B_KMAJOR ? BK / 16 : TN;
  uint32_t a_reg[NA], b_reg[NB];
  {
    const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int x = 0; x < NA; ++x) {
      if constexpr (A_KMAJOR)
        a_reg[x] = (wm * WM + l32) * ROW_BYTES + (((2 * x + h) ^ swz_bits(l32)) << 4);
      else
        a_reg[x] = MNMajorDirect<BM>::frag_off(wm * WM + x * 32, lane);
      asm volatile("" : "+v"(a_reg[x]));
    }
#pragma unroll
    for (int x = 0; x < NB; ++x) {
      if constexpr (B_KMAJOR)
        b_reg[x] = (wn * WN + l32) * ROW_BYTES + (((2 * x + h) ^ swz_bits(l32)) << 4);
      else
        b_reg[x] = MNMajorDirect<BN>::frag_off(wn * WN + x * 32, lane);
      asm volatile("" : "+v"(b_reg[x]));
    }
  }
  typedef const __attribute__((address_space(3))) uint8_t* lds_ptr;
  bf16x8 af[2][TM], bfr[2][TN];
  auto rd = [&](lds_ptr la, lds_ptr lb, int kk, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if constexpr (A_KMAJOR) {
        af[slot][i] = *(const lds_bf16x8_t*)(la + a_reg[kk] + i * 32 * ROW_BYTES);
      } else {
        constexpr uint32_t R = MNMajorDirect<BM>::ROWB;
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(la + a_reg[i] + kk * 16 * R));
        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(la + a_reg[i] + kk * 16 * R + 4 * R));
        af[slot][i] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (B_KMAJOR) {
        bfr[slot][j] = *(const lds_bf16x8_t*)(lb + b_reg[kk] + j * 32 * ROW_BYTES);
      } else {
        constexpr uint32_t R = MNMajorDirect<BN>::ROWB;
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(lb + b_reg[j] + kk * 16 * R));
        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(lb + b_reg[j] + kk * 16 * R + 4 * R));
        bfr[slot][j] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    }
  };
  auto mm = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[slot][j], af[slot][i], acc[i][j], 0, 0, 0);
  };
  // The order of a k16 step: its next-step fragment reads (8, 12 or 16 LDS
  // instructions) and the loads spread between its 16 MFMAs.
  constexpr int NR = (A_KMAJOR ? TM : 2 * TM) + (B_KMAJOR ? TN : 2 * TN);
  auto order = [](bool loads) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if constexpr (NR == 12) {
        if (q & 1) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        else __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      } else {
        __builtin_amdgcn_sched_group_barrier(0x100, NR / 8, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (loads && (q & 1)) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
  };

  const int phase = (6 - KT % 6) % 6;
  {
    // k-tile 0 whole, then k-tile 1's A and the first half of its B, into the
    // stages of positions phase and phase + 1
    auto pro = [&](uint8_t* a0, uint8_t* b0, uint8_t* a1, uint8_t* b1) __attribute__((always_inline)) {
      const rsrc_t r_a0 = ra_at(tk(0)), r_b0 = rb_at(tk(0));
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ld_a.issue_one(r_a0, i, a0);
        ld_b.issue_one(r_b0, i, b0);
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      const rsrc_t r_a1 = ra_at(tk(1)), r_b1 = rb_at(tk(1));
#pragma unroll
      for (int i = 0; i < 8; ++i) ld_a.issue_one(r_a1, i, a1);
#pragma unroll
      for (int i = 0; i < 4; ++i) ld_b.issue_one(r_b1, i, b1);
      rd((lds_ptr)a0, (lds_ptr)b0, 0, 0);
    };
    switch (phase) {
      case 0: pro(As0, Bs0, As1, Bs1); break;
      case 1: pro(As1, Bs1, As2, Bs0); break;
      case 2: pro(As2, Bs0, As0, Bs1); break;
      case 3: pro(As0, Bs1, As1, Bs0); break;
      case 4: pro(As1, Bs0, As2, Bs1); break;
      default: pro(As2, Bs1, As0, Bs0); break;
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // k-tile u on A stage SA and B stage SB
  auto tile = [&](int u, auto sac, auto sbc) __attribute__((always_inline)) {
    constexpr int SA = decltype(sac)::value, SB = decltype(sbc)::value;
    uint8_t* la_ = SA == 0 ? As0 : SA == 1 ? As1 : As2;
    uint8_t* na_ = SA == 0 ? As1 : SA == 1 ? As2 : As0;
    uint8_t* fa_ = SA == 0 ? As2 : SA == 1 ? As0 : As1;  // A of k-tile u + 2
    uint8_t* lb_ = SB == 0 ? Bs0 : Bs1;                  // after the barrier: B of k-tile u + 2
    uint8_t* nb_ = SB == 0 ? Bs1 : Bs0;                  // B of k-tile u + 1
    const lds_ptr la = (lds_ptr)la_, lb = (lds_ptr)lb_;
    const rsrc_t r_b1 = rb_at(tk(u + 1)), r_a2 = ra_at(tk(u + 2)), r_b2 = rb_at(tk(u + 2));
    rd(la, lb, 1, 1);
#pragma unroll
    for (int i = 4; i < 8; ++i) ld_b.issue_one(r_b1, i, nb_);
    mm(0);
    order(true);
    __builtin_amdgcn_sched_barrier(0);
    rd(la, lb, 2, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) ld_a.issue_one(r_a2, i, fa_);
    mm(1);
    order(true);
    __builtin_amdgcn_sched_barrier(0);
    rd(la, lb, 3, 1);
#pragma unroll
    for (int i = 4; i < 8; ++i) ld_a.issue_one(r_a2, i, fa_);
    mm(0);
    order(true);
    __builtin_amdgcn_sched_barrier(0);
    // Every read of this stage done, k-tile u + 1 landed (the 8 A loads of
    // k-tile u + 2 may be in flight): a plain barrier, no memory fence.
    asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    rd((lds_ptr)na_, (lds_ptr)nb_, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) ld_b.issue_one(r_b2, i, lb_);
    mm(1);
    order(true);
    __builtin_amdgcn_sched_barrier(0);
  };
  {
    int u = 0;
    if (phase <= 0) tile(u++, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    if (phase <= 1) tile(u++, std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
    if (phase <= 2) tile(u++, std::integral_constant<int, 2>{}, std::integral_constant<int, 0>{});
    if (phase <= 3) tile(u++, std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{});
    if (phase <= 4) tile(u++, std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{});
    tile(u++, std::integral_constant<int, 2>{}, std::integral_constant<int, 1>{});
    for (; u < KT; u += 6) {
      tile(u, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
      tile(u + 1, std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
      tile(u + 2, std::integral_constant<int, 2>{}, std::integral_constant<int, 0>{});
      tile(u + 3, std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{});
      tile(u + 4, std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{});
      tile(u + 5, std::integral_constant<int, 2>{}, std::integral_constant<int, 1>{});
    }
  }
  // the repeated last loads land, every wave is past its reads: LDS is free
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (p.ksplit > 1) {  // raw partial tile; the reduce kernel applies the epilogue
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    float* out = p.ws + (static_cast<int64_t>(bid) * p.ksplit + split) * (BM * BN);
    const int lrow = (lane >> 5) * 4, lcol = lane & 31;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi)
          *reinterpret_cast<f32x4*>(out + (wm * WM + i * 32 + lcol) * BN + wn * WN + j * 32 + gi * 8 + lrow) =
              f32x4{acc[i][j][4 * gi], acc[i][j][4 * gi + 1], acc[i][j][4 * gi + 2], acc[i][j][4 * gi + 3]};
    return;
  }
  uint8_t* region = wave == 0 ? As0 : wave == 1 ? As1 : wave == 2 ? As2 : Bs0;
  store_tile<WM, WN, STAGE, EPI, OUT_BF16>(p, acc, m0, n0, wm, wn, lane, region);
}

// Sums the k-split partial tiles of a launch in split order and applies the
// epilogue the whole-K kernel would have: one thread per 4 columns of a tile
// row (for SwiGLU, per 4 act columns: gate and up sit 32 columns apart).
template <int BM, int BN, int EPI, bool OUT_BF16>
__global__ __launch_bounds__(256) void gemm_reduce(GemmParams p) {
  constexpr int CW = EPI == EPI_SWIGLU ? BN / 2 : BN;  // output columns per tile
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t per_tile = static_cast<int64_t>(BM) * (CW / 4);
  if (idx >= per_tile * p.n_tiles) return;
  const int t = static_cast<int>(idx / per_tile);
  const int rem = static_cast<int>(idx % per_tile);
  const int r = rem / (CW / 4), c4 = (rem % (CW / 4)) * 4;
  int bm, bn;
  tile_coords(p.tile0 + t, p.grid_m, p.grid_n, bm, bn);
  const int row = bm * BM + r;
  if (row >= p.M) return;
  const float* part = p.ws + static_cast<int64_t>(t) * p.ksplit * (BM * BN) + r * BN;
  auto sum4 = [&](int c) {  // columns c .. c + 3 of the tile, splits in order
    float4 a = *reinterpret_cast<const float4*>(part + c);
    for (int sp = 1; sp < p.ksplit; ++sp) {
      const float4 b = *reinterpret_cast<const float4*>(part + static_cast<int64_t>(sp) * (BM * BN) + c);
      a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
    }
    return a;
  };
  if constexpr (EPI == EPI_SWIGLU) {
    const int gc = (c4 / 32) * 64 + c4 % 32;  // tile column of the gate
    const float4 g4 = sum4(gc), u4 = sum4(gc + 32);
    const float gs[4] = {g4.x, g4.y, g4.z, g4.w}, us[4] = {u4.x, u4.y, u4.z, u4.w};
    uint16_t* act = static_cast<uint16_t*>(p.C);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int col = (bn * BN) / 2 + c4 + k;
      const int gcol = bn * BN + gc + k;
      if (col >= p.n_out) continue;
      act[static_cast<int64_t>(row) * p.ldc + col] = f32_to_bf16(silu(gs[k]) * us[k]);
      if (p.gu) {
        p.gu[static_cast<int64_t>(row) * p.ldgu + gcol] = f32_to_bf16(gs[k]);
        p.gu[static_cast<int64_t>(row) * p.ldgu + gcol + 32] = f32_to_bf16(us[k]);
      }
    }
  } else {
    const float4 v4 = sum4(c4);
    const float vs[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int col = bn * BN + c4 + k;
      if (col >= p.N) continue;
      if constexpr (EPI == EPI_SWIGLU_BWD) {
        const int gcol = (col >> 5) * 64 + (col & 31);
        const int64_t o = static_cast<int64_t>(row) * p.ldgu + gcol;
        const float g = bf16_to_f32(p.gu[o]), u = bf16_to_f32(p.gu[o + 32]);
        const float sg = sigmoid(g);
        const float dsilu = sg * (1.0f + g * (1.0f - sg));
        uint16_t* dgu = static_cast<uint16_t*>(p.C);
        const int64_t od = static_cast<int64_t>(row) * p.ldc + gcol;
        dgu[od] = f32_to_bf16(vs[k] * u * dsilu);
        dgu[od + 32] = f32_to_bf16(vs[k] * g * sg);
      } else {
        float x = vs[k] + (p.bias ? p.bias[col] : 0.0f);
        if constexpr (EPI == EPI_RESID) x = p.resid[static_cast<int64_t>(row) * p.ldr + col] + x;
        const int64_t o = static_cast<int64_t>(row) * p.ldc + col;
        if constexpr (OUT_BF16) static_cast<uint16_t*>(p.C)[o] = f32_to_bf16(x);
        else static_cast<float*>(p.C)[o] = x;
      }
    }
  }
}

// The k-split tails' partial tiles live in a workspace the caller passes in
// (mr_gemm_workspace_bytes gives the size the plan below wants; a smaller or
// absent one narrows or drops the split). kSplitCapBytes bounds the plan.
constexpr int64_t kSplitCapBytes = 128ll << 20;
constexpr int kSplitMinKt = 96;

// Blocks per tile for the remainder past the last whole wave of large tiles
// (1 = no split), with its partials within ws_bytes.
int split_plan(int64_t tiles, int KT, int64_t ws_bytes) {
  constexpr int64_t wave = 256, tile_bytes = 256ll * 256 * 4;
  const int64_t tail = tiles % wave;
  int split = 1;
  if (!tail || KT < kSplitMinKt) return 1;
  const int64_t cap = ws_bytes < kSplitCapBytes ? ws_bytes : kSplitCapBytes;
  double best = 1.0;
  for (int sp = 2; sp <= 16 && sp <= KT; ++sp) {
    if (tail * sp * tile_bytes > cap) break;
    const double t = static_cast<double>((tail * sp + wave - 1) / wave) / sp;
    if (t < best - 1e-9) {
      best = t;
      split = sp;
    }
  }
  return split;
}

// Bytes of partials the plan uses for an M x N x K product (0: no split).
int64_t split_bytes(int64_t M, int64_t N, int64_t K) {
  const int KT = static_cast<int>(K / BK);
  if (KT < kSplitMinKt) return 0;  // short K: whole-K tiles of either size
  const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
  const int split = split_plan(tiles, KT, kSplitCapBytes);
  if (split == 1) return 0;
  const int kt_per = (KT + split - 1) / split;
  const int ksplit = (KT + kt_per - 1) / kt_per;
  return (tiles % 256) * ksplit * 256ll * 256 * 4;
}

// Large tiles go out in whole waves of 256 (one per CU). When K is long (at
// least kSplitMinKt steps, so a tile takes far longer than the partial-tile
// round trip), a remainder that would leave CUs idle in a last, partial wave
// (or a whole grid under one wave) is cut along K instead: ksplit blocks per
// tile, chosen (up to 16) to minimise the remainder's time in tile units,
// ceil(tail * ksplit / 256) / ksplit, within the workspace. (Small tiles run
// two per CU and are not split: measured, the split did not pay for them.)
// Whole 256 x 256 tiles tile0 .. tile0 + n - 1 of p, without a k split: the
// 4-wave kernel (K of at least two k-tiles), else the 8-wave one.
// MR_GEMM_8WAVE=1 in the environment keeps every launch on the 8-wave kernel
// (read at every launch; the two kernels give bit-identical results, which
// the tests check).
bool use_4wave(int KT) {
  const char* e = getenv("MR_GEMM_8WAVE");
  return !(e && e[0] == '1') && KT >= 2;
}

template <bool AK, bool BKM, int EPI, bool OB>
void launch_whole(GemmParams q, int tile0, int64_t n, hipStream_t s) {
  q.tile0 = tile0;
  q.n_tiles = static_cast<int>(n);
  q.ksplit = 1;
  q.kt_per = q.K / BK;
  q.sub = 0;
  if (use_4wave(q.K / BK))
    hipLaunchKernelGGL((gemm4_kernel<AK, BKM, EPI, OB>), dim3(static_cast<unsigned>(n)), dim3(64 * kWaves4), 0, s, q);
  else
    hipLaunchKernelGGL((gemm_kernel<256, 256, AK, BKM, EPI, OB>), dim3(static_cast<unsigned>(n)), dim3(kThreads), 0,
                       s, q);
}

template <int BM, int BN, bool AK, bool BKM, int EPI, bool OB>
int launch(GemmParams p, hipStream_t s) {
  p.grid_m = (p.M + BM - 1) / BM;
  p.grid_n = (p.N + BN - 1) / BN;
  const int64_t tiles = static_cast<int64_t>(p.grid_m) * p.grid_n;
  if (tiles > 0x7fffffff) return fail(MR_EINVAL, "mr_gemm: problem too large");
  const int KT = p.K / BK;
  constexpr int64_t wave = 256;
  const int64_t tail = tiles % wave, full = tiles - tail;
  const int split = BM == 256 && p.ws ? split_plan(tiles, KT, p.ws_bytes) : 1;
  if constexpr (BM == 256 && EPI == EPI_STORE) {
    // A last wave at most half full runs as quarter tiles (two per CU)
    // instead of leaving half the CUs or more idle: measured 5-6 % faster on
    // the 7B block's q/k/v projection (4.5 waves) and its attention-output and
    // q/k/v input gradients (3.5 waves). (The residual and SwiGLU-backward
    // epilogues ran no faster or slower on quarter tiles.)
    if (split == 1 && full && tail && tail <= wave / 2) {
      launch_whole<AK, BKM, EPI, OB>(p, 0, full, s);
      GemmParams q = p;
      q.ksplit = 1;
      q.kt_per = KT;
      q.tile0 = static_cast<int>(full);
      q.n_tiles = static_cast<int>(4 * tail);
      q.sub = 1;
      hipLaunchKernelGGL((gemm_kernel<BM / 2, BN / 2, AK, BKM, EPI, OB>),
                         dim3(static_cast<unsigned>(4 * tail)), dim3(kThreads), 0, s, q);
      MR_LAUNCH_CHECK("mr_gemm");
      return MR_OK;
    }
  }
  if (split == 1) {
    if constexpr (BM == 256) {
      launch_whole<AK, BKM, EPI, OB>(p, 0, tiles, s);
    } else {
      p.tile0 = 0;
      p.n_tiles = static_cast<int>(tiles);
      p.ksplit = 1;
      p.kt_per = KT;
      hipLaunchKernelGGL((gemm_kernel<BM, BN, AK, BKM, EPI, OB>), dim3(static_cast<unsigned>(tiles)),
                         dim3(kThreads), 0, s, p);
    }
    MR_LAUNCH_CHECK("mr_gemm");
    return MR_OK;
  }
  if (full) launch_whole<AK, BKM, EPI, OB>(p, 0, full, s);
  p.tile0 = static_cast<int>(full);
  p.n_tiles = static_cast<int>(tail);
  p.kt_per = (KT + split - 1) / split;
  p.ksplit = (KT + p.kt_per - 1) / p.kt_per;  // no empty split
  if (BM == 256 && use_4wave(p.kt_per))
    hipLaunchKernelGGL((gemm4_kernel<AK, BKM, EPI, OB>), dim3(static_cast<unsigned>(tail * p.ksplit)),
                       dim3(64 * kWaves4), 0, s, p);
  else
    hipLaunchKernelGGL((gemm_kernel<BM, BN, AK, BKM, EPI, OB>),
                       dim3(static_cast<unsigned>(tail * p.ksplit)), dim3(kThreads), 0, s, p);
  constexpr int CW = EPI == EPI_SWIGLU ? BN / 2 : BN;
  const int64_t threads = tail * BM * (CW / 4);
  hipLaunchKernelGGL((gemm_reduce<BM, BN, EPI, OB>), dim3(static_cast<unsigned>((threads + 255) / 256)),
                     dim3(256), 0, s, p);
  MR_LAUNCH_CHECK("mr_gemm");
  return MR_OK;
}

// Large tiles unless small ones finish sooner. A long K (at least
// kSplitMinKt steps) always takes 256 x 256 tiles: a remainder wave, or a
// grid under one wave, is cut along K (measured on the weight gradients of the
// small models, M, N <= 3584 and K = 16384, and the short-sequence input
// gradients: 1.1-3.6x faster than small tiles, which leave CUs idle when the
// output is small). Otherwise the two sizes are compared in whole waves: 256
// large tiles per wave, 512 small ones (two per CU), a wave of small tiles
// taking kSmallWave of a large one's time at the same K (0.58 measured with
// K = 3584; 0.45 for K <= 1024, where the prologue and epilogue of the two
// co-resident small tiles overlap each other's k loops). Small tiles win for
// K = 896 (the 0.5B block: its qkv projection 1.6x faster) and when large
// ones leave a last wave mostly idle (the 3B qkv projection: 2.5 waves). The
// residual epilogue (an fp32 read and write per output) stays on large tiles:
// measured, the 0.5B o projection ran 1.2x slower on small ones.
template <bool AK, bool BKM, int EPI, bool OB>
int dispatch(GemmParams p, hipStream_t s) {
  const int KT = p.K / BK;
  if (KT >= kSplitMinKt) return launch<256, 256, AK, BKM, EPI, OB>(p, s);
  const int64_t big = static_cast<int64_t>((p.M + 255) / 256) * ((p.N + 255) / 256);
  const int64_t small = static_cast<int64_t>((p.M + 127) / 128) * ((p.N + 127) / 128);
  const double wave_small = KT <= 16 ? 0.45 : 0.58;
  const double t_big = static_cast<double>((big + 255) / 256);
  const double t_small = static_cast<double>((small + 511) / 512) * wave_small;
  if (EPI != EPI_RESID && t_small < 0.97 * t_big) return launch<128, 128, AK, BKM, EPI, OB>(p, s);
  return launch<256, 256, AK, BKM, EPI, OB>(p, s);
}

// Load offsets are 32-bit: 256 rows of a K-major tile span 256 * ld * 2 bytes;
// the epilogues' lane offsets within a 32-row slice of an output are 32-bit too.
constexpr int kMaxLd = 1 << 22;

bool ok16(const void* p, int64_t ld) {
  return aligned16(p) && (ld % 8) == 0;
}

// The caller's k-split workspace: null or zero bytes disable the split.
bool set_workspace(GemmParams& p, void* ws, size_t bytes) {
  if (!ws || !bytes) {
    p.ws = nullptr;
    p.ws_bytes = 0;
    return true;
  }
  if (!aligned16(ws)) return false;
  p.ws = static_cast<float*>(ws);
  p.ws_bytes = static_cast<int64_t>(bytes);
  return true;
}

}  // namespace
}  // namespace mr

namespace mr {
namespace {

// Bytes from the first element of a rows x width matrix (leading dimension
// ld, esize-byte elements) to one past its last.
int64_t span_bytes(int64_t rows, int64_t ld, int64_t width, int64_t esize) {
  return ((rows - 1) * ld + width) * esize;
}

// A region the launch writes (outputs, k-split partials) against the regions
// it reads: tiles read operand panels while other tiles write, so any shared
// byte changes results. Each pair is (pointer, bytes); null pointers are
// skipped. Returns whether any written region overlaps any other region.
struct Region {
  const void* p;
  int64_t n;
};
template <int NW, int NR>
bool writes_overlap(const Region (&w)[NW], const Region (&r)[NR]) {
  for (int a = 0; a < NW; ++a) {
    if (!w[a].p) continue;
    for (int b = 0; b < NR; ++b)
      if (r[b].p && overlap(w[a].p, w[a].n, r[b].p, r[b].n)) return true;
    for (int b = a + 1; b < NW; ++b)
      if (w[b].p && overlap(w[a].p, w[a].n, w[b].p, w[b].n)) return true;
  }
  return false;
}

}  // namespace
}  // namespace mr

extern "C" {

size_t mr_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return static_cast<size_t>(mr::split_bytes(M, N, K));
}

int mr_gemm(int layout, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
            const void* B, int64_t ldb, void* C, int c_dtype, int64_t ldc, const float* bias,
            const float* resid, int64_t ldr, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace mr;
  clear_error();
  if (M < 0 || N < 0 || K < 0) return fail(MR_EINVAL, "mr_gemm: negative size");
  if (M == 0 || N == 0) return MR_OK;
  if (!A || !B || !C) return fail(MR_EINVAL, "mr_gemm: null operand");
  if (M % 8 || N % 8 || K % BK || K == 0)
    return fail(MR_EINVAL, "mr_gemm: M and N must be multiples of 8 and K a positive multiple of %d "
                "(M=%lld N=%lld K=%lld)", BK, (long long)M, (long long)N, (long long)K);
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return fail(MR_EINVAL, "mr_gemm: too large");
  if (lda > kMaxLd || ldb > kMaxLd || ldc > kMaxLd || (resid && ldr > kMaxLd))
    return fail(MR_EINVAL, "mr_gemm: leading dimensions above %d are not supported", kMaxLd);
  if (!ok16(A, lda) || !ok16(B, ldb))
    return fail(MR_EINVAL, "mr_gemm: operands must be 16-byte aligned with ld a multiple of 8");
  if (c_dtype != MR_F32 && c_dtype != MR_BF16) return fail(MR_EINVAL, "mr_gemm: C must be fp32 or bf16");
  if (!aligned16(C) || ldc % (c_dtype == MR_BF16 ? 8 : 4) || (resid && (!aligned16(resid) || ldr % 4)))
    return fail(MR_EINVAL, "mr_gemm: C and resid must be 16-byte aligned with 16-byte rows");
  if (resid && c_dtype != MR_F32) return fail(MR_EINVAL, "mr_gemm: the residual form writes fp32");
  if (layout < 0 || layout > 2) return fail(MR_EINVAL, "mr_gemm: unknown layout %d", layout);
  {
    const bool a_kmajor = layout != 2, b_kmajor = layout == 0;
    if (lda < (a_kmajor ? K : M) || ldb < (b_kmajor ? K : N) || ldc < N || (resid && ldr < N))
      return fail(MR_EINVAL, "mr_gemm: a leading dimension is smaller than its row");
    // C may be the residual itself (same place, same rows), nothing else it reads
    const int64_t nc = span_bytes(M, ldc, N, c_dtype == MR_BF16 ? 2 : 4);
    const bool in_place = resid == C && ldr == ldc;
    const Region w[2] = {{C, nc}, {workspace, static_cast<int64_t>(workspace_bytes)}};
    const Region r[3] = {{A, a_kmajor ? span_bytes(M, lda, K, 2) : span_bytes(K, lda, M, 2)},
                         {B, b_kmajor ? span_bytes(N, ldb, K, 2) : span_bytes(K, ldb, N, 2)},
                         {in_place ? nullptr : resid, resid ? span_bytes(M, ldr, N, 4) : 0}};
    if (writes_overlap(w, r) || (in_place && workspace && overlap(workspace, workspace_bytes, C, nc)))
      return fail(MR_EINVAL, "mr_gemm: C and the workspace must not overlap A, B, the residual (unless C is "
                  "the residual itself) or each other");
  }
  GemmParams p{};
  p.M = static_cast<int>(M);
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.A = static_cast<const uint16_t*>(A);
  p.lda = lda;
  p.B = static_cast<const uint16_t*>(B);
  p.ldb = ldb;
  p.C = C;
  p.ldc = ldc;
  p.bias = bias;
  p.resid = resid;
  p.ldr = ldr;
  if (!set_workspace(p, workspace, workspace_bytes))
    return fail(MR_EINVAL, "mr_gemm: workspace must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool ob = c_dtype == MR_BF16;
#define MR_GEMM_CASE(AK, BKM)                                                             \
  if (resid) return dispatch<AK, BKM, EPI_RESID, false>(p, s);                            \
  return ob ? dispatch<AK, BKM, EPI_STORE, true>(p, s)                                    \
            : dispatch<AK, BKM, EPI_STORE, false>(p, s);
  switch (layout) {
    case 0: { MR_GEMM_CASE(true, true) }    // NT: Y = X W^T
    case 1: { MR_GEMM_CASE(true, false) }   // NN: dX = dY W
    case 2: { MR_GEMM_CASE(false, false) }  // TN: dW = dY^T X
    default: return fail(MR_EINVAL, "mr_gemm: unknown layout %d", layout);
  }
#undef MR_GEMM_CASE
}

int mr_gemm_swiglu(int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx, const void* Wgu,
                   int64_t ldw, void* act, int64_t ldact, void* gu, int64_t ldgu, void* workspace,
                   size_t workspace_bytes, void* stream) {
  using namespace mr;
  clear_error();
  if (M <= 0 || N <= 0) return MR_OK;
  if (!X || !Wgu || !act) return fail(MR_EINVAL, "mr_gemm_swiglu: null operand");
  if (M % 8 || N % 32 || K % BK || K == 0)
    return fail(MR_EINVAL, "mr_gemm_swiglu: M %% 8, N %% 32 and K %% %d must be 0", BK);
  if (!ok16(X, ldx) || !ok16(Wgu, ldw) || !ok16(act, ldact) || (gu && !ok16(gu, ldgu)))
    return fail(MR_EINVAL, "mr_gemm_swiglu: operands and outputs must be 16-byte aligned with leading "
                "dimensions multiples of 8");
  if (ldx < K || ldw < K || ldact < N || (gu && ldgu < 2 * N) || ldx > kMaxLd || ldw > kMaxLd ||
      ldact > kMaxLd || (gu && ldgu > kMaxLd))
    return fail(MR_EINVAL, "mr_gemm_swiglu: bad leading dimension");
  {
    const Region w[3] = {{act, span_bytes(M, ldact, N, 2)}, {gu, gu ? span_bytes(M, ldgu, 2 * N, 2) : 0},
                         {workspace, static_cast<int64_t>(workspace_bytes)}};
    const Region r[2] = {{X, span_bytes(M, ldx, K, 2)}, {Wgu, span_bytes(2 * N, ldw, K, 2)}};
    if (writes_overlap(w, r))
      return fail(MR_EINVAL, "mr_gemm_swiglu: act, gu and the workspace must not overlap X, Wgu or each other");
  }
  GemmParams p{};
  p.M = static_cast<int>(M);
  p.N = static_cast<int>(2 * N);
  p.n_out = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.A = static_cast<const uint16_t*>(X);
  p.lda = ldx;
  p.B = static_cast<const uint16_t*>(Wgu);
  p.ldb = ldw;
  p.C = act;
  p.ldc = ldact;
  p.gu = static_cast<uint16_t*>(gu);
  p.ldgu = ldgu;
  if (!set_workspace(p, workspace, workspace_bytes))
    return fail(MR_EINVAL, "mr_gemm_swiglu: workspace must be 16-byte aligned");
  return dispatch<true, true, EPI_SWIGLU, true>(p, static_cast<hipStream_t>(stream));
}

int mr_gemm_swiglu_bwd(int64_t M, int64_t N, int64_t K, const void* dd, int64_t ldd,
                       const void* Wd, int64_t ldw, const void* gu, int64_t ldgu, void* dgu,
                       int64_t lddgu, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace mr;
  clear_error();
  if (M <= 0 || N <= 0) return MR_OK;
  if (!dd || !Wd || !gu || !dgu) return fail(MR_EINVAL, "mr_gemm_swiglu_bwd: null operand");
  if (M % 8 || N % 32 || K % BK || K == 0)
    return fail(MR_EINVAL, "mr_gemm_swiglu_bwd: M %% 8, N %% 32 and K %% %d must be 0", BK);
  if (!ok16(dd, ldd) || !ok16(Wd, ldw) || !ok16(gu, ldgu) || !ok16(dgu, lddgu))
    return fail(MR_EINVAL, "mr_gemm_swiglu_bwd: operands and gu/dgu must be 16-byte aligned with leading "
                "dimensions multiples of 8");
  if (ldd < K || ldw < N || lddgu < 2 * N || ldd > kMaxLd || ldw > kMaxLd || lddgu > kMaxLd)
    return fail(MR_EINVAL, "mr_gemm_swiglu_bwd: bad leading dimension");
  if (ldgu != lddgu) return fail(MR_EINVAL, "mr_gemm_swiglu_bwd: gu and dgu must share a layout");
  {
    // dgu may be written over gu itself: each piece of gu is read before the
    // same piece of dgu is written, by the same lane
    const int64_t ng = span_bytes(M, ldgu, 2 * N, 2);
    const Region w[2] = {{dgu, ng}, {workspace, static_cast<int64_t>(workspace_bytes)}};
    const Region r[3] = {{dd, span_bytes(M, ldd, K, 2)}, {Wd, span_bytes(K, ldw, N, 2)},
                         {dgu == gu ? nullptr : gu, ng}};
    if (writes_overlap(w, r) || (dgu == gu && workspace && overlap(workspace, workspace_bytes, gu, ng)))
      return fail(MR_EINVAL, "mr_gemm_swiglu_bwd: dgu and the workspace must not overlap dd, Wd, gu (unless dgu "
                  "is gu itself) or each other");
  }
  GemmParams p{};
  p.M = static_cast<int>(M);
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.A = static_cast<const uint16_t*>(dd);
  p.lda = ldd;
  p.B = static_cast<const uint16_t*>(Wd);
  p.ldb = ldw;
  p.C = dgu;
  p.ldc = lddgu;
  p.gu = const_cast<uint16_t*>(static_cast<const uint16_t*>(gu));
  p.ldgu = ldgu;
  if (!set_workspace(p, workspace, workspace_bytes))
    return fail(MR_EINVAL, "mr_gemm_swiglu_bwd: workspace must be 16-byte aligned");
  return dispatch<true, false, EPI_SWIGLU_BWD, true>(p, static_cast<hipStream_t>(stream));
}

}  // extern "C"
