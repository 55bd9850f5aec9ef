/*
 * mround_hip.h -- C ABI of libmround_hip.so, the MI355X (gfx950) kernels of
 * the SignRound v2 tuning path.
 *
 * The reference has no FFI: its hot path is a set of Python operator
 * functions evaluated by MLX. Each entry point below replaces one of them and
 * cites it. The Python package mround_amd binds these through ctypes
 * (mround_amd/kernels/__init__.py) under the reference's own function names.
 *
 * Conventions shared by every entry point:
 *   - All array arguments are device pointers owned by the caller.
 *     Reductions, the GEMMs' k-split partials and the attention backward's
 *     dK/dV partials live in a caller-provided workspace whose size the
 *     matching *_workspace_bytes() query returns. The library allocates no
 *     device memory and keeps no state between calls, so calls on different
 *     streams with their own workspaces do not interfere.
 *   - Every call enqueues work on `stream` (a hipStream_t, NULL = default
 *     stream) and returns without synchronising.
 *   - The return value is MR_OK, MR_EINVAL (bad shape or argument, checked on
 *     the host before anything is launched) or MR_EHIP - hipError_t for a HIP
 *     runtime error. mr_last_error() gives the message for the calling thread.
 *   - Weights are row-major (rows = out_features, cols = in_features).
 *     Quantization groups run along cols. With group_size == -1 a whole row
 *     is one group. Per-weight learnable perturbations (v) and codes use the
 *     reference's grouped layout (rows, n_groups, group_size), which pads the
 *     last group with zeros when cols % group_size != 0; per-group
 *     quantities (alpha, beta, scale, zero point) are (rows, n_groups).
 *   - `mode` is MR_ASYM (unsigned codes, learned zero point), MR_SYM (signed
 *     codes, signed scale) or MR_SYM_SEARCHED (signed codes, scale =
 *     init_scale * beta).
 */
#ifndef MROUND_HIP_H
#define MROUND_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { MR_OK = 0, MR_EINVAL = -22, MR_EHIP = -1000 };
enum { MR_F32 = 0, MR_BF16 = 1, MR_F16 = 2 };
enum { MR_ASYM = 0, MR_SYM = 1, MR_SYM_SEARCHED = 2 };

/* Message of the last failed call on this thread ("" if none). */
const char* mr_last_error(void);
/* ABI version of this library. */
int mr_abi_version(void);

/*
 * Fake-quantize forward: quantize and dequantize in one pass, optionally also
 * returning the integer codes and the per-group scale and zero point.
 * Replaces mround/core/quantizer.py:287-347 (fake_quantize) and 350-398
 * (quantize_codes); oracle mround/reference/quantize.py:249-319.
 *   w          (rows, cols) in w_dtype (MR_F32 / MR_BF16 / MR_F16)
 *   v, alpha, beta  fp32 learnables, or all NULL for round-to-nearest
 *   init_scale fp32 (rows, n_groups), required iff mode == MR_SYM_SEARCHED
 *   wq_out     (rows, cols) in wq_dtype, or NULL
 *   codes_out  (rows, n_groups, group_size) bytes (uint8 asym, int8 sym), or NULL
 *   scale_out, zp_out  fp32 (rows, n_groups), or NULL (zp only for MR_ASYM)
 */
int mr_fq_forward(const void* w, int w_dtype, const float* v, const float* alpha,
                  const float* beta, const float* init_scale, int64_t rows, int64_t cols,
                  int group_size, int bits, int mode, float eps, void* wq_out, int wq_dtype,
                  void* codes_out, float* scale_out, float* zp_out, void* stream);

/*
 * Row placement of wq_out (forward) or of g (backward) inside a larger
 * row-major buffer with the same number of columns: weight row r lives at
 * row (r / block) * stride + offset + r % block. block == 0 is the identity.
 * It lets several layers' W' land in one GEMM operand (q/k/v stacked:
 * block = rows, offset = first row; gate/up interleaved by 32: block = 32,
 * stride = 64, offset 0 or 32) and their gradients be read back from it.
 */
int mr_fq_forward_mapped(const void* w, int w_dtype, const float* v, const float* alpha,
                         const float* beta, const float* init_scale, int64_t rows, int64_t cols,
                         int group_size, int bits, int mode, float eps, void* wq_out, int wq_dtype,
                         int64_t row_block, int64_t row_stride, int64_t row_offset, void* stream);

/*
 * Straight-through backward fused with the sign-SGD step and the projection.
 * Replaces the MLX autodiff of fake_quantize (oracle
 * mround/reference/quantize.py:399-522), SignSGD.apply
 * (mround/core/signsgd.py:125-145) and project_params
 * (mround/core/quantizer.py:430-446), for one layer:
 *   g        dL/dW' (rows, cols) in g_dtype
 *   update   1: v, alpha, beta <- clip(p - lr * sign(dL/dp), bounds), in place
 *            0: parameters untouched
 *   grad_*_out  optional fp32 outputs of dL/dv (grouped), dL/dalpha, dL/dbeta;
 *               when update == 0 at least one must be non-NULL.
 * The gradients are taken at the parameters as they were on entry.
 */
int mr_fq_backward_signsgd(const void* w, int w_dtype, float* v, float* alpha, float* beta,
                           const float* init_scale, const void* g, int g_dtype, int64_t rows,
                           int64_t cols, int group_size, int bits, int mode, float eps,
                           int update, float lr, float coef_lo, float coef_hi, float v_bound,
                           float* grad_v_out, float* grad_alpha_out, float* grad_beta_out,
                           void* stream);

/* The fused step with g read through the row placement of mr_fq_forward_mapped. */
int mr_fq_backward_signsgd_mapped(const void* w, int w_dtype, float* v, float* alpha, float* beta,
                                  const float* init_scale, const void* g, int g_dtype,
                                  int64_t rows, int64_t cols, int group_size, int bits, int mode,
                                  float eps, float lr, float coef_lo, float coef_hi, float v_bound,
                                  int64_t row_block, int64_t row_stride, int64_t row_offset,
                                  void* stream);

/*
 * The fused step, then W' of the updated parameters written to wq_out (in
 * wq_dtype) through the same row placement: the next tuning step's operand,
 * bit-identical to mr_fq_forward_mapped on the parameters just written, made
 * while W and the new v are still in registers. Replaces the step's
 * SignSGD.apply + project_params and the next step's fake_quantize
 * (mround/pipeline/runner.py:920-935, mround/core/quantizer.py:287-347).
 */
int mr_fq_step_requant_mapped(const void* w, int w_dtype, float* v, float* alpha, float* beta,
                              const float* init_scale, const void* g, int g_dtype, int64_t rows,
                              int64_t cols, int group_size, int bits, int mode, float eps, float lr,
                              float coef_lo, float coef_hi, float v_bound, int64_t row_block,
                              int64_t row_stride, int64_t row_offset, void* wq_out, int wq_dtype,
                              void* stream);

/*
 * The same with the rate read on the device: lr = lr_table[*step] (the index
 * clamped to [0, lr_len)), both device pointers, so that a recorded sequence
 * of launches (a HIP graph of one tuning step) replays with each step's rate
 * of the LinearDecay schedule (mround/core/signsgd.py:23-40). mr_counter_add
 * advances the step index inside the same sequence.
 */
int mr_fq_step_requant_mapped_sched(const void* w, int w_dtype, float* v, float* alpha, float* beta,
                                    const float* init_scale, const void* g, int g_dtype,
                                    int64_t rows, int64_t cols, int group_size, int bits, int mode,
                                    float eps, const float* lr_table, int lr_len, const int* step,
                                    float coef_lo, float coef_hi, float v_bound, int64_t row_block,
                                    int64_t row_stride, int64_t row_offset, void* wq_out,
                                    int wq_dtype, void* stream);
/* counter[0] += delta on the stream (device int). No counterpart in the reference. */
int mr_counter_add(int* counter, int delta, void* stream);

/*
 * Pack one-byte codes into MLX uint32 words, element 0 in the least
 * significant bits; widths 3/5/6/7 use the cross-word bitstream.
 * Replaces mround/formats/packing.py:119-163 (pack_codes); oracle
 * mround/reference/packing.py:73-122.
 *   codes        (rows, cols) bytes; read as int8 when codes_signed, else uint8
 *   code_offset  added to every code first (2^(bits-1) for symmetric codes)
 *   range_out    optional device int32[2]: {min, max} of the offset codes;
 *                the caller raises if they leave [0, 2^bits - 1].
 */
int mr_pack_codes(const void* codes, int codes_signed, int code_offset, int64_t rows,
                  int64_t cols, int bits, uint32_t* packed_out, int32_t* range_out,
                  void* stream);

/*
 * Quantize and pack in one pass, for export: the codes of mr_fq_forward (same
 * arguments, same arithmetic) packed into MLX uint32 words as mr_pack_codes
 * packs them (symmetric codes offset by 2^(bits-1)), and the MLX metadata of
 * mr_to_affine, without the one-byte codes in between. Replaces
 * _tensors_for_layer's quantize -> pack_codes -> to_affine chain
 * (mround/formats/mlx_export.py:198-235) and the round-to-nearest export of
 * the remainder (mround/api.py:1877-1937).
 *   w            (rows, cols) bf16 or fp32, 16-byte aligned
 *   packed_out   (rows, cols * bits / 32) uint32
 *   scales_out, biases_out  (rows, cols / group_size) in out_dtype
 * group_size a power of two >= 32 dividing cols; cols a multiple of 32.
 */
int mr_quantize_pack(const void* w, int w_dtype, const float* v, const float* alpha, const float* beta,
                     const float* init_scale, int64_t rows, int64_t cols, int group_size, int bits,
                     int mode, float eps, uint32_t* packed_out, void* scales_out, void* biases_out,
                     int out_dtype, void* stream);

/* Words per row, or MR_EINVAL (mround/formats/packing.py:84-116). */
int64_t mr_packed_width(int64_t cols, int bits);

/* Inverse of mr_pack_codes (mround/formats/packing.py:166-206). */
int mr_unpack_codes(const uint32_t* packed, int64_t rows, int64_t cols, int bits,
                    uint8_t* codes_out, void* stream);

/*
 * MLX affine metadata from scale and zero point:
 * scales = out(scale), biases = out(-scales * out(zp)), zp = 2^(bits-1)
 * when zp == NULL (symmetric). Replaces mround/formats/mlx_export.py:159-195.
 */
int mr_to_affine(const float* scale, const float* zp, int64_t n_groups, int bits,
                 int out_dtype, void* scales_out, void* biases_out, void* stream);

/*
 * Block reconstruction losses with dL/dpred written in the same pass.
 * Replaces mround/core/losses.py:42-130 (reconstruction_loss,
 * outlier_suppressed_loss, outlier_threshold, piece_loss).
 *   loss = sum(r_kept^2) / denom, r = pred - target (fp32), grad = 2 r_kept / denom
 * mr_loss_mse keeps every element. mr_loss_outlier keeps |r| < threshold,
 * where threshold is the k-th largest |r| over the n elements (exact radix
 * select on the float bit pattern; every element tied at the threshold is
 * excluded), unless threshold_in is non-NULL. loss_out and threshold_out are
 * device scalars; grad_out may be NULL. When the threshold is computed,
 * grad_out must not overlap pred or target (refused with MR_EINVAL).
 */
size_t mr_loss_workspace_bytes(int64_t n);
int mr_loss_mse(const float* pred, const float* target, int64_t n, int64_t denom,
                float* loss_out, float* grad_out, void* workspace, void* stream);
int mr_loss_outlier(const float* pred, const float* target, int64_t n, int64_t k, int64_t denom,
                    const float* threshold_in, float* threshold_out, float* loss_out,
                    float* grad_out, void* workspace, void* stream);

/*
 * mr_loss_outlier without a workspace argument and without any allocation:
 * its workspace (4,778,016 bytes: block partials, the radix and sample
 * histograms, the select state and the per-wave candidate lists) is a static
 * device array of the library, one per GPU, held
 * until the process ends; zero_hist clears what must start at zero on every
 * call. No counterpart in the reference: it is for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc). n is at most 2^32 - 1 (MR_EINVAL beyond). Every call on
 * one GPU shares that array, so calls that overlap on one GPU (different
 * streams, or threads) race; issue them in order on one stream.
 */
int mr_loss_outlier_noalloc(const float* pred, const float* target, int64_t n, int64_t k,
                            int64_t denom, const float* threshold_in, float* threshold_out,
                            float* loss_out, float* grad_out, void* stream);

/*
 * DeltaLoss accumulation: scores_out[i] += sum |g * (rtn_i(W) - W)| for each
 * width bits_list[i] (round-to-nearest at that width, fp32 terms, fp64 sum).
 * Replaces the per-batch term of mround/pipeline/scoring.py:238-266;
 * oracle mround/planner/sensitivity.py:190-229. At most 8 widths.
 */
size_t mr_delta_loss_workspace_bytes(int64_t rows, int64_t cols, int n_bits);
int mr_delta_loss(const void* w, int w_dtype, const float* g, int64_t rows, int64_t cols,
                  int group_size, const int* bits_list, int n_bits, int mode, float eps,
                  double* scores_out, void* workspace, void* stream);

/*
 * The same accumulation with the gradient read through a row placement (as in
 * mr_fq_forward_mapped: gradient row r at (r / block) * stride + offset +
 * r % block; block 0 is the identity), and with MR_SYM_SEARCHED allowed:
 * init_scales is then a host array of n_bits device pointers, each width's
 * searched scale grid (rows, n_groups) fp32, and rtn_i quantizes with that
 * scale (mround/pipeline/scoring.py:196-221, the searched grid at scoring
 * time). init_scales may be NULL for the other modes.
 */
int mr_delta_loss_mapped(const void* w, int w_dtype, const float* g, int64_t rows, int64_t cols,
                         int group_size, const int* bits_list, int n_bits, int mode, float eps,
                         const float* const* init_scales, int64_t g_row_block,
                         int64_t g_row_stride, int64_t g_row_offset, double* scores_out,
                         void* workspace, void* stream);

/*
 * Causal-LM cross-entropy over bf16 logits rows (T, V) with leading dimension
 * ld: row_loss[t] = logsumexp(logits[t]) - logits[t, labels[t]] (0 for a
 * negative label, NaN for a label >= V), and, if loss_out is non-NULL,
 * loss_out = scale * sum_t row_loss[t] (fixed-order fp64 sum). If dlogits is
 * non-NULL it receives scale * (softmax(logits[t]) - onehot(labels[t])) as
 * bf16 (zero rows for negative labels); dlogits may be the logits buffer.
 * Replaces _causal_loss and its autodiff (mround/pipeline/scoring.py:183-192,
 * 507-514): scale = 1 / number of labelled positions gives the mean.
 */
int mr_cross_entropy(const void* logits, int64_t ld, int64_t T, int64_t V, const int32_t* labels,
                     float scale, float* row_loss, float* loss_out, void* dlogits, int64_t ldd,
                     void* stream);

/*
 * Embedding lookup into the fp32 residual stream: out[t, :] = table[ids[t], :]
 * (table (V, H) in dtype, leading dimension ldt; out leading dimension ldo).
 * An id outside [0, V) yields a NaN row. Replaces the model's embedding
 * lookup at the head of the scoring forward (mround/pipeline/scoring.py:190)
 * and of the captured block-0 inputs (mround/pipeline/blocks.py:444-520).
 */
int mr_embed_rows(const void* table, int dtype, int64_t V, int64_t H, int64_t ldt,
                  const int32_t* ids, int64_t T, float* out, int64_t ldo, void* stream);

/*
 * bf16 GEMM on the MFMA cores, fp32 accumulation:
 *   C[m, n] = sum_k A(m, k) B(n, k) (+ bias[n]) (+ resid[m, n])
 * layout MR_NT: A = X [M, K], B = W [N, K]  (forward, y = x W^T)
 *        MR_NN: A = dY [M, K], B = W [K, N] (input gradient, dx = dy W)
 *        MR_TN: A = dY [K, M], B = X [K, N] (weight gradient, dW = dy^T x)
 * All row-major with leading dimensions lda/ldb/ldc/ldr in elements; M, N
 * multiples of 8, K a multiple of 64, operands, C and resid 16-byte aligned
 * with rows a multiple of 16 bytes apart. C is fp32 or
 * bf16; with resid (fp32) C is fp32. Long-K problems whose 256 x 256 tiles
 * leave a partial last wave sum that remainder from k-split partial tiles in
 * the caller's workspace: mr_gemm_workspace_bytes(M, N, K) bytes (0 when the
 * shape is not split; N is the product's width, 2N for mr_gemm_swiglu), at
 * most 128 MB, 16-byte aligned. A NULL or smaller workspace narrows or
 * drops the split: the same product, summed in another order. Outputs and
 * the workspace must not overlap the operands or each other (refused with
 * MR_EINVAL); C may be resid itself (same pointer and leading dimension), and
 * mr_gemm_swiglu_bwd's dgu may be its gu. Replaces the
 * matmul of the reference's tunable linear, `x @ weight.T`
 * (mround/pipeline/runner.py:364-368), and the two products MLX autodiff
 * forms for its backward.
 */
enum { MR_NT = 0, MR_NN = 1, MR_TN = 2 };
size_t mr_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K);
int mr_gemm(int layout, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
            const void* B, int64_t ldb, void* C, int c_dtype, int64_t ldc, const float* bias,
            const float* resid, int64_t ldr, void* workspace, size_t workspace_bytes,
            void* stream);

/*
 * fp32 GEMM on the MFMA cores (fp32 products and accumulation), any sizes:
 *   C[m, n] = sum_k A(m, k) (B(n, k) - B2(n, k))   (B2 may be NULL)
 * in the layouts of mr_gemm (B2 shares B's layout and ldb); C fp32 [M, N]
 * row-major. Replaces the float32 products of the reference's single-layer
 * loop, the layer residual x (W' - W)^T and the weight gradient
 * (dL/dr)^T x (mround/core/tuning.py:140-190).
 */
int mr_gemm_f32(int layout, int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B,
                const float* B2, int64_t ldb, float* C, int64_t ldc, void* stream);

/*
 * SwiGLU projection pair in one product: act = silu(x Wg^T) * (x Wu^T), bf16
 * [M, N], from the row-interleaved weight Wgu [2N, K] (rows 64b .. 64b+31 are
 * gate rows 32b .. 32b+31, rows 64b+32 .. 64b+63 the matching up rows; the
 * fake-quant forward writes this layout directly). Optionally also the bf16
 * gate and up values, gu [M, 2N], interleaved the same way by column. X, Wgu,
 * act and gu are 16-byte aligned with leading dimensions multiples of 8.
 * Replaces the mlp's gate/up linears and `nn.silu(g) * u` of the mlx-lm
 * block reached at mround/pipeline/blocks.py:605.
 */
int mr_gemm_swiglu(int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx, const void* Wgu,
                   int64_t ldw, void* act, int64_t ldact, void* gu, int64_t ldgu, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * Input gradient of the down projection fused with the SwiGLU backward:
 * dact = dd Wd (dd [M, K] bf16, Wd [K, N] bf16 = down weight [hidden, inter]),
 * then from the saved gu (mr_gemm_swiglu's interleaved gate/up):
 *   dgate = dact * u * silu'(g), dup = dact * silu(g), written interleaved to
 *   dgu [M, 2N] bf16 (same layout as gu). The MLX autodiff of the mlp's
 *   silu(g) * u and down linear (mround/pipeline/runner.py:920).
 * Every operand, gu and dgu 16-byte aligned with leading dimensions
 * multiples of 8; M % 8, N % 32 and K % 64 zero.
 */
int mr_gemm_swiglu_bwd(int64_t M, int64_t N, int64_t K, const void* dd, int64_t ldd,
                       const void* Wd, int64_t ldw, const void* gu, int64_t ldgu, void* dgu,
                       int64_t lddgu, void* workspace, size_t workspace_bytes, void* stream);

/*
 * RMSNorm over rows of the fp32 residual stream, y = h rsqrt(mean(h^2) + eps) w
 * as bf16 (the next GEMM's operand) plus the per-row rsqrt for the backward;
 * the backward adds the residual gradient: dh = dres + d(rmsnorm)/dh^T dy.
 * mlx-lm's RMSNorm in the block (mround/pipeline/blocks.py:605).
 */
int mr_rmsnorm_fwd(const float* h, const float* w, int64_t T, int64_t H, float eps, void* y_bf16,
                   float* rstd_out, void* stream);
int mr_rmsnorm_bwd(const float* dy, const float* h, const float* w, const float* rstd,
                   const float* dres, int64_t T, int64_t H, void* dh_bf16, float* dh_f32,
                   void* stream);

/*
 * Split-precision operands: the reference's remedy for the block objective's
 * subtraction of two block outputs (mround DOCUMENTATION.md:885-925, three
 * products A_hi B_hi + A_hi B_lo + A_lo B_hi), which its code documents but
 * does not ship; these have no counterpart in the reference's code. An fp32
 * value y is carried as hi = bf16(y) and lo = bf16(y - hi). A product runs as
 * one bf16 GEMM over K' = 3K with A' = [A_hi | A_hi | A_lo] (order 0, for
 * activations) and B' = [B_hi | B_lo | B_hi] (order 1, for weights) along K.
 *
 * mr_rmsnorm_fwd_split: mr_rmsnorm_fwd with y also written split, order 0,
 *   into rows of 3H bf16 (y_split); y_bf16 (hi alone) and rstd_out optional.
 *   H a multiple of 4 up to 16384, h and w 16-byte aligned, outputs 8-byte.
 * mr_split_bf16: fp32 rows [rows, cols] (ld_src) into split rows (ld_dst >=
 *   3 cols) in the given order, hi alone into plain (ld_plain) when given;
 *   cols and the leading dimensions multiples of 4.
 * mr_swiglu_split: act = silu(g) u from fp32 gate/up rows [T, 2N] interleaved
 *   every 32 columns (the gate/up GEMM's layout), written split (order 0,
 *   rows of 3N), hi alone into act [T, N], and the gate/up values in bf16
 *   into gu [T, 2N] for the backward; N a multiple of 32.
 */
int mr_rmsnorm_fwd_split(const float* h, const float* w, int64_t T, int64_t H, float eps, void* y_split,
                         void* y_bf16, float* rstd_out, void* stream);
int mr_split_bf16(const float* src, int64_t ld_src, int64_t rows, int64_t cols, int order, void* dst,
                  int64_t ld_dst, void* plain, int64_t ld_plain, void* stream);
int mr_swiglu_split(const float* gu32, int64_t T, int64_t N, void* act_split, void* act, void* gu,
                    void* stream);

/*
 * Rotary embedding (non-interleaved halves) in place on the first n_heads
 * heads of rows of x (bf16, leading dimension ld), position = row % S, with
 * cos/sin from cos_sin [S, head_dim/2, 2] fp32; backward = 1 applies the
 * transpose rotation to gradients. mlx-lm's rope (traditional=False).
 */
int mr_rope(void* x_bf16, int64_t ld, int64_t T, int S, int n_heads, int head_dim,
            const float* cos_sin, int backward, void* stream);

/*
 * Split precision for the attention (the reference's three-product remedy,
 * DOCUMENTATION.md:885-925, carried through the scaled-dot-product attention
 * of mround/pipeline/blocks.py:605): fp32 q/k/v rows x [T, ldx] (the split
 * q/k/v product's output), the first n_rope_heads of the n_heads heads
 * rotated in fp32 as mr_rope does and the rest passed through, written as
 * bf16 hi = bf16(y) and lo = bf16(y - hi) rows (leading dimension ld).
 */
int mr_rope_split(const float* x, int64_t ldx, int64_t T, int S, int n_rope_heads, int n_heads, int head_dim,
                  const float* cos_sin, void* hi, void* lo, int64_t ld, void* stream);

/*
 * Causal grouped-query attention on the packed bf16 qkv rows [B*S, ld]
 * (q heads, then k heads, then v heads; query head h uses kv head
 * h / (Hq / Hkv)), head_dim 64 or 128, S a multiple of 128. The forward
 * writes out [B*S, Hq*head_dim] bf16 (leading dimension ldo) and the natural
 * log-sum-exp per (b, h, s) for the backward. The backward takes dout, writes
 * the gradient of the (post-rope) q/k/v into dqkv (same layout as qkv) and
 * uses dsum_ws (B*Hq*S floats) as workspace. The backward may split each kv
 * head's G = Hq / Hkv query heads over hsplit blocks, summing their fp32
 * dK/dV partials in a fixed order from `workspace`
 * (mr_attn_bwd_workspace_bytes(..., hsplit) bytes, 16-byte aligned).
 * hsplit = 0 picks the split automatically (more blocks when fewer than 512
 * blocks of 128 keys would run, Hkv * B * S / 128, within the workspace
 * given; query the size with hsplit = 0); 1..G forces it and refuses a
 * workspace too small for it. Outputs that share memory with the inputs
 * (out with qkv; dqkv or dsum_ws with qkv, out, dout or each other) are
 * refused with MR_EINVAL. The scaled-dot-product attention of the
 * mlx-lm block (mround/pipeline/blocks.py:605) and its autodiff.
 */
int mr_attn_fwd(const void* qkv, int64_t ld, int B, int S, int Hq, int Hkv, int head_dim,
                float scale, void* out, int64_t ldo, float* lse, void* stream);
/*
 * mr_attn_fwd in split precision: q, k and v as the hi and lo halves of
 * mr_rope_split (same layout, leading dimension ld), the scores and the
 * probability-value product each as three bf16 products (hi hi, lo hi,
 * hi lo). Writes the output's hi half into out (what the backward reads) and
 * the output split into out_split rows of 3 Hq head_dim values,
 * [hi | hi | lo] (the activation operand of a split product over
 * K' = 3 Hq head_dim), and the log-sum-exp.
 */
int mr_attn_fwd_split(const void* qkv_hi, const void* qkv_lo, int64_t ld, int B, int S, int Hq, int Hkv,
                      int head_dim, float scale, void* out, int64_t ldo, void* out_split, int64_t ld_split,
                      float* lse, void* stream);
size_t mr_attn_bwd_workspace_bytes(int B, int S, int Hq, int Hkv, int head_dim, int hsplit);
int mr_attn_bwd(const void* qkv, int64_t ld, const void* out, const void* dout, int64_t ldo,
                const float* lse, float* dsum_ws, int B, int S, int Hq, int Hkv, int head_dim,
                float scale, void* dqkv, int hsplit, void* workspace, size_t workspace_bytes,
                void* stream);

/*
 * v2 candidate-scale grid search for symmetric schemes: per group, the
 * signed largest-magnitude element anchors the effective range nmax
 * (= 2^(bits-1)); candidates nmax - step * i for i in [-half_count,
 * half_count] \ {0} follow it in order; the kept scale is the first with the
 * least sum((scale * clip(rne(inverse * w)) - w)^2 * importance[col]) in fp32,
 * summed in column order (inverse = -eff / anchor, scale = 1 / inverse, 0 for
 * an all-zero group). Replaces mround/core/scale_search.py:71-187 (oracle
 * mround/reference/scale_search.py:130-211). importance: fp32 [cols] or NULL.
 * scale_out: fp32 (rows, cols / group_size). group_size 32, 64 or 128.
 */
int mr_search_scales(const void* w, int w_dtype, const float* importance, int64_t rows,
                     int64_t cols, int group_size, int bits, double step, int half_count,
                     float* scale_out, void* stream);

/*
 * out[c] += sum_r x[r, c]^2 over a (rows, cols) fp32/bf16 matrix with leading
 * dimension ld, in a fixed order (row blocks, then blocks in order): the
 * per-input-channel importance a linear collects in the reference's stats
 * forward (mround/pipeline/runner.py:346-363). workspace:
 * mr_colsumsq_workspace_bytes(cols) bytes.
 */
int64_t mr_colsumsq_workspace_bytes(int64_t cols);
int mr_colsumsq(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ld, float* out,
                void* workspace, void* stream);

/*
 * Exact mixed-precision bit allocation (host code, no device work): one
 * option per layer minimizing the summed delta_loss with the summed
 * cost_bits <= budget_bits. Replaces mround/planner/allocator.py:98-194
 * (allocate_bits, with its Pareto pruning and tie order). Layer i's options
 * are entries [sum(n_options[:i]), + n_options[i]) of cost_bits/delta_loss.
 * max_states > 0 thins each frontier to that many evenly ranked states
 * (approximate, as the reference's max_states); 0 keeps the search exact.
 * Writes the chosen option index per layer, the predicted loss and the cost.
 */
int mr_allocate_bits(int n_layers, const int32_t* n_options, const int64_t* cost_bits,
                     const double* delta_loss, int64_t budget_bits, int64_t max_states,
                     int32_t* choice_out, double* loss_out, int64_t* cost_out);

/*
 * fp32 -> bf16 (round to nearest even), n elements: the block output's
 * gradient as a GEMM operand for the backward. No counterpart in the
 * reference, whose block runs in fp32 throughout (mround/pipeline/runner.py:337).
 */
int mr_cast_f32_bf16(const float* x, void* y, int64_t n, void* stream);

/* Plain device copy of `bytes` bytes, used to calibrate traffic counters.
 * No counterpart in the reference (measurement support only). */
int mr_copy_bytes(const void* src, void* dst, size_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MROUND_HIP_H */
