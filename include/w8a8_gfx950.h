/*
 * w8a8_gfx950.h - C ABI of libw8a8_gfx950.so, the MI355X (gfx950) W8A8
 * quantized linear path of nanopointllm.
 *
 * The reference has no FFI: its boundary is the Python call sites of
 * F.linear / torch.matmul in nanopointllm/llama/{lightweight_runner,
 * paged_attention}.py and the function API of nanopointllm/compression/
 * {w8a8,quantized_tensor_package}.py.  Each entry point below names the
 * reference interface it replaces.  A Python binding (ctypes) is in
 * nano-pointllm_amd/nanopointllm_amd/_lib.py.
 *
 * Conventions
 *  - Every pointer is device memory owned by the caller, except where noted.
 *    The library never allocates; scratch is the caller's `workspace`
 *    (size from w8a8_workspace_bytes), so every call is graph-capturable.
 *  - Work is enqueued on `stream` and never synchronizes the host.
 *  - Return value: W8A8_OK (0) or a negative w8a8_status.  Nothing throws.
 *  - Integer results are exact; int8 values are in [-127, 127]; scales are
 *    binary32 holding binary16-representable values (CONTRACT,
 *    nanopointllm/compression/w8a8.py:14-30).
 *  - Packed weights use the 16x64 tile layout described at
 *    w8a8_pack_rows; their size is w8a8_packed_bytes(rows, k).
 *  - Outputs (y, scales, workspace) must not overlap the inputs, as for
 *    F.linear, which always writes a new tensor: the product kernels read x
 *    in every workgroup while others already write y.  The one exception,
 *    residual_out and x_out of w8a8_rmsnorm_linear, is stated there.
 */
#ifndef W8A8_GFX950_H
#define W8A8_GFX950_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W8A8_ABI_VERSION 7

typedef enum w8a8_dtype {
  W8A8_F32 = 0,
  W8A8_F16 = 1,
  W8A8_BF16 = 2,
  W8A8_I32 = 3,
  W8A8_I8 = 4
} w8a8_dtype;

typedef enum w8a8_status {
  W8A8_OK = 0,
  W8A8_ERR_NULL = -1,      /* required pointer is null */
  W8A8_ERR_SHAPE = -2,     /* negative size, rows/N above INT32_MAX, leading dimension too small, K overflow */
  W8A8_ERR_DTYPE = -3,     /* unsupported dtype / epilogue combination */
  W8A8_ERR_ALIGN = -4,     /* pointer or leading dimension misaligned */
  W8A8_ERR_WORKSPACE = -5, /* workspace missing or too small */
  W8A8_ERR_HIP = -6,       /* kernel launch failed; see w8a8_last_hip_error */
  W8A8_ERR_TOO_LARGE = -7, /* w8a8_linear_noalloc: more than its static scratch */
  W8A8_ERR_OVERLAP = -8    /* an output overlaps an input other than row for row */
} w8a8_status;

/* Bytes of the static device scratch of w8a8_linear_noalloc (per GPU). */
#define W8A8_NOALLOC_SCRATCH_BYTES (16 << 20)

typedef enum w8a8_epilogue {
  /* y[m, n] = int32 accumulator */
  W8A8_EPI_I32 = 0,
  /* y[m, n] = cast(f32(acc) * s_x[m] * s_w[n] + bias[n]), binary32 steps
   * (integer_linear_per_output_reference, w8a8.py:134-137) */
  W8A8_EPI_DEQUANT = 1,
  /* interleaved packed gate/up (rows g0,u0,g1,u1,...):
   * g,u = inter(dequant); y[m, c] = inter(inter(SiLU(g)) * u)
   * (LightweightMLP packed branch, lightweight_runner.py:344-358) */
  W8A8_EPI_SILU_MUL = 2,
  /* as W8A8_EPI_SILU_MUL, then int8 = quantize_symmetric(h, y_scale)
   * (static A8 requant feeding the down projection, w8a8.py:33-43,94-103) */
  W8A8_EPI_SILU_MUL_Q8 = 3,
  /* int8 y[m, n] = requantize_int32(acc, bias_i32[n], multiplier[n],
   * right_shift[n]): (acc + bias) * multiplier, magnitude rounded to nearest
   * even at the shift, sign restored, clipped to [-127, 127]
   * (architecture_simulator/gtsu_cycle/requant.py:98-119).  Used through
   * w8a8_linear_i8in_requant only. */
  W8A8_EPI_REQUANT = 4,
  /* bfloat16 y[m, n] = acc * s_x[m] * s_w[n] rounded once (ties to even,
   * subnormals kept, overflow to infinity), the scales taken as binary16
   * (architecture_simulator/gtsu_cycle/bf16_dequant.py:47-77).  y_dtype
   * BF16, no bias. */
  W8A8_EPI_DEQUANT_BF16_EXACT = 5
} w8a8_epilogue;

typedef enum w8a8_row_layout {
  W8A8_ROWS_AS_IS = 0,
  /* source rows [gate(0..R/2); up(0..R/2)] packed as g0,u0,g1,u1,...
   * (_pack_gateup_tensors layout "interleave", lightweight_runner.py:81-92) */
  W8A8_ROWS_INTERLEAVE_HALVES = 1
} w8a8_row_layout;

/* Library ABI version (W8A8_ABI_VERSION). */
int w8a8_abi_version(void);

/* Static text for a w8a8_status value. */
const char* w8a8_status_string(int status);

/* hipError_t of the last failed launch on the calling thread (0 if none). */
int w8a8_last_hip_error(void);

/* Bytes of a packed [rows, k] int8 operand: ceil(rows/16)*16 * ceil(k/64)*64. */
int64_t w8a8_packed_bytes(int64_t rows, int64_t k);

/* Workspace bytes needed by w8a8_linear / w8a8_linear_i8in / w8a8_gemm_i32
 * for an [m, k] activation. */
int64_t w8a8_workspace_bytes(int64_t m, int64_t k);

/* GEMM workgroup tile that w8a8_gemm_i32 / w8a8_linear / w8a8_linear_i8in
 * launch for an m x n product in the GEMM regime, on a device with `cus`
 * compute units: 0 = 32x32 (one wave, ring stages of four k-blocks), 1 =
 * 64x64 (stages of four k-blocks), 2 = 128x128 (one workgroup per CU, stages
 * of two k-blocks), 3 = 128x128, 4 = 128x192, 5 = 128x224, 6 = 128x256,
 * 7 = 256x256 (one workgroup per CU, stages of two k-blocks), 8 = 64x32
 * (stages of four k-blocks, past 64 rows), 9 = 112x256 (weights straight
 * to registers four k-blocks ahead, one workgroup per CU), 10 = 112x96
 * (stages of three k-blocks), 11 = 128x96 (stages of four k-blocks); -1
 * for a negative or zero size.  A pure function of its arguments (no device
 * call): it lets tests name the configuration a shape exercises.  No
 * counterpart in the reference, whose products are dense F.linear calls. */
int w8a8_gemm_tile_config(int64_t m, int64_t n, int64_t cus);

/*
 * Per-row symmetric int8 quantization with a dynamic scale per row:
 *   scales[r] = scale_from_absmax(max_k |x[r, k]|)
 *   q[r, k]   = quantize_symmetric(x[r, k], scales[r])
 * Replaces dynamic_per_token_activation_qdq (w8a8.py:106-115, integer part)
 * for activations and per_output_weight_qdq (w8a8.py:53-62) for weights.
 * x: [rows, ldx] of x_dtype (F32/F16/BF16); q: int8 [rows, ldq]; scales: [rows].
 */
int w8a8_quant_rows(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                    int8_t* q, int64_t ldq, float* scales, hipStream_t stream);

/*
 * quantize_symmetric (w8a8.py:33-43) with caller scales: scale[r * scale_stride]
 * (scale_stride 0: one per-tensor scale, the static_activation_qdq case,
 * w8a8.py:101-103).  Scales must be positive; the caller checks that, as the
 * reference's ValueError check does on the host.
 */
int w8a8_quant_rows_scaled(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                           const float* scale, int64_t scale_stride, int8_t* q, int64_t ldq,
                           hipStream_t stream);

/*
 * Packs a row-major int8 [rows, k] matrix (leading dimension ld) into 16x64
 * MFMA tiles: tile (rb, kb) at byte (rb*ceil(k/64) + kb)*1024; inside it lane
 * slot l = r + 16g (16 bytes) holds row 16rb + r, columns 64kb + 16g .. +15;
 * padding is zero.  layout W8A8_ROWS_INTERLEAVE_HALVES reorders rows as the
 * reference's interleaved gate/up packing.  Replaces the packed-weight
 * construction of PagedLlamaAttention.from_hf (paged_attention.py:1242-1262)
 * and _pack_gateup_tensors (lightweight_runner.py:57-93) for int8 weights.
 * packed: w8a8_packed_bytes(rows, k) bytes, 16-byte aligned.
 */
int w8a8_pack_rows(const int8_t* src, int64_t rows, int64_t k, int64_t ld, int layout,
                   int8_t* packed, hipStream_t stream);

/*
 * Raw int32 accumulators acc[m, n] = sum_k xq[m, k] * wq[n, k]: the
 * `flat @ qweight_cpu.transpose(0, 1)` of integer_linear_per_output_reference
 * (w8a8.py:131-133) and QuantizedLinearTensors.integer_golden
 * (quantized_tensor_package.py:39-43).  xq: int8 [m, ldq]; w_packed from
 * w8a8_pack_rows; acc: int32 [m, ldacc].
 */
int w8a8_gemm_i32(const int8_t* xq, int64_t ldq, const int8_t* w_packed, int32_t* acc,
                  int64_t ldacc, int64_t m, int64_t n, int64_t k, void* workspace,
                  int64_t workspace_bytes, hipStream_t stream);

/*
 * Fused W8A8 linear with dynamic per-token activation quantization:
 *   s_x = scale_from_absmax(row absmax of x); xq = quantize_symmetric(x, s_x);
 *   acc = xq @ wq^T (int32); y = epilogue(acc).
 * Replaces F.linear(x, W, b) at the packed QKV / O / gate-up / down call sites
 * (paged_attention.py:97-124,1349-1352,1488; lightweight_runner.py:38-54,
 * 329-379) with the W8A8 contract of integer_linear_per_output_reference
 * (w8a8.py:118-139, per-token activation scale).
 *   x: [m, ldx] of x_dtype; w_packed/w_scale/bias: [n] per output (bias
 *   nullable, binary32); y: [m, ldy] of y_dtype (n/2 columns for the SiLU
 *   epilogues); y_scale: static scale of W8A8_EPI_SILU_MUL_Q8; inter_dtype
 *   (F16/BF16): rounding type of the SiLU intermediates; x_scale_out: nullable
 *   [m], receives s_x.
 * Decode inputs (F16/BF16 x, 1 <= m <= 8 with k <= 12288 or m <= 16 with
 * k <= 6144, k % 8 == 0, 16-byte aligned, and per CU at least 64 KiB of
 * weights and 4 weight bytes per activation element, 2 when m > 8) run as
 * one kernel with
 * the quantization fused in and need no workspace (it may be null); every
 * other case needs w8a8_workspace_bytes(m, k) bytes.
 */
int w8a8_linear(const void* x, int x_dtype, int64_t ldx, const int8_t* w_packed,
                const float* w_scale, const float* bias, int epilogue, void* y, int y_dtype,
                int64_t ldy, float y_scale, int inter_dtype, int64_t m, int64_t n, int64_t k,
                float* x_scale_out, void* workspace, int64_t workspace_bytes,
                hipStream_t stream);

/*
 * w8a8_linear without a workspace argument and without any allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Shapes that w8a8_linear runs fused need
 * no scratch; every other shape stages its quantized activations in a static
 * device array of W8A8_NOALLOC_SCRATCH_BYTES per GPU, and a problem with
 * w8a8_workspace_bytes(m, k) above that returns W8A8_ERR_TOO_LARGE before any
 * launch (16 MiB: every LLaMA-7B projection up to M = 1024, and up to 2048
 * rows at K = 4096; the array is reserved on every GPU the library loads on).  All calls on one GPU share that array, so calls that overlap on
 * one GPU (concurrent streams, or host threads) race: serialize them, e.g. on
 * one stream.  Arguments, results and errors are otherwise w8a8_linear's.
 */
int w8a8_linear_noalloc(const void* x, int x_dtype, int64_t ldx, const int8_t* w_packed,
                        const float* w_scale, const float* bias, int epilogue, void* y,
                        int y_dtype, int64_t ldy, float y_scale, int inter_dtype, int64_t m,
                        int64_t n, int64_t k, float* x_scale_out, hipStream_t stream);

/*
 * LightweightRMSNorm (lightweight_runner.py:239-257) in front of a W8A8
 * linear with per-token dynamic quantization of the normalized rows: the W8A8
 * form of the reference's fused RMSNorm + packed QKV decode projection
 * (_rmsnorm_packed_qkv_kernel, paged_attention.py:163-234, used by
 * _rmsnorm_staged_packed_qkv_decode, :283-305).
 *   x [m, ldx] F16/BF16; residual (nullable, same dtype): x <- x + residual,
 *   written to residual_out (residual_norm); norm_weight [k] of x's dtype:
 *   y = w * dtype(x / sqrt(mean(x^2) + eps)); x_out (nullable) receives y;
 *   then w8a8_linear on y (epilogues I32 / DEQUANT / SILU_MUL / SILU_MUL_Q8 /
 *   DEQUANT_BF16_EXACT), x_scale_out (nullable) its per-row scales.
 * Any m, k <= 32768.  Decode shapes of the fused decode route with m <= 8
 * and k <= 4096 (and enough weight per CU to cover reading x and the
 * residual on every CU) run as one kernel and need no workspace, with the
 * epilogues I32 / DEQUANT / SILU_MUL / SILU_MUL_Q8; the others
 * run the activation prologue (w8a8_prologue_quant), which writes the int8
 * rows straight into the layout the product reads (row-major for the GEMV,
 * the packed tiles for the GEMM: no packing pass), then the product, and
 * need w8a8_workspace_bytes(m, k).  Every route sums the binary32 squares in
 * the same order, so a row gets the same bits whatever batch it is in.
 * residual_out and x_out may each be the very rows of x or of the residual
 * (the same pointer and leading dimension: an in-place update, which takes
 * the prologue route); any other overlap with an input, or between the two,
 * returns W8A8_ERR_OVERLAP before any launch.  y must not overlap any input.
 */
int w8a8_rmsnorm_linear(const void* x, int x_dtype, int64_t ldx, const void* residual,
                        int64_t ld_residual, void* residual_out, int64_t ld_residual_out,
                        const void* norm_weight, float eps, const int8_t* w_packed,
                        const float* w_scale, const float* bias, int epilogue, void* y,
                        int y_dtype, int64_t ldy, float y_scale, int inter_dtype, int64_t m,
                        int64_t n, int64_t k, float* x_scale_out, void* x_out, int64_t ld_x_out,
                        void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * The residual add of a decoder layer folded into the dequant linear, with
 * the RMSNorm sums of squares its next norm needs: the reference's
 * `residual = hidden + attn_out` and `hidden + mlp_out` in the activation
 * dtype (lightweight_runner.py:247-257, 552; residual_norm), after the
 * o_proj / down_proj F.linear of lightweight_runner.py:329-383.
 *   y = dtype(dtype(x W^T dequant (+ bias)) + residual): each product
 *   rounded to y's dtype, then the sum rounded once (as torch does on two
 *   16-bit tensors); y_dtype F16/BF16, residual [m, ld_residual] of y's
 *   dtype; ss_parts (nullable) [m, ld_parts >= ceil(n/8)] binary32 receives,
 *   per row and 8-column chunk c, fl(...fl(y[8c]^2) + ... + y[8c+7]^2) in
 *   column order (columns past n count 0): the partial sums of
 *   w8a8_rmsnorm_linear_ss.
 * x, workspace and errors as w8a8_linear (epilogue DEQUANT).  y, residual
 * and ss_parts must not overlap (W8A8_ERR_OVERLAP).  The decode routes add
 * in their epilogue; the GEMM route runs one elementwise pass after it.
 */
int w8a8_linear_residual(const void* x, int x_dtype, int64_t ldx, const int8_t* w_packed,
                         const float* w_scale, const float* bias, void* y, int y_dtype,
                         int64_t ldy, const void* residual, int64_t ld_residual, float* ss_parts,
                         int64_t ld_parts, int64_t m, int64_t n, int64_t k, void* workspace,
                         int64_t workspace_bytes, hipStream_t stream);

/* w8a8_linear_residual on int8 activations with per-row scales (as
 * w8a8_linear_i8in). */
int w8a8_linear_i8in_residual(const int8_t* xq, int64_t ldq, const float* x_scale,
                              const int8_t* w_packed, const float* w_scale, const float* bias,
                              void* y, int y_dtype, int64_t ldy, const void* residual,
                              int64_t ld_residual, float* ss_parts, int64_t ld_parts, int64_t m,
                              int64_t n, int64_t k, void* workspace, int64_t workspace_bytes,
                              hipStream_t stream);

/*
 * w8a8_rmsnorm_linear without a residual, on rows x that a residual-add
 * linear wrote together with their sums of squares ss_parts (nullable,
 * [m, ld_parts >= ceil(k/8)]): the one-kernel decode route reads those sums
 * instead of summing x in every workgroup, which removes the barrier in front
 * of its weight stream; the other routes sum x themselves.  Every route
 * gives the bits of w8a8_rmsnorm_linear on x (the sums are taken in the norm
 * kernels' order), provided ss_parts are the sums of these very rows.
 */
int w8a8_rmsnorm_linear_ss(const void* x, int x_dtype, int64_t ldx, const float* ss_parts,
                           int64_t ld_parts, const void* norm_weight, float eps,
                           const int8_t* w_packed, const float* w_scale, const float* bias,
                           int epilogue, void* y, int y_dtype, int64_t ldy, float y_scale,
                           int inter_dtype, int64_t m, int64_t n, int64_t k, float* x_scale_out,
                           void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * As w8a8_linear for already-quantized activations xq (int8 [m, ldq]) with
 * per-row scales x_scale[m]: the int8-in down projection fed by
 * W8A8_EPI_SILU_MUL_Q8 or w8a8_quant_rows (w8a8.py:118-139 with a given
 * activation_scale).
 */
int w8a8_linear_i8in(const int8_t* xq, int64_t ldq, const float* x_scale,
                     const int8_t* w_packed, const float* w_scale, const float* bias,
                     int epilogue, void* y, int y_dtype, int64_t ldy, float y_scale,
                     int inter_dtype, int64_t m, int64_t n, int64_t k, void* workspace,
                     int64_t workspace_bytes, hipStream_t stream);

/*
 * As w8a8_linear_i8in for activations already in the packed 16x64 tile
 * layout of an [m, k] int8 operand (w8a8_packed_bytes(m, k) bytes, as
 * w8a8_pack_rows with W8A8_ROWS_AS_IS writes them; pad rows and columns
 * zero): the MFMA GEMM runs directly on them, with no packing pass and no
 * workspace, for any m.  Epilogues as w8a8_linear_i8in.  No counterpart in
 * the reference (its linears take row-major activations): for callers that
 * keep activations packed between kernels, and to time the GEMM kernel
 * alone.
 */
int w8a8_linear_packed(const int8_t* xq_packed, const float* x_scale, const int8_t* w_packed,
                       const float* w_scale, const float* bias, int epilogue, void* y,
                       int y_dtype, int64_t ldy, float y_scale, int inter_dtype, int64_t m,
                       int64_t n, int64_t k, hipStream_t stream);

/*
 * Packed gate/up with SiLU*mul and the two-phase per-token dynamic int8
 * requantization of its output h (the dynamic_per_token_activation_qdq
 * contract, w8a8.py:106-115, applied to the down projection's input of the
 * LightweightMLP packed branch, lightweight_runner.py:344-379), with each
 * row's absmax kept as per-block partial maxima in the workspace (no atomics,
 * nothing to zero), and h and hq not overlapping.
 *   Phase 1: h [m, ldh] (h_dtype F16/BF16, n/2 columns) = SiLU(g) * u as
 *            W8A8_EPI_SILU_MUL of w8a8_linear (x of F32/F16/BF16, quantized
 *            per token) or of w8a8_linear_i8in (x_dtype W8A8_I8 with per-row
 *            x_scale); the epilogue also writes each row's max |h| over each
 *            16-row weight block to the workspace.
 *   Phase 2: h_scale[r] = scale_from_absmax(max over the row's blocks),
 *            hq [m, ldhq] = quantize_symmetric(h, h_scale[r]): exactly
 *            dynamic per-token quantization of h, without a second read of h
 *            for its absmax.
 * Workspace: w8a8_gateup_workspace_bytes(m, n, k) bytes, 256-byte aligned,
 * always required (no state survives the call).
 */
int w8a8_gateup_silu_mul(const void* x, int x_dtype, int64_t ldx, const float* x_scale,
                         const int8_t* w_packed, const float* w_scale, const float* bias, void* h,
                         int h_dtype, int64_t ldh, int8_t* hq, int64_t ldhq, float* h_scale,
                         int64_t m, int64_t n, int64_t k, void* workspace,
                         int64_t workspace_bytes, hipStream_t stream);

/* Workspace bytes of w8a8_gateup_silu_mul for an m x n x k problem. */
int64_t w8a8_gateup_workspace_bytes(int64_t m, int64_t n, int64_t k);

/*
 * Activation prologue fused into the quantization, one pass per row of x
 * (F16/BF16 [m, ldx]), each step optional:
 *   residual add   s = x + residual (x's dtype), written to residual_out
 *                  (LightweightRMSNorm.residual_norm, lightweight_runner.py:247-257);
 *   RMSNorm        y = w * dtype(f32(s) / sqrt(mean(f32(s)^2) + eps)) with
 *                  norm_weight [k] of x's dtype or F32 (norm_weight_dtype); an
 *                  F32 weight keeps y in binary32 (lightweight_runner.py:239-245);
 *   smooth divide  y = dtype(y / smooth[k]), smooth of x's dtype (the
 *                  SmoothQuant input transform, w8a8.py:351-359);
 *   quantization   per-row dynamic scale (w8a8.py:106-115), or the one
 *                  static_scale (w8a8.py:94-103): q int8 [m, ldq] (k columns),
 *                  scales_out [m] (nullable with a static scale).
 * x_out (nullable, [m, ld_x_out], x's dtype or F32 as y) receives y.  The
 * binary32 sum of squares is summed in the kernel's order; every other step
 * is exactly rounded.  k <= 32768.  residual_out and x_out may each be the
 * very rows of x or of the residual (same pointer, leading dimension and
 * element size: each row is read before it is written); any other overlap
 * with an input, or between the two, returns W8A8_ERR_OVERLAP.
 */
int w8a8_prologue_quant(const void* x, int x_dtype, int64_t ldx, const void* residual,
                        int64_t ld_residual, void* residual_out, int64_t ld_residual_out,
                        const void* norm_weight, int norm_weight_dtype, float eps,
                        const void* smooth, const float* static_scale, int64_t m, int64_t k,
                        int8_t* q, int64_t ldq, float* scales_out, void* x_out,
                        int64_t ld_x_out, hipStream_t stream);

/*
 * Static-A8 linear with the hardware model's integer requantization
 * (architecture_simulator/gtsu_cycle/requant.py:62-119): xq int8 [m, ldq]
 * (activations quantized with one static scale), y int8 [m, ldy] =
 * requantize_int32(xq @ wq^T, bias_i32[n], multiplier[n], right_shift[n]).
 * multiplier (uint32) and right_shift (0..63) per output come from
 * compile_fp16_requant_scale(activation scale, weight scale[n], output scale)
 * (requant.py:62-95); bias_i32 is nullable.  Needs
 * w8a8_workspace_bytes(m, k) bytes of workspace.
 */
int w8a8_linear_i8in_requant(const int8_t* xq, int64_t ldq, const int8_t* w_packed,
                             const uint32_t* multiplier, const int32_t* right_shift,
                             const int32_t* bias_i32, int8_t* y, int64_t ldy, int64_t m,
                             int64_t n, int64_t k, void* workspace, int64_t workspace_bytes,
                             hipStream_t stream);

/*
 * requantize_int32 (architecture_simulator/gtsu_cycle/requant.py:98-119) over
 * caller int32 accumulators acc [m, ld_acc], per column n: bias_i32[n]
 * (nullable), multiplier[n], right_shift[n]; y int8 [m, ldy].
 */
int w8a8_requantize_i32(const int32_t* acc, int64_t ld_acc, const int32_t* bias_i32,
                        const uint32_t* multiplier, const int32_t* right_shift, int8_t* y,
                        int64_t ldy, int64_t m, int64_t n, hipStream_t stream);

/*
 * dequantize_int32_to_bf16 (architecture_simulator/gtsu_cycle/bf16_dequant.py:
 * 47-77) over caller int32 accumulators acc [m, ld_acc] with binary16 scale
 * bit patterns sa_bits[m] (activation) and sw_bits[n] (weight); y bfloat16
 * bit patterns [m, ldy].  A non-finite scale gives the quiet NaN 0x7fc0 (the
 * reference raises ValueError).
 */
int w8a8_dequant_i32_bf16(const int32_t* acc, int64_t ld_acc, const uint16_t* sa_bits,
                          const uint16_t* sw_bits, uint16_t* y, int64_t ldy, int64_t m,
                          int64_t n, hipStream_t stream);

/*
 * The LM head at decode batches: a plain 16-bit linear, y = x @ w^T (+ bias),
 * which replaces _decode_linear_rows / _decode_staged_linear on lm_head
 * (nanopointllm/llama/lightweight_runner.py:38-43, 96-99, 676-681; the
 * reference's F.linear on the final-norm rows).  x [m, ldx], w [n, ldw]
 * (nn.Linear's own row-major weight), bias [n] (nullable) and y [m, ldy] are
 * all of `dtype` (W8A8_F16 or W8A8_BF16); products are accumulated in
 * binary32 (per half of each 64-column step: 32 columns per matrix
 * instruction, the steps of one of 16 column ranges in order; then the two
 * halves, then the 16 ranges in order), the bias added, and the sum rounded
 * once to `dtype`.  The order is the same for every row and batch size: the
 * result is deterministic and a row's values do not depend on the other
 * rows.  1 <= m <= 16, k % 8 == 0, k <= 8192, ldx and
 * ldw multiples of 8 with x and w 16-byte aligned, m * ldx and 16 * ldw
 * below 2^30; y must not overlap x, w or bias (W8A8_ERR_OVERLAP).  Larger
 * batches belong to a GEMM (the reference's F.linear).
 */
int w8a8_dense_gemv(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                    void* y, int64_t ldy, int dtype, int64_t m, int64_t n, int64_t k,
                    hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* W8A8_GFX950_H */
