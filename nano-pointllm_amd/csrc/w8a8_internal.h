// Internal launch interface shared by the kernel translation units and the
// C ABI layer (capi.hip).  Nothing here is exported from the shared library.
#pragma once

#include "w8a8_common.h"

namespace w8a8 {

// Epilogue selector shared by the GEMV and GEMM kernels.
enum Epilogue : int {
  kEpiI32 = 0,      // raw int32 accumulators
  kEpiDequant = 1,  // f32(acc) * s_x * s_w (+ bias) -> output type
  kEpiSilu = 2,     // packed interleaved gate/up: SiLU(g) * u -> output type
  kEpiSiluQ8 = 3,   // as kEpiSilu, then int8 with a static scale
  kEpiRequant = 4,  // int8: (acc + bias_i32) * multiplier >> shift (requant1)
  kEpiBf16Exact = 5,  // bf16: acc * s_x * s_w rounded once (dequant_bf16_exact)
};

struct LinearOperands {
  // Activations.  GEMV: row-major int8 [M, lda], lda % 16 == 0, 16-byte
  // aligned, readable and zero past K up to KB*64.  GEMM: packed tiles.
  const int8_t* a;
  int64_t lda;
  const float* sx;  // per-row activation scales [M]
  const int8_t* w;  // packed weights [NB][KB] tiles
  const float* sw;  // per-output weight scales [N]
  const float* bias;  // [N] or null
  void* y;
  int64_t ldy;
  int y_dtype;      // output element type (kF32/kF16/kBF16/kI32/kI8)
  int h_dtype;      // SiLU intermediate rounding type for kEpiSiluQ8 (kF16/kBF16)
  float out_scale;  // static requant scale for kEpiSiluQ8
  // kEpiRequant: per-output multiplier, right shift and int32 bias (nullable).
  const uint32_t* rq_mult = nullptr;
  const int32_t* rq_shift = nullptr;
  const int32_t* rq_bias = nullptr;
  // kEpiSilu only (nullable): absmax_parts[m * NB + nb] (NB = ceil(N/16))
  // receives the max |h| of row m over the 8 outputs of packed block nb; the
  // first phase of the two-phase per-token requantization of h.  Every
  // (m, nb) with m < M is written by exactly one thread, so no atomics and no
  // initialization are needed.
  float* absmax_parts = nullptr;
  // kEpiDequant with a 16-bit output only (nullable): y = dtype(dtype(dequant)
  // + res[m, n]) (res [M, ld_res] of y's dtype), and with ss_parts the
  // RMSNorm sums of squares of y per 8-column chunk (chunk_sumsq8),
  // ss_parts[m * ld_parts + n / 8].  Taken by gemv_kernel and the fused
  // decode kernels; launch_gemv routes such calls to them.
  const void* res = nullptr;
  int64_t ld_res = 0;
  float* ss_parts = nullptr;
  int64_t ld_parts = 0;
  int64_t M, N, K;
  int epi;
};

// Activation prologue (prologue.hip): per row of 16-bit x, optional
// residual add (written to residual_out), RMSNorm with a weight of x's dtype
// or F32 (w_dtype), division by a per-channel smooth scale of x's dtype, then
// int8 quantization with a per-row dynamic or one static scale.  Row-major
// q [M, ldq] (K columns), or with `packed` the GEMM's 16x64 tiles
// (ceil(M/16)*16 rows x ceil(K/64)*64 columns, zero padded; ldq unused),
// scales_out [M] (nullable), x_out [M, ld_xout] (nullable) receives the rows
// before quantization (x's dtype, or F32 with an F32 RMSNorm weight).  The
// row-major q gets q_cols columns per row (at least K, at most
// min(ldq, round_up(K, 64))), zeros past K.  K <= prologue_max_k().
int64_t prologue_max_k();
hipError_t launch_prologue_quant(const void* x, int x_dtype, int64_t ldx, const void* residual,
                                 int64_t ld_res, void* residual_out, int64_t ld_res_out,
                                 const void* norm_weight, int w_dtype, float eps,
                                 const void* smooth, const float* static_scale, int64_t M,
                                 int64_t K, int8_t* q, int64_t ldq, float* scales_out,
                                 void* x_out, int64_t ld_xout, hipStream_t st,
                                 bool packed = false, int64_t q_cols = 0);

// Elementwise epilogues over caller int32 accumulators acc[m, ld_acc]:
// requant1 per element with per-column multiplier / shift / bias (nullable)
// into int8 y, or dequant_bf16_exact with binary16 scale bit patterns
// sa_bits[m] and sw_bits[n] into bfloat16 y.
hipError_t launch_requant_i32(const int32_t* acc, int64_t ld_acc, const int32_t* bias,
                              const uint32_t* mult, const int32_t* shift, int8_t* y, int64_t ldy,
                              int64_t M, int64_t N, hipStream_t st);
hipError_t launch_dequant_i32_bf16(const int32_t* acc, int64_t ld_acc, const uint16_t* sa_bits,
                                   const uint16_t* sw_bits, uint16_t* y, int64_t ldy, int64_t M,
                                   int64_t N, hipStream_t st);

// y[m, n] = dtype(y[m, n] + res[m, n]) over 16-bit rows (dtype kF16 / kBF16)
// and, with parts (nullable), their RMSNorm sums of squares per 8-column
// chunk (chunk_sumsq8) into parts[m * ld_parts + n / 8].
hipError_t launch_add_rows_ss(void* y, int dtype, int64_t ldy, const void* res, int64_t ld_res,
                              float* parts, int64_t ld_parts, int64_t M, int64_t N,
                              hipStream_t st);

// Quantizes each row of x (scale_in == nullptr: dynamic per-row scale).
// Row-major output writes columns [0, ncols_out) (zeros past K); packed
// output writes whole tiles for ceil(rows/16)*16 rows.
hipError_t launch_quant_rows(const void* x, int x_dtype, int64_t ldx, int64_t rows, int64_t K,
                             const float* scale_in, int64_t scale_stride, int8_t* q,
                             int64_t ldq, int64_t ncols_out, bool packed, float* scales_out,
                             hipStream_t st);

// Second phase of the two-phase per-token requantization: row r of 16-bit x
// is quantized with scale_from_absmax of max(parts[r * nparts + i], i <
// nparts), the maxima the first phase left; scales_out[r] receives the
// scale.  Row-major q [rows, ldq] (K columns).
hipError_t launch_quant_rows_parts(const void* x, int x_dtype, int64_t ldx, int64_t rows,
                                   int64_t K, const float* parts, int64_t nparts, int8_t* q,
                                   int64_t ldq, float* scales_out, hipStream_t st);

hipError_t launch_pack_rows(const int8_t* src, int64_t rows, int64_t K, int64_t ld, int layout,
                            int8_t* dst, hipStream_t st);

// Copies a row-major int8 [rows, K] matrix into [rows, ldd] with zeros in
// columns K..ldd-1 (ldd % 16 == 0).
hipError_t launch_pad_rows(const int8_t* src, int64_t rows, int64_t K, int64_t ld, int8_t* dst,
                           int64_t ldd, hipStream_t st);

// GEMM workgroup tiles (gemm.hip), as chosen by gemm_tile_choice for MB x NB
// 16-row blocks on `cus` compute units with two workgroup slots each.
enum GemmTile : int {
  kGemmTinyDeep = 0,   // 32x32, 1 wave, 3-stage ring of four k-blocks
  kGemmSmallDeep = 1,  // 64x64, 4 waves, 2-stage ring of four k-blocks
  kGemmBigDeep = 2,    // 128x128, 16 waves, 4-stage ring of two k-blocks, 1 per CU
  kGemmBig = 3,        // 128x128, 16 waves, 4-stage ring of one k-block
  kGemmW192 = 4,       // 128x192, 8 waves
  kGemmW224 = 5,       // 128x224, 8 waves
  kGemmW256 = 6,       // 128x256, 8 waves
  kGemmW256Sq = 7,     // 256x256, 16 waves, 2-stage ring of two k-blocks, 1 per CU
  kGemmMid = 8,        // 64x32, 4 waves, 3-stage ring of four k-blocks, 2 per CU
  kGemmWd7x2 = 9,      // 112x256 weights-direct, 8 waves of 112x32, 4 k-blocks ahead, 1 per CU
  kGemmT112x96 = 10,   // 112x96, 14 waves of 16x48, 3-stage ring of three k-blocks, 1 per CU
  kGemmT128x96 = 11,   // 128x96, 8 waves of 32x48, 2-stage ring of four k-blocks, 1 per CU
};
int gemm_tile_choice(int64_t MB, int64_t NB, int64_t cus);

// M <= 64 (the GEMV regime).
hipError_t launch_gemv(const LinearOperands& op, hipStream_t st);
// Any M; activations packed.
hipError_t launch_gemm(const LinearOperands& op, hipStream_t st);

constexpr int64_t kGemvMaxRows = 64;

// Decode linear with the per-token quantization fused in (gemv_fused.hip):
// 16-bit x, 1 <= M <= 8, K % 8 == 0, K <= 12288, 16-byte aligned rows,
// N <= 1024 * CUs, and enough weight bytes per CU to hide the quantization.
// Compute units of the current device.
int cu_count();
// Persistent workgroups for nb output blocks: nb up to the CU count, else the
// fewest that keep every workgroup at ceil(nb / CUs) blocks or one less.
int balanced_grid(int64_t nb);
// epi: the epilogue (kEpiDequant also admits the o_proj shapes of the
// split kernel), or -1; residual: the call adds a residual in its epilogue.
bool fused_gemv_supported(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t N,
                          int64_t K, int epi = -1, bool residual = false);
// The fused kernel's weight stream on int8 activations (op.a row-major as for
// the GEMV, op.sx per-row scales); decode shapes only.
bool fused_gemv_i8_supported(int64_t M, int64_t N, int64_t K, int64_t lda, int epi);
hipError_t launch_gemv_fused_i8(const LinearOperands& op, hipStream_t st);
hipError_t launch_gemv_fused(const void* x, int x_dtype, int64_t ldx, const LinearOperands& op,
                             float* sx_out, hipStream_t st);
// The fused decode linear with LightweightRMSNorm's residual add and RMSNorm
// (norm_w of x's dtype) in front of the quantization; residual_out and x_out
// (nullable) receive the summed and normalized rows.  Decode shapes only.
bool fused_norm_supported(const void* x, int x_dtype, int64_t ldx, const void* residual,
                          int64_t ld_res, const void* residual_out, int64_t ld_res_out,
                          const void* norm_w, const void* x_out, int64_t ld_xout, int64_t M,
                          int64_t N, int64_t K);
// ss_in (nullable, [M, ld_ss_in] binary32): the RMSNorm sums of squares of
// x per 8-column chunk as the residual-add epilogue wrote them (residual
// must then be null); they replace the workgroup's own sums (same bits).
hipError_t launch_gemv_fused_norm(const void* x, int x_dtype, int64_t ldx, const void* residual,
                                  int64_t ld_res, void* residual_out, int64_t ld_res_out,
                                  const void* norm_w, float eps, void* x_out, int64_t ld_xout,
                                  const LinearOperands& op, float* sx_out, hipStream_t st,
                                  const float* ss_in = nullptr, int64_t ld_ss_in = 0);

// Dense 16-bit GEMV (gemv_dense.hip): y[M, ldy] = dtype(x[M, ldx] @ w[N, ldw]^T
// (+ bias)) with binary32 accumulation, dtype kF16 or kBF16; 1 <= M <= 16,
// K % 8 == 0, K <= dense_gemv_max_k(), 16-byte aligned x and w rows,
// M * ldx * 2 < 2^31 and 16 * ldw * 2 < 2^31 (host-checked).
int64_t dense_gemv_max_k();
hipError_t launch_gemv_dense(const void* x, int64_t ldx, const void* w, int64_t ldw,
                             const void* bias, void* y, int64_t ldy, int dtype, int64_t M,
                             int64_t N, int64_t K, hipStream_t st);

}  // namespace w8a8
