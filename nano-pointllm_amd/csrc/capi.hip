// extern "C" entry points of libw8a8_gfx950.so (declared in
// include/w8a8_gfx950.h).  Validation and dispatch only: shapes, dtypes,
// alignment and workspace are checked here and reported as status codes; the
// kernels live in quant.hip, gemv.hip and gemm.hip.
#include <mutex>
#include <utility>

#include "w8a8_gfx950.h"
#include "w8a8_internal.h"

using namespace w8a8;

// Scratch of w8a8_linear_noalloc: the per-call workspace of w8a8_linear
// (activation scales + staged int8 activations) in a static device array, so
// that entry point never allocates.  Every GPU the library runs on holds its
// own copy for the life of the process.  In host code `scratch` names a
// host-side stand-in, not the device address: only the address that
// hipGetSymbolAddress returns for the current device may reach a kernel.
static __device__ __align__(256) int8_t scratch[W8A8_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local int g_last_hip_error = 0;

// Device address of `scratch`, looked up once per device with that device
// current (each device has the array at its own address).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Largest K whose worst-case dot product K * 127^2 fits a signed int32
// (the overflow guard of compare_linear_bf16_qdq_integer, w8a8.py:152-153).
constexpr int64_t kMaxK = ((int64_t{1} << 31) - 1) / (127 * 127);

// Row and column counts are carried as int in the kernels' parameters and
// launch one workgroup per row in the quantizers; the margin keeps a count
// rounded up to whole 256-row tiles inside int as well.
constexpr int64_t kMaxRows = INT32_MAX - 256;

inline int status_of(hipError_t e) {
  if (e == hipSuccess) return W8A8_OK;
  g_last_hip_error = static_cast<int>(e);
  return W8A8_ERR_HIP;
}

inline bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

inline int64_t round_up(int64_t v, int64_t m) { return ceil_div(v, m) * m; }

// Whether the byte ranges of two [rows, ld] matrices of `elem`-byte values
// (k used columns) overlap; a null pointer overlaps nothing.
// Whether the [rows, k] row sets at a (leading dimension lda, elements of ea
// bytes) and b (ldb, eb) share a byte of their address ranges.
inline bool overlap(const void* a, int64_t lda, int64_t ea, const void* b, int64_t ldb, int64_t eb,
                    int64_t rows, int64_t k) {
  if (a == nullptr || b == nullptr || rows <= 0 || k <= 0) return false;
  // 128-bit ends: a huge leading dimension cannot wrap the comparison.
  using u128 = unsigned __int128;
  const u128 a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
  const u128 a1 = a0 + (static_cast<u128>(rows - 1) * static_cast<u128>(lda) + k) * ea;
  const u128 b1 = b0 + (static_cast<u128>(rows - 1) * static_cast<u128>(ldb) + k) * eb;
  return a0 < b1 && b0 < a1;
}

// Whether a row-wise kernel, which reads each row of its inputs before it
// writes that row of an output, may write output rows `out` over input rows
// `in`: they are disjoint, or they are the very same rows (in place).
inline bool rows_alias_ok(const void* out, int64_t ld_out, int64_t e_out, const void* in,
                          int64_t ld_in, int64_t e_in, int64_t rows, int64_t k) {
  if (!overlap(out, ld_out, e_out, in, ld_in, e_in, rows, k)) return true;
  return out == in && e_out == e_in && (rows == 1 || ld_out == ld_in);
}

inline bool float_dtype(int d) { return d == kF32 || d == kF16 || d == kBF16; }
inline bool half_dtype(int d) { return d == kF16 || d == kBF16; }

inline int64_t elem_size(int d) {
  switch (d) {
    case kF32:
    case kI32:
      return 4;
    case kF16:
    case kBF16:
      return 2;
    case kI8:
      return 1;
    default:
      return 0;
  }
}

// Workspace layout: [activation scales: round_up(4m, 256)] [int8 activations:
// ceil(m/16)*16 rows x ceil(k/64)*64 columns, row-major (GEMV) or packed (GEMM)].
inline int64_t scale_region(int64_t m) { return round_up(4 * m, 256); }
inline int64_t act_region(int64_t m, int64_t k) {
  return round_up(m, kTileRows) * round_up(k, kTileK);
}
// Per-row, per-16-row-block partial maxima of the two-phase requantization.
inline int64_t parts_region(int64_t m, int64_t n) {
  return round_up(4 * m * ceil_div(n, kTileRows), 256);
}

// Checks an epilogue / output dtype pair and returns the number of output
// columns, or -1 when the combination is unsupported.
inline int64_t output_cols(int epi, int y_dtype, int inter_dtype, int64_t n) {
  switch (epi) {
    case W8A8_EPI_I32:
      return y_dtype == kI32 ? n : -1;
    case W8A8_EPI_DEQUANT:
      return float_dtype(y_dtype) ? n : -1;
    case W8A8_EPI_SILU_MUL:
      return (half_dtype(y_dtype) && n % 2 == 0) ? n / 2 : -1;
    case W8A8_EPI_SILU_MUL_Q8:
      return (y_dtype == kI8 && half_dtype(inter_dtype) && n % 2 == 0) ? n / 2 : -1;
    case W8A8_EPI_REQUANT:
      return y_dtype == kI8 ? n : -1;
    case W8A8_EPI_DEQUANT_BF16_EXACT:
      return y_dtype == kBF16 ? n : -1;
    default:
      return -1;
  }
}

// Common checks of the weight side and output of a linear.
inline int check_linear(const int8_t* w_packed, const float* w_scale, int epi, void* y,
                        int y_dtype, int64_t ldy, float y_scale, int inter_dtype, int64_t m,
                        int64_t n, int64_t k) {
  if (m < 0 || n < 0 || k < 0) return W8A8_ERR_SHAPE;
  if (k > kMaxK || m > kMaxRows || n > kMaxRows) return W8A8_ERR_SHAPE;
  const int64_t cols = output_cols(epi, y_dtype, inter_dtype, n);
  if (cols < 0) return W8A8_ERR_DTYPE;
  if (m == 0 || n == 0) return W8A8_OK;
  // With k == 0 the packed weights are empty (and may be null): the product
  // kernels read no k-blocks and write bias-only / zero outputs.
  if ((k > 0 && w_packed == nullptr) || y == nullptr) return W8A8_ERR_NULL;
  if (epi != W8A8_EPI_I32 && epi != W8A8_EPI_REQUANT && w_scale == nullptr)
    return W8A8_ERR_NULL;
  if (ldy < cols) return W8A8_ERR_SHAPE;
  if (!aligned(w_packed, 16) || !aligned(y, static_cast<uintptr_t>(elem_size(y_dtype))))
    return W8A8_ERR_ALIGN;
  if (epi == W8A8_EPI_SILU_MUL_Q8 && !(y_scale > 0.0f)) return W8A8_ERR_SHAPE;
  return W8A8_OK;
}

LinearOperands make_ops(const int8_t* a, int64_t lda, const float* sx, const int8_t* w,
                        const float* sw, const float* bias, int epi, void* y, int y_dtype,
                        int64_t ldy, float y_scale, int inter_dtype, int64_t m, int64_t n,
                        int64_t k) {
  LinearOperands op;
  op.a = a;
  op.lda = lda;
  op.sx = sx;
  op.w = w;
  op.sw = sw;
  op.bias = bias;
  op.y = y;
  op.ldy = ldy;
  op.y_dtype = y_dtype;
  op.h_dtype = inter_dtype;
  op.out_scale = y_scale;
  op.M = m;
  op.N = n;
  op.K = k;
  op.epi = epi;
  return op;
}

// GEMV or GEMM for an m x n x k product.  The GEMV's time grows with M
// (each weight fragment meets M activation rows) while the GEMM's barely
// does at M <= 64; measured on MI355X with LLaMA-7B shapes at M = 17..64
// (quantize + product, graphs of 32 layers), the GEMV takes every projection
// up to M = 32 (QKV at M = 32 in 15.8 against 19.8 us) and those with
// N <= 12288 up to M = 64 (QKV at M = 48 / 64 16.6 / 17.5 against 20.9 /
// 21.1), and with K <= 4096 (the 17-64-row kernel, x read in whole lines)
// gate/up up to M = 64 too (24.6 / 25.8 against 26.5 / 27.2 us on the GEMM).
inline bool use_gemv(int64_t m, int64_t n, int64_t k) {
  return m <= kGemvMaxRows && (m <= 32 || n <= 12288 || k <= 4096);
}

// Runs the int8 product for activations already staged in `act` (row-major
// [m, round_up(k,64)] for the GEMV, packed tiles for the GEMM).  The GEMV
// kernels take the residual-add epilogue (op.res) themselves; the GEMM
// writes its output first and the add runs over it.
inline hipError_t run_product(const LinearOperands& op, hipStream_t st) {
  if (use_gemv(op.M, op.N, op.K)) return launch_gemv(op, st);
  if (op.res == nullptr) return launch_gemm(op, st);
  LinearOperands plain = op;
  plain.res = nullptr;
  plain.ss_parts = nullptr;
  const hipError_t e = launch_gemm(plain, st);
  if (e != hipSuccess) return e;
  return launch_add_rows_ss(op.y, op.y_dtype, op.ldy, op.res, op.ld_res, op.ss_parts,
                            op.ld_parts, op.M, op.N, st);
}

// The residual add of a decoder layer folded into a linear's epilogue
// (w8a8_linear_residual and friends): y = dtype(dtype(x W^T) + res), and
// with parts (nullable) the RMSNorm sums of squares of y per 8 columns.
struct ResidualAdd {
  const void* res;
  int64_t ld_res;
  float* parts;
  int64_t ld_parts;
};

// Whether the byte ranges of [rows, ka] at a (lda, ea-byte elements) and
// [rows, kb] at b (ldb, eb) share a byte; null pointers overlap nothing.
inline bool overlap2(const void* a, int64_t lda, int64_t ea, int64_t ka, const void* b,
                     int64_t ldb, int64_t eb, int64_t kb, int64_t rows) {
  if (a == nullptr || b == nullptr || rows <= 0 || ka <= 0 || kb <= 0) return false;
  using u128 = unsigned __int128;
  const u128 a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
  const u128 a1 = a0 + (static_cast<u128>(rows - 1) * static_cast<u128>(lda) + ka) * ea;
  const u128 b1 = b0 + (static_cast<u128>(rows - 1) * static_cast<u128>(ldb) + kb) * eb;
  return a0 < b1 && b0 < a1;
}

// Checks of the residual-add operands for an [m, n] 16-bit output y.
inline int check_residual(const ResidualAdd& ra, const void* y, int y_dtype, int64_t ldy,
                          int64_t m, int64_t n) {
  if (!half_dtype(y_dtype)) return W8A8_ERR_DTYPE;
  if (m == 0 || n == 0) return W8A8_OK;
  if (ra.res == nullptr) return W8A8_ERR_NULL;
  const int64_t chunks = ceil_div(n, 8);
  if (ra.ld_res < n || (ra.parts != nullptr && ra.ld_parts < chunks)) return W8A8_ERR_SHAPE;
  if (!aligned(ra.res, 2) || !aligned(ra.parts, 4)) return W8A8_ERR_ALIGN;
  if (overlap2(y, ldy, 2, n, ra.res, ra.ld_res, 2, n, m) ||
      overlap2(ra.parts, ra.ld_parts, 4, chunks, y, ldy, 2, n, m) ||
      overlap2(ra.parts, ra.ld_parts, 4, chunks, ra.res, ra.ld_res, 2, n, m))
    return W8A8_ERR_OVERLAP;
  return W8A8_OK;
}

inline void set_residual(LinearOperands& op, const ResidualAdd* ra) {
  if (ra == nullptr) return;
  op.res = ra->res;
  op.ld_res = ra->ld_res;
  op.ss_parts = ra->parts;
  op.ld_parts = ra->ld_parts;
}

// Stages caller int8 activations for run_product: the GEMV reads them in
// place when rows are 16-byte aligned and zero-padded reads are not needed;
// otherwise they are copied (GEMV) or packed (GEMM) into the workspace.
inline hipError_t stage_i8(const int8_t* xq, int64_t ldq, int64_t m, int64_t n, int64_t k,
                           int8_t* act, const int8_t** a, int64_t* lda, hipStream_t st) {
  const int64_t kp = round_up(k, kTileK);
  if (use_gemv(m, n, k)) {
    if (k % kTileK == 0 && ldq % 16 == 0 && aligned(xq, 16)) {
      *a = xq;
      *lda = ldq;
      return hipSuccess;
    }
    *a = act;
    *lda = kp;
    return launch_pad_rows(xq, m, k, ldq, act, kp, st);
  }
  *a = act;
  *lda = kp;
  return launch_pack_rows(xq, m, k, ldq, W8A8_ROWS_AS_IS, act, st);
}

// w8a8_linear; absmax_parts (nullable, W8A8_EPI_SILU_MUL only, [m][ceil(n/16)]
// binary32) receives the first phase of the two-phase per-token
// requantization of the output.
int linear_impl(const void* x, int x_dtype, int64_t ldx, const int8_t* w_packed,
                const float* w_scale, const float* bias, int epilogue, void* y, int y_dtype,
                int64_t ldy, float y_scale, int inter_dtype, int64_t m, int64_t n, int64_t k,
                float* x_scale_out, void* workspace, int64_t workspace_bytes,
                float* absmax_parts, hipStream_t stream, const ResidualAdd* ra = nullptr) {
  if (!float_dtype(x_dtype)) return W8A8_ERR_DTYPE;
  // The integer requant needs int8 activations with a static scale
  // (w8a8_linear_i8in_requant); the single-rounding bf16 dequant has no bias.
  if (epilogue == W8A8_EPI_REQUANT) return W8A8_ERR_DTYPE;
  if (epilogue == W8A8_EPI_DEQUANT_BF16_EXACT && bias != nullptr) return W8A8_ERR_DTYPE;
  int rc = check_linear(w_packed, w_scale, epilogue, y, y_dtype, ldy, y_scale, inter_dtype, m,
                        n, k);
  if (rc != W8A8_OK || m == 0 || n == 0) return rc;
  if (x == nullptr) return W8A8_ERR_NULL;
  if (ldx < k) return W8A8_ERR_SHAPE;
  if (!aligned(x, static_cast<uintptr_t>(elem_size(x_dtype)))) return W8A8_ERR_ALIGN;
  if (x_scale_out != nullptr && !aligned(x_scale_out, 4)) return W8A8_ERR_ALIGN;
  if (k > 0 && epilogue <= W8A8_EPI_SILU_MUL_Q8 &&
      fused_gemv_supported(x, x_dtype, ldx, m, n, k, epilogue, ra != nullptr)) {
    // Decode: quantization fused into the GEMV, no workspace.
    LinearOperands op = make_ops(nullptr, 0, nullptr, w_packed, w_scale, bias, epilogue, y,
                                 y_dtype, ldy, y_scale, inter_dtype, m, n, k);
    op.absmax_parts = absmax_parts;
    set_residual(op, ra);
    return status_of(launch_gemv_fused(x, x_dtype, ldx, op, x_scale_out, stream));
  }
  if (workspace == nullptr || workspace_bytes < w8a8_workspace_bytes(m, k))
    return W8A8_ERR_WORKSPACE;
  if (!aligned(workspace, 16)) return W8A8_ERR_ALIGN;
  float* sx = x_scale_out != nullptr ? x_scale_out : static_cast<float*>(workspace);
  int8_t* act = static_cast<int8_t*>(workspace) + scale_region(m);
  const int64_t kp = round_up(k, kTileK);
  const bool gemv = use_gemv(m, n, k);
  hipError_t e = launch_quant_rows(x, x_dtype, ldx, m, k, nullptr, 0, act, kp, kp, !gemv, sx,
                                   stream);
  if (e != hipSuccess) return status_of(e);
  LinearOperands op = make_ops(act, kp, sx, w_packed, w_scale, bias, epilogue, y, y_dtype, ldy,
                               y_scale, inter_dtype, m, n, k);
  op.absmax_parts = absmax_parts;
  set_residual(op, ra);
  return status_of(run_product(op, stream));
}

// w8a8_linear_i8in; absmax_parts as in linear_impl.
int linear_i8in_impl(const int8_t* xq, int64_t ldq, const float* x_scale,
                     const int8_t* w_packed, const float* w_scale, const float* bias,
                     int epilogue, void* y, int y_dtype, int64_t ldy, float y_scale,
                     int inter_dtype, int64_t m, int64_t n, int64_t k, void* workspace,
                     int64_t workspace_bytes, float* absmax_parts, hipStream_t stream,
                     const ResidualAdd* ra = nullptr) {
  if (epilogue == W8A8_EPI_REQUANT) return W8A8_ERR_DTYPE;  // w8a8_linear_i8in_requant
  if (epilogue == W8A8_EPI_DEQUANT_BF16_EXACT && bias != nullptr) return W8A8_ERR_DTYPE;
  int rc = check_linear(w_packed, w_scale, epilogue, y, y_dtype, ldy, y_scale, inter_dtype, m,
                        n, k);
  if (rc != W8A8_OK || m == 0 || n == 0) return rc;
  if (xq == nullptr || (epilogue != W8A8_EPI_I32 && x_scale == nullptr)) return W8A8_ERR_NULL;
  if (ldq < k) return W8A8_ERR_SHAPE;
  if (workspace == nullptr || workspace_bytes < w8a8_workspace_bytes(m, k))
    return W8A8_ERR_WORKSPACE;
  if (!aligned(workspace, 16)) return W8A8_ERR_ALIGN;
  int8_t* act = static_cast<int8_t*>(workspace) + scale_region(m);
  const int8_t* a = nullptr;
  int64_t lda = 0;
  hipError_t e = stage_i8(xq, ldq, m, n, k, act, &a, &lda, stream);
  if (e != hipSuccess) return status_of(e);
  LinearOperands op = make_ops(a, lda, x_scale, w_packed, w_scale, bias, epilogue, y, y_dtype,
                               ldy, y_scale, inter_dtype, m, n, k);
  op.absmax_parts = absmax_parts;
  set_residual(op, ra);
  return status_of(run_product(op, stream));
}

// w8a8_rmsnorm_linear; ss_in (nullable, only without a residual): the
// RMSNorm sums of squares of x per 8 columns as a residual-add epilogue wrote
// them, which the one-kernel route reads instead of summing x itself (the
// same bits: the epilogue sums in the norm kernels' order); the other routes
// sum x in the activation prologue.
int rmsnorm_linear_impl(const void* x, int x_dtype, int64_t ldx, const void* residual,
                        int64_t ld_residual, void* residual_out, int64_t ld_residual_out,
                        const void* norm_weight, float eps, const int8_t* w_packed,
                        const float* w_scale, const float* bias, int epilogue, void* y,
                        int y_dtype, int64_t ldy, float y_scale, int inter_dtype, int64_t m,
                        int64_t n, int64_t k, float* x_scale_out, void* x_out, int64_t ld_x_out,
                        void* workspace, int64_t workspace_bytes, hipStream_t stream,
                        const float* ss_in, int64_t ld_ss_in) {
  if (!half_dtype(x_dtype)) return W8A8_ERR_DTYPE;
  if (epilogue == W8A8_EPI_REQUANT) return W8A8_ERR_DTYPE;
  if (epilogue == W8A8_EPI_DEQUANT_BF16_EXACT && bias != nullptr) return W8A8_ERR_DTYPE;
  int rc = check_linear(w_packed, w_scale, epilogue, y, y_dtype, ldy, y_scale, inter_dtype, m,
                        n, k);
  if (rc != W8A8_OK || m == 0 || n == 0) return rc;
  if (k > prologue_max_k()) return W8A8_ERR_SHAPE;
  if (x == nullptr || norm_weight == nullptr) return W8A8_ERR_NULL;
  if (residual != nullptr && residual_out == nullptr) return W8A8_ERR_NULL;
  if (ldx < k || (residual != nullptr && (ld_residual < k || ld_residual_out < k)) ||
      (x_out != nullptr && ld_x_out < k))
    return W8A8_ERR_SHAPE;
  if (!(eps >= 0.0f)) return W8A8_ERR_SHAPE;
  const uintptr_t xs = static_cast<uintptr_t>(elem_size(x_dtype));
  if (!aligned(x, xs) || !aligned(residual, xs) || !aligned(residual_out, xs) ||
      !aligned(norm_weight, xs) || !aligned(x_out, xs) || !aligned(x_scale_out, 4))
    return W8A8_ERR_ALIGN;
  LinearOperands op = make_ops(nullptr, 0, nullptr, w_packed, w_scale, bias, epilogue, y, y_dtype,
                               ldy, y_scale, inter_dtype, m, n, k);
  // residual_out and x_out are written row by row after the row is read
  // (the prologue), so each may be the very rows of an input; no other
  // overlap is allowed.  The one-kernel route has workgroup 0 write them
  // while the others still read x and the residual, so it is taken only
  // when they overlap neither input.
  const int64_t es = elem_size(x_dtype);
  const void* r_out = residual != nullptr ? residual_out : nullptr;  // written only with a residual
  if (!rows_alias_ok(r_out, ld_residual_out, es, x, ldx, es, m, k) ||
      !rows_alias_ok(r_out, ld_residual_out, es, residual, ld_residual, es, m, k) ||
      !rows_alias_ok(x_out, ld_x_out, es, x, ldx, es, m, k) ||
      !rows_alias_ok(x_out, ld_x_out, es, residual, ld_residual, es, m, k) ||
      overlap(r_out, ld_residual_out, es, x_out, ld_x_out, es, m, k))
    return W8A8_ERR_OVERLAP;
  const bool in_place = overlap(r_out, ld_residual_out, es, x, ldx, es, m, k) ||
                        overlap(r_out, ld_residual_out, es, residual, ld_residual, es, m, k) ||
                        overlap(x_out, ld_x_out, es, x, ldx, es, m, k) ||
                        overlap(x_out, ld_x_out, es, residual, ld_residual, es, m, k);
  const bool fused_epilogue = epilogue <= W8A8_EPI_SILU_MUL || epilogue == W8A8_EPI_SILU_MUL_Q8;
  if (k > 0 && fused_epilogue && !in_place &&
      fused_norm_supported(x, x_dtype, ldx, residual, ld_residual, residual_out,
                           ld_residual_out, norm_weight, x_out, ld_x_out, m, n, k)) {
    // One kernel: residual add, RMSNorm, per-token quantization, GEMV, epilogue.
    return status_of(launch_gemv_fused_norm(x, x_dtype, ldx, residual, ld_residual, residual_out,
                                            ld_residual_out, norm_weight, eps, x_out, ld_x_out,
                                            op, x_scale_out, stream,
                                            residual == nullptr ? ss_in : nullptr, ld_ss_in));
  }
  // Otherwise the activation prologue writes the int8 rows the product
  // reads: row-major for the GEMV, the packed tiles for the GEMM.
  if (workspace == nullptr || workspace_bytes < w8a8_workspace_bytes(m, k))
    return W8A8_ERR_WORKSPACE;
  if (!aligned(workspace, 16)) return W8A8_ERR_ALIGN;
  float* sx = x_scale_out != nullptr ? x_scale_out : static_cast<float*>(workspace);
  int8_t* act = static_cast<int8_t*>(workspace) + scale_region(m);
  const int64_t kp = round_up(k, kTileK);
  const bool gemv = use_gemv(m, n, k);
  // The GEMV reads whole 64-column blocks: the prologue writes zeros in the
  // pad columns K..kp of its row-major rows.
  hipError_t e = launch_prologue_quant(x, x_dtype, ldx, residual, ld_residual, residual_out,
                                       ld_residual_out, norm_weight, x_dtype, eps, nullptr,
                                       nullptr, m, k, act, kp, sx, x_out, ld_x_out, stream, !gemv,
                                       kp);
  if (e != hipSuccess) return status_of(e);
  op.a = act;
  op.lda = kp;
  op.sx = sx;
  return status_of(gemv ? launch_gemv(op, stream) : launch_gemm(op, stream));
}

// Looks up (once per device) the current device's address of `scratch`.
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return status_of(e);
  if (dev < 0 || dev >= kMaxDevices) return W8A8_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return status_of(e);
    if (p == nullptr) return W8A8_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return W8A8_OK;
}

}  // namespace

extern "C" {

int w8a8_abi_version(void) { return W8A8_ABI_VERSION; }

const char* w8a8_status_string(int status) {
  switch (status) {
    case W8A8_OK:
      return "ok";
    case W8A8_ERR_NULL:
      return "required pointer is null";
    case W8A8_ERR_SHAPE:
      return "invalid shape, leading dimension or scale";
    case W8A8_ERR_DTYPE:
      return "unsupported dtype or epilogue";
    case W8A8_ERR_ALIGN:
      return "misaligned pointer or leading dimension";
    case W8A8_ERR_WORKSPACE:
      return "workspace missing or too small";
    case W8A8_ERR_HIP:
      return "HIP kernel launch failed";
    case W8A8_ERR_TOO_LARGE:
      return "problem needs more than the static scratch of w8a8_linear_noalloc";
    case W8A8_ERR_OVERLAP:
      return "an output overlaps an input other than row for row";
    default:
      return "unknown status";
  }
}

int w8a8_last_hip_error(void) { return g_last_hip_error; }

int64_t w8a8_packed_bytes(int64_t rows, int64_t k) {
  if (rows < 0 || k < 0) return -1;
  return round_up(rows, kTileRows) * round_up(k, kTileK);
}

int64_t w8a8_workspace_bytes(int64_t m, int64_t k) {
  if (m < 0 || k < 0) return -1;
  return scale_region(m) + act_region(m, k);
}

int w8a8_gemm_tile_config(int64_t m, int64_t n, int64_t cus) {
  if (m <= 0 || n <= 0 || cus <= 0 || m > kMaxRows || n > kMaxRows) return -1;
  return gemm_tile_choice(ceil_div(m, kTileRows), ceil_div(n, kTileRows), cus);
}

int w8a8_quant_rows(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                    int8_t* q, int64_t ldq, float* scales, hipStream_t stream) {
  if (rows < 0 || k < 0 || rows > kMaxRows) return W8A8_ERR_SHAPE;
  if (!float_dtype(x_dtype)) return W8A8_ERR_DTYPE;
  if (rows == 0) return W8A8_OK;
  if (x == nullptr || q == nullptr || scales == nullptr) return W8A8_ERR_NULL;
  if (ldx < k || ldq < k) return W8A8_ERR_SHAPE;
  if (!aligned(x, static_cast<uintptr_t>(elem_size(x_dtype))) || !aligned(scales, 4))
    return W8A8_ERR_ALIGN;
  return status_of(launch_quant_rows(x, x_dtype, ldx, rows, k, nullptr, 0, q, ldq, k, false,
                                     scales, stream));
}

int w8a8_quant_rows_scaled(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                           const float* scale, int64_t scale_stride, int8_t* q, int64_t ldq,
                           hipStream_t stream) {
  if (rows < 0 || k < 0 || scale_stride < 0 || rows > kMaxRows) return W8A8_ERR_SHAPE;
  if (!float_dtype(x_dtype)) return W8A8_ERR_DTYPE;
  if (rows == 0) return W8A8_OK;
  if (x == nullptr || q == nullptr || scale == nullptr) return W8A8_ERR_NULL;
  if (ldx < k || ldq < k) return W8A8_ERR_SHAPE;
  if (!aligned(x, static_cast<uintptr_t>(elem_size(x_dtype))) || !aligned(scale, 4))
    return W8A8_ERR_ALIGN;
  return status_of(launch_quant_rows(x, x_dtype, ldx, rows, k, scale, scale_stride, q, ldq, k,
                                     false, nullptr, stream));
}

int w8a8_pack_rows(const int8_t* src, int64_t rows, int64_t k, int64_t ld, int layout,
                   int8_t* packed, hipStream_t stream) {
  if (rows < 0 || k < 0 || rows > kMaxRows) return W8A8_ERR_SHAPE;
  if (layout != W8A8_ROWS_AS_IS && layout != W8A8_ROWS_INTERLEAVE_HALVES) return W8A8_ERR_DTYPE;
  if (layout == W8A8_ROWS_INTERLEAVE_HALVES && rows % 2 != 0) return W8A8_ERR_SHAPE;
  if (rows == 0 || k == 0) return W8A8_OK;
  if (src == nullptr || packed == nullptr) return W8A8_ERR_NULL;
  if (ld < k) return W8A8_ERR_SHAPE;
  if (!aligned(packed, 16)) return W8A8_ERR_ALIGN;
  return status_of(launch_pack_rows(src, rows, k, ld, layout, packed, stream));
}

int w8a8_gemm_i32(const int8_t* xq, int64_t ldq, const int8_t* w_packed, int32_t* acc,
                  int64_t ldacc, int64_t m, int64_t n, int64_t k, void* workspace,
                  int64_t workspace_bytes, hipStream_t stream) {
  int rc = check_linear(w_packed, nullptr, W8A8_EPI_I32, acc, kI32, ldacc, 0.0f, kF16, m, n, k);
  if (rc != W8A8_OK || m == 0 || n == 0) return rc;
  if (k > 0 && xq == nullptr) return W8A8_ERR_NULL;
  if (ldq < k) return W8A8_ERR_SHAPE;
  if (workspace == nullptr || workspace_bytes < w8a8_workspace_bytes(m, k))
    return W8A8_ERR_WORKSPACE;
  if (!aligned(workspace, 16)) return W8A8_ERR_ALIGN;
  int8_t* act = static_cast<int8_t*>(workspace) + scale_region(m);
  const int8_t* a = nullptr;
  int64_t lda = 0;
  hipError_t e = stage_i8(xq, ldq, m, n, k, act, &a, &lda, stream);
  if (e != hipSuccess) return status_of(e);
  LinearOperands op = make_ops(a, lda, nullptr, w_packed, nullptr, nullptr, W8A8_EPI_I32, acc,
                               kI32, ldacc, 0.0f, kF16, m, n, k);
  return status_of(run_product(op, stream));
}

int w8a8_linear(const void* x, int x_dtype, int64_t ldx, const int8_t* w_packed,
                const float* w_scale, const float* bias, int epilogue, void* y, int y_dtype,
                int64_t ldy, float y_scale, int inter_dtype, int64_t m, int64_t n, int64_t k,
                float* x_scale_out, void* workspace, int64_t workspace_bytes,
                hipStream_t stream) {
  return linear_impl(x, x_dtype, ldx, w_packed, w_scale, bias, epilogue, y, y_dtype, ldy,
                     y_scale, inter_dtype, m, n, k, x_scale_out, workspace, workspace_bytes,
                     nullptr, stream);
}

int w8a8_linear_i8in(const int8_t* xq, int64_t ldq, const float* x_scale,
                     const int8_t* w_packed, const float* w_scale, const float* bias,
                     int epilogue, void* y, int y_dtype, int64_t ldy, float y_scale,
                     int inter_dtype, int64_t m, int64_t n, int64_t k, void* workspace,
                     int64_t workspace_bytes, hipStream_t stream) {
  return linear_i8in_impl(xq, ldq, x_scale, w_packed, w_scale, bias, epilogue, y, y_dtype, ldy,
                          y_scale, inter_dtype, m, n, k, workspace, workspace_bytes, nullptr,
                          stream);
}

int64_t w8a8_gateup_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m < 0 || n < 0 || k < 0) return -1;
  return parts_region(m, n) + w8a8_workspace_bytes(m, k);
}

int w8a8_gateup_silu_mul(const void* x, int x_dtype, int64_t ldx, const float* x_scale,
                         const int8_t* w_packed, const float* w_scale, const float* bias, void* h,
                         int h_dtype, int64_t ldh, int8_t* hq, int64_t ldhq, float* h_scale,
                         int64_t m, int64_t n, int64_t k, void* workspace,
                         int64_t workspace_bytes, hipStream_t stream) {
  if (!half_dtype(h_dtype)) return W8A8_ERR_DTYPE;
  if (m < 0 || n < 0 || k < 0) return W8A8_ERR_SHAPE;
  if (m == 0 || n == 0)
    return check_linear(w_packed, w_scale, W8A8_EPI_SILU_MUL, h, h_dtype, ldh, 0.0f, h_dtype, m,
                        n, k);
  if (h == nullptr || hq == nullptr || h_scale == nullptr) return W8A8_ERR_NULL;
  if (ldhq < n / 2) return W8A8_ERR_SHAPE;
  if (!aligned(h_scale, 4)) return W8A8_ERR_ALIGN;
  if (workspace == nullptr || workspace_bytes < w8a8_gateup_workspace_bytes(m, n, k))
    return W8A8_ERR_WORKSPACE;
  if (!aligned(workspace, 256)) return W8A8_ERR_ALIGN;
  // Workspace: [partial maxima, m x ceil(n/16) binary32][w8a8_linear's].
  float* parts = static_cast<float*>(workspace);
  void* ws = static_cast<int8_t*>(workspace) + parts_region(m, n);
  const int64_t ws_bytes = workspace_bytes - parts_region(m, n);
  // Phase 1: the SiLU*mul linear; its epilogue leaves every row's max |h|
  // per 16-row weight block in `parts`.
  int rc;
  if (x_dtype == W8A8_I8) {
    rc = linear_i8in_impl(static_cast<const int8_t*>(x), ldx, x_scale, w_packed, w_scale, bias,
                          W8A8_EPI_SILU_MUL, h, h_dtype, ldh, 0.0f, h_dtype, m, n, k, ws, ws_bytes,
                          parts, stream);
  } else {
    rc = linear_impl(x, x_dtype, ldx, w_packed, w_scale, bias, W8A8_EPI_SILU_MUL, h, h_dtype, ldh,
                     0.0f, h_dtype, m, n, k, nullptr, ws, ws_bytes, parts, stream);
  }
  if (rc != W8A8_OK) return rc;
  // Phase 2: per-token int8 h with scale_from_absmax of each row's max.
  return status_of(launch_quant_rows_parts(h, h_dtype, ldh, m, n / 2, parts,
                                           ceil_div(n, kTileRows), hq, ldhq, h_scale, stream));
}

int w8a8_rmsnorm_linear(const void* x, int x_dtype, int64_t ldx, const void* residual,
                        int64_t ld_residual, void* residual_out, int64_t ld_residual_out,
                        const void* norm_weight, float eps, const int8_t* w_packed,
                        const float* w_scale, const float* bias, int epilogue, void* y,
                        int y_dtype, int64_t ldy, float y_scale, int inter_dtype, int64_t m,
                        int64_t n, int64_t k, float* x_scale_out, void* x_out, int64_t ld_x_out,
                        void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  return rmsnorm_linear_impl(x, x_dtype, ldx, residual, ld_residual, residual_out,
                             ld_residual_out, norm_weight, eps, w_packed, w_scale, bias, epilogue,
                             y, y_dtype, ldy, y_scale, inter_dtype, m, n, k, x_scale_out, x_out,
                             ld_x_out, workspace, workspace_bytes, stream, nullptr, 0);
}

int w8a8_rmsnorm_linear_ss(const void* x, int x_dtype, int64_t ldx, const float* ss_parts,
                           int64_t ld_parts, const void* norm_weight, float eps,
                           const int8_t* w_packed, const float* w_scale, const float* bias,
                           int epilogue, void* y, int y_dtype, int64_t ldy, float y_scale,
                           int inter_dtype, int64_t m, int64_t n, int64_t k, float* x_scale_out,
                           void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  if (m > 0 && n > 0 && k > 0 && ss_parts != nullptr) {
    if (ld_parts < ceil_div(k, 8)) return W8A8_ERR_SHAPE;
    if (!aligned(ss_parts, 4)) return W8A8_ERR_ALIGN;
  }
  return rmsnorm_linear_impl(x, x_dtype, ldx, nullptr, 0, nullptr, 0, norm_weight, eps, w_packed,
                             w_scale, bias, epilogue, y, y_dtype, ldy, y_scale, inter_dtype, m, n,
                             k, x_scale_out, nullptr, 0, workspace, workspace_bytes, stream,
                             ss_parts, ld_parts);
}

int w8a8_linear_residual(const void* x, int x_dtype, int64_t ldx, const int8_t* w_packed,
                         const float* w_scale, const float* bias, void* y, int y_dtype,
                         int64_t ldy, const void* residual, int64_t ld_residual, float* ss_parts,
                         int64_t ld_parts, int64_t m, int64_t n, int64_t k, void* workspace,
                         int64_t workspace_bytes, hipStream_t stream) {
  const ResidualAdd ra{residual, ld_residual, ss_parts, ld_parts};
  if (m < 0 || n < 0) return W8A8_ERR_SHAPE;
  const int rc = check_residual(ra, y, y_dtype, ldy, m, n);
  if (rc != W8A8_OK) return rc;
  return linear_impl(x, x_dtype, ldx, w_packed, w_scale, bias, W8A8_EPI_DEQUANT, y, y_dtype, ldy,
                     0.0f, y_dtype, m, n, k, nullptr, workspace, workspace_bytes, nullptr, stream,
                     &ra);
}

int w8a8_linear_i8in_residual(const int8_t* xq, int64_t ldq, const float* x_scale,
                              const int8_t* w_packed, const float* w_scale, const float* bias,
                              void* y, int y_dtype, int64_t ldy, const void* residual,
                              int64_t ld_residual, float* ss_parts, int64_t ld_parts, int64_t m,
                              int64_t n, int64_t k, void* workspace, int64_t workspace_bytes,
                              hipStream_t stream) {
  const ResidualAdd ra{residual, ld_residual, ss_parts, ld_parts};
  if (m < 0 || n < 0) return W8A8_ERR_SHAPE;
  const int rc = check_residual(ra, y, y_dtype, ldy, m, n);
  if (rc != W8A8_OK) return rc;
  return linear_i8in_impl(xq, ldq, x_scale, w_packed, w_scale, bias, W8A8_EPI_DEQUANT, y, y_dtype,
                          ldy, 0.0f, y_dtype, m, n, k, workspace, workspace_bytes, nullptr, stream,
                          &ra);
}

int w8a8_linear_packed(const int8_t* xq_packed, const float* x_scale, const int8_t* w_packed,
                       const float* w_scale, const float* bias, int epilogue, void* y,
                       int y_dtype, int64_t ldy, float y_scale, int inter_dtype, int64_t m,
                       int64_t n, int64_t k, hipStream_t stream) {
  if (epilogue == W8A8_EPI_REQUANT) return W8A8_ERR_DTYPE;  // w8a8_linear_i8in_requant
  if (epilogue == W8A8_EPI_DEQUANT_BF16_EXACT && bias != nullptr) return W8A8_ERR_DTYPE;
  int rc = check_linear(w_packed, w_scale, epilogue, y, y_dtype, ldy, y_scale, inter_dtype, m,
                        n, k);
  if (rc != W8A8_OK || m == 0 || n == 0) return rc;
  if (xq_packed == nullptr || (epilogue != W8A8_EPI_I32 && x_scale == nullptr))
    return W8A8_ERR_NULL;
  if (!aligned(xq_packed, 16)) return W8A8_ERR_ALIGN;
  LinearOperands op = make_ops(xq_packed, round_up(k, kTileK), x_scale, w_packed, w_scale, bias,
                               epilogue, y, y_dtype, ldy, y_scale, inter_dtype, m, n, k);
  return status_of(launch_gemm(op, stream));
}

int w8a8_linear_noalloc(const void* x, int x_dtype, int64_t ldx, const int8_t* w_packed,
                        const float* w_scale, const float* bias, int epilogue, void* y,
                        int y_dtype, int64_t ldy, float y_scale, int inter_dtype, int64_t m,
                        int64_t n, int64_t k, float* x_scale_out, hipStream_t stream) {
  // Without a workspace, w8a8_linear validates every argument and either runs
  // (decode shapes fused with the quantization need none) or reports
  // W8A8_ERR_WORKSPACE before any launch.
  int rc = w8a8_linear(x, x_dtype, ldx, w_packed, w_scale, bias, epilogue, y, y_dtype, ldy,
                       y_scale, inter_dtype, m, n, k, x_scale_out, nullptr, 0, stream);
  if (rc != W8A8_ERR_WORKSPACE) return rc;
  if (w8a8_workspace_bytes(m, k) > W8A8_NOALLOC_SCRATCH_BYTES) return W8A8_ERR_TOO_LARGE;
  void* ws = nullptr;
  rc = scratch_address(&ws);
  if (rc != W8A8_OK) return rc;
  // The quantization writes every scratch byte the product then reads (the
  // scales, and the int8 rows with their zero padding), so no clearing is
  // needed between calls.
  return w8a8_linear(x, x_dtype, ldx, w_packed, w_scale, bias, epilogue, y, y_dtype, ldy,
                     y_scale, inter_dtype, m, n, k, x_scale_out, ws,
                     W8A8_NOALLOC_SCRATCH_BYTES, stream);
}

int w8a8_prologue_quant(const void* x, int x_dtype, int64_t ldx, const void* residual,
                        int64_t ld_residual, void* residual_out, int64_t ld_residual_out,
                        const void* norm_weight, int norm_weight_dtype, float eps,
                        const void* smooth, const float* static_scale, int64_t m, int64_t k,
                        int8_t* q, int64_t ldq, float* scales_out, void* x_out,
                        int64_t ld_x_out, hipStream_t stream) {
  if (!half_dtype(x_dtype)) return W8A8_ERR_DTYPE;
  const bool w32 = norm_weight != nullptr && norm_weight_dtype == kF32;
  if (norm_weight != nullptr && norm_weight_dtype != x_dtype && !w32) return W8A8_ERR_DTYPE;
  if (m < 0 || k < 0 || k > prologue_max_k() || m > kMaxRows) return W8A8_ERR_SHAPE;
  if (m == 0 || k == 0) return W8A8_OK;
  if (x == nullptr || q == nullptr) return W8A8_ERR_NULL;
  if (residual != nullptr && residual_out == nullptr) return W8A8_ERR_NULL;
  if (static_scale == nullptr && scales_out == nullptr) return W8A8_ERR_NULL;
  if (ldx < k || ldq < k) return W8A8_ERR_SHAPE;
  if (residual != nullptr && (ld_residual < k || ld_residual_out < k)) return W8A8_ERR_SHAPE;
  if (x_out != nullptr && ld_x_out < k) return W8A8_ERR_SHAPE;
  if (!(eps >= 0.0f)) return W8A8_ERR_SHAPE;
  const uintptr_t xs = static_cast<uintptr_t>(elem_size(x_dtype));
  if (!aligned(x, xs) || !aligned(residual, xs) || !aligned(residual_out, xs) ||
      !aligned(smooth, xs) || !aligned(norm_weight, w32 ? 4 : xs) || !aligned(static_scale, 4) ||
      !aligned(scales_out, 4) || !aligned(x_out, w32 ? 4 : xs))
    return W8A8_ERR_ALIGN;
  // Each row is read before it is written: an output may be the very rows of
  // an input, and must not overlap one otherwise, nor the other output.
  const int64_t es = static_cast<int64_t>(xs), eo = w32 ? 4 : es;
  const void* r_out = residual != nullptr ? residual_out : nullptr;  // written only with a residual
  if (!rows_alias_ok(r_out, ld_residual_out, es, x, ldx, es, m, k) ||
      !rows_alias_ok(r_out, ld_residual_out, es, residual, ld_residual, es, m, k) ||
      !rows_alias_ok(x_out, ld_x_out, eo, x, ldx, es, m, k) ||
      !rows_alias_ok(x_out, ld_x_out, eo, residual, ld_residual, es, m, k) ||
      overlap(r_out, ld_residual_out, es, x_out, ld_x_out, eo, m, k))
    return W8A8_ERR_OVERLAP;
  return status_of(launch_prologue_quant(x, x_dtype, ldx, residual, ld_residual, residual_out,
                                         ld_residual_out, norm_weight, norm_weight_dtype, eps,
                                         smooth, static_scale, m, k, q, ldq, scales_out, x_out,
                                         ld_x_out, stream));
}

int w8a8_linear_i8in_requant(const int8_t* xq, int64_t ldq, const int8_t* w_packed,
                             const uint32_t* multiplier, const int32_t* right_shift,
                             const int32_t* bias_i32, int8_t* y, int64_t ldy, int64_t m,
                             int64_t n, int64_t k, void* workspace, int64_t workspace_bytes,
                             hipStream_t stream) {
  int rc = check_linear(w_packed, nullptr, W8A8_EPI_REQUANT, y, kI8, ldy, 0.0f, kF16, m, n, k);
  if (rc != W8A8_OK || m == 0 || n == 0) return rc;
  if (xq == nullptr || multiplier == nullptr || right_shift == nullptr) return W8A8_ERR_NULL;
  if (!aligned(multiplier, 4) || !aligned(right_shift, 4) || !aligned(bias_i32, 4))
    return W8A8_ERR_ALIGN;
  if (ldq < k) return W8A8_ERR_SHAPE;
  if (workspace == nullptr || workspace_bytes < w8a8_workspace_bytes(m, k))
    return W8A8_ERR_WORKSPACE;
  if (!aligned(workspace, 16)) return W8A8_ERR_ALIGN;
  int8_t* act = static_cast<int8_t*>(workspace) + scale_region(m);
  const int8_t* a = nullptr;
  int64_t lda = 0;
  hipError_t e = stage_i8(xq, ldq, m, n, k, act, &a, &lda, stream);
  if (e != hipSuccess) return status_of(e);
  LinearOperands op = make_ops(a, lda, nullptr, w_packed, nullptr, nullptr, W8A8_EPI_REQUANT, y,
                               kI8, ldy, 0.0f, kF16, m, n, k);
  op.rq_mult = multiplier;
  op.rq_shift = right_shift;
  op.rq_bias = bias_i32;
  return status_of(run_product(op, stream));
}

int w8a8_requantize_i32(const int32_t* acc, int64_t ld_acc, const int32_t* bias_i32,
                        const uint32_t* multiplier, const int32_t* right_shift, int8_t* y,
                        int64_t ldy, int64_t m, int64_t n, hipStream_t stream) {
  if (m < 0 || n < 0) return W8A8_ERR_SHAPE;
  if (m == 0 || n == 0) return W8A8_OK;
  if (acc == nullptr || multiplier == nullptr || right_shift == nullptr || y == nullptr)
    return W8A8_ERR_NULL;
  if (ld_acc < n || ldy < n) return W8A8_ERR_SHAPE;
  if (!aligned(acc, 4) || !aligned(multiplier, 4) || !aligned(right_shift, 4) ||
      !aligned(bias_i32, 4))
    return W8A8_ERR_ALIGN;
  return status_of(
      launch_requant_i32(acc, ld_acc, bias_i32, multiplier, right_shift, y, ldy, m, n, stream));
}

int w8a8_dequant_i32_bf16(const int32_t* acc, int64_t ld_acc, const uint16_t* sa_bits,
                          const uint16_t* sw_bits, uint16_t* y, int64_t ldy, int64_t m,
                          int64_t n, hipStream_t stream) {
  if (m < 0 || n < 0) return W8A8_ERR_SHAPE;
  if (m == 0 || n == 0) return W8A8_OK;
  if (acc == nullptr || sa_bits == nullptr || sw_bits == nullptr || y == nullptr)
    return W8A8_ERR_NULL;
  if (ld_acc < n || ldy < n) return W8A8_ERR_SHAPE;
  if (!aligned(acc, 4) || !aligned(sa_bits, 2) || !aligned(sw_bits, 2) || !aligned(y, 2))
    return W8A8_ERR_ALIGN;
  return status_of(launch_dequant_i32_bf16(acc, ld_acc, sa_bits, sw_bits, y, ldy, m, n, stream));
}

int w8a8_dense_gemv(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                    void* y, int64_t ldy, int dtype, int64_t m, int64_t n, int64_t k,
                    hipStream_t stream) {
  if (!half_dtype(dtype)) return W8A8_ERR_DTYPE;
  if (m < 0 || n < 0 || k < 0 || m > 16) return W8A8_ERR_SHAPE;
  if (m == 0 || n == 0) return W8A8_OK;
  if (k == 0 || k % 8 != 0 || k > dense_gemv_max_k()) return W8A8_ERR_SHAPE;
  if (ldx < k || ldw < k || ldy < n || ldx % 8 != 0 || ldw % 8 != 0) return W8A8_ERR_SHAPE;
  if (m * ldx * 2 >= (int64_t{1} << 31) || 16 * ldw * 2 >= (int64_t{1} << 31))
    return W8A8_ERR_SHAPE;
  if (x == nullptr || w == nullptr || y == nullptr) return W8A8_ERR_NULL;
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(y, 2) || !aligned(bias, 2))
    return W8A8_ERR_ALIGN;
  // y is written while x, w and bias are read by other workgroups.
  auto span = [](const void* p, int64_t rows, int64_t ld, int64_t cols) {
    const uintptr_t b = reinterpret_cast<uintptr_t>(p);
    return std::make_pair(b, b + static_cast<uintptr_t>(((rows - 1) * ld + cols) * 2));
  };
  auto meets = [](std::pair<uintptr_t, uintptr_t> a, std::pair<uintptr_t, uintptr_t> b) {
    return a.first < b.second && b.first < a.second;
  };
  const auto ys = span(y, m, ldy, n);
  if (meets(ys, span(x, m, ldx, k)) || meets(ys, span(w, n, ldw, k)) ||
      (bias != nullptr && meets(ys, span(bias, 1, n, n))))
    return W8A8_ERR_OVERLAP;
  return status_of(launch_gemv_dense(x, ldx, w, ldw, bias, y, ldy, dtype, m, n, k, stream));
}

}  // extern "C"
