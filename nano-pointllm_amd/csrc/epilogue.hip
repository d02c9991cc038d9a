// Elementwise epilogues over int32 accumulators that the caller already holds
// (for example from w8a8_gemm_i32): the hardware model's integer contracts.
//
//   requant_i32_kernel     INT32 -> A8 requantization, requantize_int32
//                          (architecture_simulator/gtsu_cycle/requant.py:98-119)
//   dequant_bf16_kernel    INT32 x FP16 x FP16 -> BF16 with one rounding,
//                          dequantize_int32_to_bf16
//                          (architecture_simulator/gtsu_cycle/bf16_dequant.py:47-77)
//
//   add_rows_ss_kernel     the residual add of a decoder layer on 16-bit rows
//                          already written by a linear, with the RMSNorm sums
//                          of squares per 8-column chunk (the routes whose
//                          kernels have no residual-add epilogue)
//
// The first two are a few integer operations per 4-byte accumulator
// (HBM-bound): each thread takes four consecutive columns of a row,
// grid-strided.
#include "w8a8_internal.h"

namespace w8a8 {

namespace {

constexpr int kEpiThreads = 256;
constexpr int kCols = 4;  // columns per thread

__global__ __launch_bounds__(kEpiThreads) void requant_i32_kernel(
    const int32_t* __restrict__ acc, int64_t ld_acc, const int32_t* __restrict__ bias,
    const uint32_t* __restrict__ mult, const int32_t* __restrict__ shift,
    int8_t* __restrict__ y, int64_t ldy, int64_t M, int64_t N) {
  const int64_t groups = (N + kCols - 1) / kCols;
  const int64_t total = M * groups;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kEpiThreads + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kEpiThreads) {
    const int64_t m = i / groups;
    const int64_t n0 = (i - m * groups) * kCols;
#pragma unroll
    for (int c = 0; c < kCols; ++c) {
      const int64_t n = n0 + c;
      if (n < N) {
        y[m * ldy + n] = static_cast<int8_t>(
            requant1(acc[m * ld_acc + n], bias != nullptr ? bias[n] : 0, mult[n], shift[n]));
      }
    }
  }
}

__global__ __launch_bounds__(kEpiThreads) void dequant_bf16_kernel(
    const int32_t* __restrict__ acc, int64_t ld_acc, const uint16_t* __restrict__ sa_bits,
    const uint16_t* __restrict__ sw_bits, uint16_t* __restrict__ y, int64_t ldy, int64_t M,
    int64_t N) {
  const int64_t groups = (N + kCols - 1) / kCols;
  const int64_t total = M * groups;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kEpiThreads + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kEpiThreads) {
    const int64_t m = i / groups;
    const int64_t n0 = (i - m * groups) * kCols;
    const uint16_t sa = sa_bits[m];
#pragma unroll
    for (int c = 0; c < kCols; ++c) {
      const int64_t n = n0 + c;
      if (n < N) y[m * ldy + n] = dequant_bf16_exact(acc[m * ld_acc + n], sa, sw_bits[n]);
    }
  }
}

// y[m, n] = dtype(y[m, n] + res[m, n]) and, with parts, the chunk sums
// parts[m * ld_parts + c] of the new rows.  One thread per column of a row
// padded to whole chunks (ncol = 8 ceil(N / 8)), so the 8 lanes of a chunk
// are consecutive; every lane reaches the chunk sums (no early exit).
template <typename T>
__global__ __launch_bounds__(kEpiThreads) void add_rows_ss_kernel(
    T* __restrict__ y, int64_t ldy, const T* __restrict__ res, int64_t ld_res,
    float* __restrict__ parts, int64_t ld_parts, int64_t M, int64_t N, int64_t ncol) {
  const int64_t total = M * ncol;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kEpiThreads;
  const int64_t span = (total + step - 1) / step * step;  // every lane runs every trip
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kEpiThreads + threadIdx.x; i < span;
       i += step) {
    const int64_t m = i / ncol;
    const int64_t n = i - m * ncol;
    const bool ok = i < total && n < N;
    float v = 0.0f;
    if (ok) {
      const T o = add_rounded(y[m * ldy + n], res[m * ld_res + n]);
      y[m * ldy + n] = o;
      v = to_f32(o);
    }
    if (parts != nullptr) {
      const float cs = chunk_sumsq8(v);
      if ((n & 7) == 0 && ok) parts[m * ld_parts + (n >> 3)] = cs;
    }
  }
}

// Enough workgroups to fill the chip several times over, no more.
unsigned grid_for(int64_t items) {
  const int64_t wgs = (items + kEpiThreads - 1) / kEpiThreads;
  return static_cast<unsigned>(wgs < 4096 ? (wgs > 0 ? wgs : 1) : 4096);
}

}  // namespace

hipError_t launch_requant_i32(const int32_t* acc, int64_t ld_acc, const int32_t* bias,
                              const uint32_t* mult, const int32_t* shift, int8_t* y, int64_t ldy,
                              int64_t M, int64_t N, hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  hipLaunchKernelGGL(requant_i32_kernel, dim3(grid_for(M * ((N + kCols - 1) / kCols))),
                     dim3(kEpiThreads), 0, st, acc, ld_acc, bias, mult, shift, y, ldy, M, N);
  return hipGetLastError();
}

hipError_t launch_dequant_i32_bf16(const int32_t* acc, int64_t ld_acc, const uint16_t* sa_bits,
                                   const uint16_t* sw_bits, uint16_t* y, int64_t ldy, int64_t M,
                                   int64_t N, hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  hipLaunchKernelGGL(dequant_bf16_kernel, dim3(grid_for(M * ((N + kCols - 1) / kCols))),
                     dim3(kEpiThreads), 0, st, acc, ld_acc, sa_bits, sw_bits, y, ldy, M, N);
  return hipGetLastError();
}

hipError_t launch_add_rows_ss(void* y, int dtype, int64_t ldy, const void* res, int64_t ld_res,
                              float* parts, int64_t ld_parts, int64_t M, int64_t N,
                              hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  const int64_t ncol = (N + 7) / 8 * 8;
  const dim3 grid(grid_for(M * ncol));
  if (dtype == kF16) {
    hipLaunchKernelGGL(add_rows_ss_kernel<__half>, grid, dim3(kEpiThreads), 0, st,
                       static_cast<__half*>(y), ldy, static_cast<const __half*>(res), ld_res,
                       parts, ld_parts, M, N, ncol);
  } else if (dtype == kBF16) {
    hipLaunchKernelGGL(add_rows_ss_kernel<__hip_bfloat16>, grid, dim3(kEpiThreads), 0, st,
                       static_cast<__hip_bfloat16*>(y), ldy,
                       static_cast<const __hip_bfloat16*>(res), ld_res, parts, ld_parts, M, N,
                       ncol);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace w8a8
