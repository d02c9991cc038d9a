// Fused activation prologue of the W8A8 linear: one pass over each row of x
//   [residual add] -> [RMSNorm] -> [SmoothQuant divide] -> int8 quantization
// producing the int8 row and its scale for the int8-in GEMV / GEMM.
//
//   residual add   summed = x + residual in the input dtype, also written out
//                  (LightweightRMSNorm.residual_norm,
//                  nanopointllm/llama/lightweight_runner.py:247-257)
//   RMSNorm        y = weight * dtype(f32(x) * 1/sqrt(mean(f32(x)^2) + eps))
//                  (LightweightRMSNorm.forward, lightweight_runner.py:239-245):
//                  the product is rounded to the input dtype when the weight
//                  has that dtype and kept in binary32 for a binary32 weight,
//                  as torch's type promotion does
//   smooth divide  y = dtype(f32(y) / f32(smooth[k]))  (the SmoothQuant input
//                  transform, nanopointllm/compression/w8a8.py:351-359)
//   quantization   per-token dynamic scale (w8a8.py:46-50, 106-115) or one
//                  static scale (w8a8.py:94-103), quantize_symmetric
//                  (w8a8.py:33-43)
//
// One workgroup per row; each thread keeps REG chunks of 8 elements in
// registers between the reductions (sum of squares, absmax) and the writes,
// so x is read once.  The sum of squares is a binary32 sum: for K <= 4096
// (one chunk per thread) in the order every RMSNorm route shares (per chunk,
// pairwise over 8 consecutive chunks, then a wavefront butterfly over the 64
// tree sums), for longer rows per thread, then a wavefront butterfly, then
// across wavefronts; every other step is an exactly rounded elementwise
// operation.
#include <type_traits>

#include "w8a8_internal.h"

namespace w8a8 {

namespace {

constexpr int kProThreads = 512;

struct PrologueParams {
  const void* x;
  int64_t ldx;
  const void* residual;
  int64_t ld_res;
  void* residual_out;
  int64_t ld_res_out;
  const void* norm_weight;  // TW [K] or null
  float eps;
  const void* smooth;       // TX [K] or null
  const float* static_scale;  // one value, or null for a per-row scale
  int64_t M;
  int64_t K;
  int8_t* q;
  int64_t ldq;
  float* scales_out;
  void* x_out;  // TY [M, ld_xout] or null
  int64_t ld_xout;
  // 0: q is row-major [M, ldq].  Otherwise q is the packed 16x64 tiles of
  // the GEMM with KB k-blocks; the grid then covers ceil(M/16)*16 rows and
  // every row writes all KB*64 columns (zeros past K and in the pad rows).
  int64_t KB;
  // Row-major q: columns written per row, K <= q_cols <= ldq, zeros past K
  // (the GEMV reads whole 64-column blocks).
  int64_t q_cols;
};

__device__ inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

template <typename T>
__device__ inline float round_to(float v) {
  return to_f32(from_f32<T>(v));
}

// Sum (or max of |x|) over the workgroup of one float per thread, every
// thread getting it: the xor butterfly within each wavefront, then the
// wavefront results in order.
template <bool MAX>
__device__ inline float block_reduce(float v, float* red) {
  v = MAX ? wave_max_abs(v) : wave_sum_xor(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();  // red[] may still be read from a previous reduction
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kProThreads / 64; ++w) r = MAX ? fmaxf(r, red[w]) : r + red[w];
  return r;
}

// The RMSNorm sum of squares of a row of K <= 4096 (REG == 1): thread t
// holds chunk t's sum, every thread gets the row's sum in the shared order
// (tree8_sum over 8 consecutive chunks, then one butterfly over the 64 tree
// sums).  red holds kProThreads / 8 floats.
__device__ inline float block_tree_sum(float v, float* red) {
  static_assert(kProThreads / 8 == 64, "one tree sum per lane");
  v = tree8_sum(v);
  const int tid = threadIdx.x;
  __syncthreads();  // red[] may still be read from a previous reduction
  if ((tid & 7) == 0) red[tid >> 3] = v;
  __syncthreads();
  return wave_sum_xor(red[tid & 63]);
}

template <int REG>
__device__ inline float row_sumsq(float v, float* red) {
  if constexpr (REG == 1) return block_tree_sum(v, red);
  else return block_reduce<false>(v, red);
}

// TX: input / residual / smooth dtype (binary16 or bfloat16).  TW: RMSNorm
// weight dtype (TX or float); TY = the row's dtype after the prologue (TX,
// or float when TW is float).
// The vector body (VEC): K % 8 == 0 and every row 16-byte aligned, and the
// int8 rows 8-byte aligned (host-checked).  The x, residual, norm weight and
// smooth chunks are loaded up front with range-checked buffer loads (zeros
// past K, so the tile padding needs no branch), stores are 8 / 16 bytes
// wide, and the arithmetic is that of the generic body, in the same order:
// for binary16 rows the residual add and the norm-weight multiply are packed
// binary16 operations and the sum of squares an FMA (each the same single
// rounding as the binary32 sequence: the binary32 sum of two binary16 values
// rounds to binary16 correctly, and products of binary16 values are exact in
// binary32), and a dynamic per-row scale takes the division-free quantizer.
template <typename TX, typename TW, int REG>
__device__ inline void prologue_vec(const PrologueParams& p, float* red) {
  using TY = TW;
  using h2 = _Float16 __attribute__((ext_vector_type(2)));
  constexpr bool kHalf = std::is_same<TX, __half>::value;
  constexpr bool kW16 = sizeof(TW) == 2;
  auto as_h2 = [](uint32_t u) { return __builtin_bit_cast(h2, u); };
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int K = static_cast<int>(p.K);
  const __amdgpu_buffer_rsrc_t xd =
      raw_rsrc(static_cast<const TX*>(p.x) + row * p.ldx, K * 2);
  const __amdgpu_buffer_rsrc_t rd = raw_rsrc(
      p.residual == nullptr ? nullptr : static_cast<const TX*>(p.residual) + row * p.ld_res,
      K * 2);
  const __amdgpu_buffer_rsrc_t wd = raw_rsrc(p.norm_weight, K * static_cast<int>(sizeof(TW)));
  const __amdgpu_buffer_rsrc_t sd = raw_rsrc(p.smooth, K * 2);
  u32x4 xr[REG], rr[REG], sr[REG], wr[REG][kW16 ? 1 : 2];
#pragma unroll
  for (int c = 0; c < REG; ++c) {
    const int k0 = (tid + c * kProThreads) * 8;
    xr[c] = load16(xd, k0 * 2);
    rr[c] = load16(rd, k0 * 2);
    wr[c][0] = load16(wd, k0 * static_cast<int>(sizeof(TW)));
    if constexpr (!kW16) wr[c][1] = load16(wd, k0 * 4 + 16);
    sr[c] = load16(sd, k0 * 2);
  }

  float v[REG][8];
#pragma unroll
  for (int c = 0; c < REG; ++c) {
    const int k0 = (tid + c * kProThreads) * 8;
    if (p.residual != nullptr) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if constexpr (kHalf) {
          xr[c][q] = __builtin_bit_cast(uint32_t, as_h2(xr[c][q]) + as_h2(rr[c][q]));
        } else {
          const float lo = bits_to_f32<TX>(xr[c][q] & 0xffffu) + bits_to_f32<TX>(rr[c][q] & 0xffffu);
          const float hi = bits_to_f32<TX>(xr[c][q] >> 16) + bits_to_f32<TX>(rr[c][q] >> 16);
          xr[c][q] = pack2_bits<TX>(lo, hi);
        }
      }
      if (k0 < K)
        *reinterpret_cast<u32x4*>(static_cast<TX*>(p.residual_out) + row * p.ld_res_out + k0) =
            xr[c];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[c][2 * q] = bits_to_f32<TX>(xr[c][q] & 0xffffu);
      v[c][2 * q + 1] = bits_to_f32<TX>(xr[c][q] >> 16);
    }
  }

  if (p.norm_weight != nullptr) {
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < REG; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if constexpr (kHalf) ss = __builtin_fmaf(v[c][j], v[c][j], ss);
        else ss = __fadd_rn(ss, __fmul_rn(v[c][j], v[c][j]));
      }
    ss = row_sumsq<REG>(ss, red);
    const float var = ss / static_cast<float>(K);
    const float rs = 1.0f / sqrtf(__fadd_rn(var, p.eps));
#pragma unroll
    for (int c = 0; c < REG; ++c) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // mul_keep_sign: a -0 element stays -0 through both roundings.
        if constexpr (kHalf && kW16) {
          const h2 xn = {static_cast<_Float16>(mul_keep_sign(v[c][2 * q], rs)),
                         static_cast<_Float16>(mul_keep_sign(v[c][2 * q + 1], rs))};
          const h2 y = as_h2(wr[c][0][q]) * xn;
          v[c][2 * q] = static_cast<float>(y[0]);
          v[c][2 * q + 1] = static_cast<float>(y[1]);
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int j = 2 * q + h;
            const float xn = round_to<TX>(mul_keep_sign(v[c][j], rs));
            float w;
            if constexpr (kW16) w = bits_to_f32<TX>(h ? wr[c][0][q] >> 16 : wr[c][0][q] & 0xffffu);
            else w = __uint_as_float(wr[c][j >> 2][j & 3]);
            v[c][j] = round_to<TY>(mul_keep_sign(w, xn));
          }
        }
      }
    }
  }

  if (p.smooth != nullptr) {
#pragma unroll
    for (int c = 0; c < REG; ++c) {
      if ((tid + c * kProThreads) * 8 >= K) continue;  // zeros past K stay zeros
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t sb = j & 1 ? sr[c][j >> 1] >> 16 : sr[c][j >> 1] & 0xffffu;
        v[c][j] = round_to<TY>(v[c][j] / bits_to_f32<TX>(sb));
      }
    }
  }

  float s;
  const bool dynamic = p.static_scale == nullptr;
  if (!dynamic) {
    s = *p.static_scale;
  } else {
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < REG; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[c][j]));
    s = scale_from_absmax(block_reduce<true>(amax, red));
  }
  const float r = 1.0f / s;
  const bool fast = sizeof(TY) == 2 && __half2float(__float2half_rn(s)) == s;
  if (tid == 0 && p.scales_out != nullptr) p.scales_out[row] = s;
#pragma unroll
  for (int c = 0; c < REG; ++c) {
    const int k0 = (tid + c * kProThreads) * 8;
    u32x2 qw;
    if (sizeof(TY) == 2 && dynamic) {
      // |v / s| <= 127.07 for the row's own scale (a binary16 value).
      qw = quant8_dyn(v[c], s, r);
    } else {
      int32_t qi[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) qi[j] = fast ? quant1_h(v[c][j], s, r) : quant1(v[c][j], s);
      qw = u32x2{pack4_i8(qi[0], qi[1], qi[2], qi[3]), pack4_i8(qi[4], qi[5], qi[6], qi[7])};
    }
    if (p.KB > 0) {
      if (k0 < p.KB * kTileK) *reinterpret_cast<u32x2*>(p.q + packed_offset(row, k0, p.KB)) = qw;
    } else if (k0 < p.q_cols) {
      // K % 8 == 0 here: a chunk lies wholly before K or wholly past it.
      *reinterpret_cast<u32x2*>(p.q + row * p.ldq + k0) = k0 < K ? qw : u32x2{0u, 0u};
    }
    if (p.x_out != nullptr && k0 < K) {
      TY* xo = static_cast<TY*>(p.x_out) + row * p.ld_xout + k0;
      if constexpr (sizeof(TY) == 2) {
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = pack2_bits<TY>(v[c][2 * q], v[c][2 * q + 1]);
        *reinterpret_cast<u32x4*>(xo) = o;
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h)
          *reinterpret_cast<u32x4*>(xo + 4 * h) =
              u32x4{__float_as_uint(v[c][4 * h]), __float_as_uint(v[c][4 * h + 1]),
                    __float_as_uint(v[c][4 * h + 2]), __float_as_uint(v[c][4 * h + 3])};
      }
    }
  }
}

template <typename TX, typename TW, int REG, bool VEC>
__global__ __launch_bounds__(kProThreads) void prologue_quant_kernel(PrologueParams p) {
  using TY = TW;
  __shared__ float red[kProThreads / 8];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t K = p.K;
  if (p.KB > 0 && row >= p.M) {
    // Pad row of a packed tile: zeros.
#pragma unroll
    for (int c = 0; c < REG; ++c) {
      const int64_t k0 = (tid + static_cast<int64_t>(c) * kProThreads) * 8;
      if (k0 < p.KB * kTileK)
        *reinterpret_cast<u32x2*>(p.q + packed_offset(row, k0, p.KB)) = u32x2{0u, 0u};
    }
    return;
  }
  if constexpr (VEC) {
    prologue_vec<TX, TW, REG>(p, red);
    return;
  }
  const TX* xr = static_cast<const TX*>(p.x) + row * p.ldx;

  float v[REG][8];
#pragma unroll
  for (int c = 0; c < REG; ++c) {
    const int64_t k0 = (tid + static_cast<int64_t>(c) * kProThreads) * 8;
    const int valid = static_cast<int>(K - k0 < 8 ? (K - k0 > 0 ? K - k0 : 0) : 8);
    load8(xr + k0, v[c], aligned16(xr + k0), valid);
    if (p.residual != nullptr && valid > 0) {
      const TX* rr = static_cast<const TX*>(p.residual) + row * p.ld_res + k0;
      TX* ro = static_cast<TX*>(p.residual_out) + row * p.ld_res_out + k0;
      float rv[8];
      load8(rr, rv, aligned16(rr), valid);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j < valid) {
          const TX s = from_f32<TX>(v[c][j] + rv[j]);
          ro[j] = s;
          v[c][j] = to_f32(s);
        }
      }
    }
  }

  if (p.norm_weight != nullptr) {
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < REG; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = __fadd_rn(ss, __fmul_rn(v[c][j], v[c][j]));
    ss = row_sumsq<REG>(ss, red);
    const float var = ss / static_cast<float>(K);
    const float rr = 1.0f / sqrtf(__fadd_rn(var, p.eps));
    const TW* w = static_cast<const TW*>(p.norm_weight);
#pragma unroll
    for (int c = 0; c < REG; ++c) {
      const int64_t k0 = (tid + static_cast<int64_t>(c) * kProThreads) * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (k0 + j < K) {
          // mul_keep_sign: a -0 element stays -0 through both roundings.
          const float xn = round_to<TX>(mul_keep_sign(v[c][j], rr));
          v[c][j] = round_to<TY>(mul_keep_sign(to_f32(w[k0 + j]), xn));
        }
      }
    }
  }

  if (p.smooth != nullptr) {
    const TX* sm = static_cast<const TX*>(p.smooth);
#pragma unroll
    for (int c = 0; c < REG; ++c) {
      const int64_t k0 = (tid + static_cast<int64_t>(c) * kProThreads) * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (k0 + j < K) v[c][j] = round_to<TY>(v[c][j] / to_f32(sm[k0 + j]));
      }
    }
  }

  float s;
  if (p.static_scale != nullptr) {
    s = *p.static_scale;
  } else {
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < REG; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[c][j]));
    s = scale_from_absmax(block_reduce<true>(amax, red));
  }
  const float r = 1.0f / s;
  // The division-free quantizer needs 16-bit values and a binary16 scale.
  const bool fast = sizeof(TY) == 2 && __half2float(__float2half_rn(s)) == s;
  if (tid == 0 && p.scales_out != nullptr) p.scales_out[row] = s;

  if (p.KB > 0) {
    // Packed tiles: an aligned 8-element chunk is 8 contiguous bytes of one
    // 16-byte lane slot; columns from K to KB*64 are zeros.
#pragma unroll
    for (int c = 0; c < REG; ++c) {
      const int64_t k0 = (tid + static_cast<int64_t>(c) * kProThreads) * 8;
      if (k0 >= p.KB * kTileK) continue;
      int32_t qi[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        qi[j] = k0 + j < K ? (fast ? quant1_h(v[c][j], s, r) : quant1(v[c][j], s)) : 0;
      *reinterpret_cast<u32x2*>(p.q + packed_offset(row, k0, p.KB)) =
          u32x2{pack4_i8(qi[0], qi[1], qi[2], qi[3]), pack4_i8(qi[4], qi[5], qi[6], qi[7])};
      if (p.x_out != nullptr && k0 < K) {
        TY* xo = static_cast<TY*>(p.x_out) + row * p.ld_xout + k0;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (k0 + j < K) xo[j] = from_f32<TY>(v[c][j]);
      }
    }
    return;
  }
#pragma unroll
  for (int c = 0; c < REG; ++c) {
    const int64_t k0 = (tid + static_cast<int64_t>(c) * kProThreads) * 8;
    if (k0 >= p.q_cols) continue;
    int8_t* qr = p.q + row * p.ldq + k0;
    TY* xo = p.x_out != nullptr ? static_cast<TY*>(p.x_out) + row * p.ld_xout + k0 : nullptr;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (k0 + j < K) {
        qr[j] = static_cast<int8_t>(fast ? quant1_h(v[c][j], s, r) : quant1(v[c][j], s));
        if (xo != nullptr) xo[j] = from_f32<TY>(v[c][j]);
      } else if (k0 + j < p.q_cols) {
        qr[j] = 0;
      }
    }
  }
}

template <typename TX, typename TW, bool VEC>
hipError_t launch_reg(const PrologueParams& p, hipStream_t st) {
  const int64_t per_pass = static_cast<int64_t>(kProThreads) * 8;
  const int64_t rows = p.KB > 0 ? ceil_div(p.M, kTileRows) * kTileRows : p.M;
  const dim3 grid(static_cast<unsigned>(rows)), block(kProThreads);
  if (p.K <= per_pass)
    hipLaunchKernelGGL((prologue_quant_kernel<TX, TW, 1, VEC>), grid, block, 0, st, p);
  else if (p.K <= 2 * per_pass)
    hipLaunchKernelGGL((prologue_quant_kernel<TX, TW, 2, VEC>), grid, block, 0, st, p);
  else if (p.K <= 4 * per_pass)
    hipLaunchKernelGGL((prologue_quant_kernel<TX, TW, 4, VEC>), grid, block, 0, st, p);
  else if (p.K <= 8 * per_pass)
    hipLaunchKernelGGL((prologue_quant_kernel<TX, TW, 8, VEC>), grid, block, 0, st, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// The vector body's conditions: K % 8 == 0, every 16-bit row 16-byte
// aligned (base and leading dimension), a binary32 x_out's rows too, the
// int8 rows 8-byte aligned.
bool vec_ok(const PrologueParams& p, int w_bytes) {
  auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
  if (p.K % 8 != 0 || !a16(p.x) || p.ldx % 8 != 0) return false;
  if (p.residual != nullptr &&
      (!a16(p.residual) || p.ld_res % 8 != 0 || !a16(p.residual_out) || p.ld_res_out % 8 != 0))
    return false;
  if ((p.norm_weight != nullptr && !a16(p.norm_weight)) || (p.smooth != nullptr && !a16(p.smooth)))
    return false;
  if (p.x_out != nullptr && (!a16(p.x_out) || (p.ld_xout * w_bytes) % 16 != 0)) return false;
  return p.KB > 0 || ((reinterpret_cast<uintptr_t>(p.q) & 7u) == 0 && p.ldq % 8 == 0);
}

template <typename TX, typename TW>
hipError_t launch_tw(const PrologueParams& p, hipStream_t st) {
  return vec_ok(p, static_cast<int>(sizeof(TW))) ? launch_reg<TX, TW, true>(p, st)
                                                 : launch_reg<TX, TW, false>(p, st);
}

}  // namespace

int64_t prologue_max_k() { return static_cast<int64_t>(kProThreads) * 8 * 8; }

hipError_t launch_prologue_quant(const void* x, int x_dtype, int64_t ldx, const void* residual,
                                 int64_t ld_res, void* residual_out, int64_t ld_res_out,
                                 const void* norm_weight, int w_dtype, float eps,
                                 const void* smooth, const float* static_scale, int64_t M,
                                 int64_t K, int8_t* q, int64_t ldq, float* scales_out,
                                 void* x_out, int64_t ld_xout, hipStream_t st, bool packed,
                                 int64_t q_cols) {
  if (q_cols < K) q_cols = K;
  PrologueParams p{x,          ldx, residual, ld_res, residual_out, ld_res_out, norm_weight,
                   eps,        smooth, static_scale, M, K, q, ldq, scales_out, x_out,
                   ld_xout,    packed ? ceil_div(K, kTileK) : 0, q_cols};
  if (M == 0 || K == 0) return hipSuccess;
  // Every chunk a row writes lies inside the launch's coverage: q_cols is at
  // most round_up(K, 64), and the per-thread passes cover multiples of 4096.
  if (!packed && (q_cols > ldq || q_cols > ceil_div(K, kTileK) * kTileK)) return hipErrorInvalidValue;
  const bool w32 = norm_weight != nullptr && w_dtype == kF32;
  if (x_dtype == kF16)
    return w32 ? launch_tw<__half, float>(p, st) : launch_tw<__half, __half>(p, st);
  if (x_dtype == kBF16)
    return w32 ? launch_tw<__hip_bfloat16, float>(p, st)
               : launch_tw<__hip_bfloat16, __hip_bfloat16>(p, st);
  return hipErrorInvalidValue;
}

}  // namespace w8a8
