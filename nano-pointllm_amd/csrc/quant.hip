// Per-row symmetric int8 quantization and 16x64 tile packing.
//
// quant_rows_kernel restates, per row r of a [rows, K] matrix:
//   scale_from_absmax  (nanopointllm/compression/w8a8.py:46-50)
//   quantize_symmetric (nanopointllm/compression/w8a8.py:33-43)
// It serves both per-token activation quantization
// (dynamic_per_token_activation_qdq, w8a8.py:106-115) and per-output weight
// quantization (per_output_weight_qdq, w8a8.py:53-62): both are "one scale per
// row of a row-major matrix".
#include "w8a8_internal.h"

namespace w8a8 {

namespace {

constexpr int kQuantThreads = 256;
// Rows up to kQuantThreads * 8 * REG elements are held in registers between
// the absmax pass and the quantize pass (one global read); REG (1, 2, 4 or
// 8 chunks of 8 elements per thread) is the smallest that covers the row.
constexpr int kRegChunksMax = 8;

// Quantizes one value with the row scale s.  The division-free form needs a
// 16-bit input and a binary16-representable scale (always true for dynamic
// scales; checked per row for caller scales); otherwise divide.
template <typename TX>
__device__ inline int32_t quant_elem(float x, float s, float r, bool fast) {
  if constexpr (sizeof(TX) == 2) {
    if (fast) return quant1_h(x, s, r);
  }
  return quant1(x, s);
}

// Writes 8 quantized values of row `row` starting at column k0.
template <bool PACKED>
__device__ inline void store8(int8_t* __restrict__ q, int64_t row, int64_t k0, int64_t ldq,
                              int64_t ncols_out, int vec_out, int64_t KB, const int32_t (&qi)[8]) {
  u32x2 word = {pack4_i8(qi[0], qi[1], qi[2], qi[3]), pack4_i8(qi[4], qi[5], qi[6], qi[7])};
  if constexpr (PACKED) {
    *reinterpret_cast<u32x2*>(q + packed_offset(row, k0, KB)) = word;
  } else {
    // Row-major: columns K..ncols_out-1 are written as zeros.
    int8_t* dst = q + row * ldq + k0;
    const int nw = static_cast<int>(ncols_out - k0 < 8 ? ncols_out - k0 : 8);
    if (vec_out && nw == 8) {
      *reinterpret_cast<u32x2*>(dst) = word;
    } else {
      for (int j = 0; j < nw; ++j) dst[j] = static_cast<int8_t>(qi[j]);
    }
  }
}

// Loads the REG 8-element chunks (tid + c * NT) of a row whose elements are
// 16-byte aligned, K % 8 == 0: range-checked raw buffer loads, all issued
// before any is used (zeros past K, and for a null row).  A load under a
// branch per chunk would wait for each before issuing the next.
template <typename TX, int REG, int NT>
__device__ inline void load_row_chunks(const TX* row, int64_t K, int tid, float (&v)[REG][8]) {
  constexpr int kWords = sizeof(TX) == 4 ? 2 : 1;
  const __amdgpu_buffer_rsrc_t d = raw_rsrc(row, static_cast<int>(K * sizeof(TX)));
  u32x4 raw[REG][kWords];
#pragma unroll
  for (int c = 0; c < REG; ++c) {
    const int off = (tid + c * NT) * 8 * static_cast<int>(sizeof(TX));
#pragma unroll
    for (int w = 0; w < kWords; ++w) raw[c][w] = load16(d, off + 16 * w);
  }
#pragma unroll
  for (int c = 0; c < REG; ++c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (sizeof(TX) == 4) {
        v[c][j] = __uint_as_float(raw[c][j >> 2][j & 3]);
      } else {
        const uint32_t w = raw[c][0][j >> 1];
        v[c][j] = bits_to_f32<TX>(j & 1 ? w >> 16 : w & 0xffffu);
      }
    }
  }
}

// One workgroup per row.  The row (8 elements per thread-chunk) is read once
// into registers when it fits (REG), reduced to |x|max for a dynamic scale
// (or the caller's scale is read), then quantized and written either as a
// row-major int8 row or as the row's slots of the packed tiles.  For packed
// output the grid covers ceil(rows/16)*16 rows and every row writes all
// ceil(K/64)*64 columns, so tile padding is zero-filled.
template <typename TX, bool PACKED, bool DYNAMIC, int REG, int NT>
__global__ __launch_bounds__(NT) void quant_rows_kernel(
    const TX* __restrict__ x, int64_t ldx, int64_t rows, int64_t K, int vec_in,
    const float* __restrict__ scale_in, int64_t scale_stride, int8_t* __restrict__ q,
    int64_t ldq, int64_t ncols_out, int vec_out, int64_t KB, float* __restrict__ scales_out) {
  __shared__ float red[NT / 64];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const bool live = row < rows;
  const TX* xr = x + (live ? row : 0) * ldx;
  const int64_t nchunk_in = (K + 7) / 8;
  const int64_t nchunk_out = PACKED ? KB * 8 : (ncols_out + 7) / 8;

  float v[REG > 0 ? REG : 1][8];
  if constexpr (REG > 0) {
    if (vec_in) {
      load_row_chunks<TX, REG, NT>(live ? xr : nullptr, K, tid, v);
    } else {
#pragma unroll
      for (int c = 0; c < REG; ++c) {
        const int64_t k0 = (tid + static_cast<int64_t>(c) * NT) * 8;
        const int64_t rem = K - k0;
        if (live && rem > 0) {
          load8(xr + k0, v[c], false, static_cast<int>(rem < 8 ? rem : 8));
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) v[c][j] = 0.0f;
        }
      }
    }
  }

  float s = 1.0f;
  if constexpr (DYNAMIC) {
    float amax = 0.0f;
    if constexpr (REG > 0) {
#pragma unroll
      for (int c = 0; c < REG; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[c][j]));
    } else if (live) {
      for (int64_t c = tid; c < nchunk_in; c += NT) {
        float t[8];
        const int64_t k0 = c * 8;
        load8(xr + k0, t, vec_in != 0, static_cast<int>(K - k0 < 8 ? K - k0 : 8));
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(t[j]));
      }
    }
    amax = wave_max_abs(amax);
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) amax = fmaxf(amax, red[w]);
    s = scale_from_absmax(amax);
  } else {
    if (live) s = scale_in[row * scale_stride];
  }
  const float r = 1.0f / s;
  const bool fast = DYNAMIC || __half2float(__float2half_rn(s)) == s;
  if (live && tid == 0 && scales_out != nullptr) scales_out[row] = s;

  if constexpr (REG > 0) {
#pragma unroll
    for (int c = 0; c < REG; ++c) {
      const int64_t chunk = tid + static_cast<int64_t>(c) * NT;
      if (chunk < nchunk_out) {
        const int64_t k0 = chunk * 8;
        int32_t qi[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) qi[j] = quant_elem<TX>(v[c][j], s, r, fast);
        store8<PACKED>(q, row, k0, ldq, ncols_out, vec_out, KB, qi);
      }
    }
  } else {
    for (int64_t c = tid; c < nchunk_out; c += NT) {
      const int64_t k0 = c * 8;
      const int64_t rem = K - k0;
      const int valid = live ? static_cast<int>(rem <= 0 ? 0 : (rem < 8 ? rem : 8)) : 0;
      float t[8];
      if (valid > 0) {
        load8(xr + k0, t, vec_in != 0, valid);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j] = 0.0f;
      }
      int32_t qi[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) qi[j] = (j < valid) ? quant_elem<TX>(t[j], s, r, fast) : 0;
      store8<PACKED>(q, row, k0, ldq, ncols_out, vec_out, KB, qi);
    }
  }
}

// Second phase of the two-phase per-token requantization (one workgroup per
// row): the producing epilogue left the row's |x|max split over nparts
// partial maxima, parts[row * nparts + i]; their max gives the binary16
// scale (scale_from_absmax, w8a8.py:46-50) without a reduction over x, and
// the row is quantized (quantize_symmetric, w8a8.py:33-43) into row-major q.
// The row's chunks (REG per thread, or a second pass when REG is 0) are
// requested before the partials, so both reads are in flight together.
template <typename TX, int REG, int NT>
__global__ __launch_bounds__(NT) void quant_rows_parts_kernel(
    const TX* __restrict__ x, int64_t ldx, int64_t K, int vec_in,
    const float* __restrict__ parts, int64_t nparts, int8_t* __restrict__ q, int64_t ldq,
    int vec_out, float* __restrict__ scales_out) {
  __shared__ float red[NT / 64];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const TX* xr = x + row * ldx;
  const int64_t nchunk = (K + 7) / 8;
  float v[REG > 0 ? REG : 1][8];
  if constexpr (REG > 0) {
    if (vec_in) {
      load_row_chunks<TX, REG, NT>(xr, K, tid, v);
    } else {
#pragma unroll
      for (int c = 0; c < REG; ++c) {
        const int64_t k0 = (tid + static_cast<int64_t>(c) * NT) * 8;
        const int64_t rem = K - k0;
        if (rem > 0) {
          load8(xr + k0, v[c], false, static_cast<int>(rem < 8 ? rem : 8));
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) v[c][j] = 0.0f;
        }
      }
    }
  }
  const float* pr = parts + row * nparts;
  float amax = 0.0f;
  for (int64_t i = tid; i < nparts; i += NT) amax = fmaxf(amax, pr[i]);
  amax = wave_max_abs(amax);
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) amax = fmaxf(amax, red[w]);
  const float s = scale_from_absmax(amax);
  const float r = 1.0f / s;
  if (tid == 0) scales_out[row] = s;
  if constexpr (REG > 0) {
#pragma unroll
    for (int c = 0; c < REG; ++c) {
      const int64_t chunk = tid + static_cast<int64_t>(c) * NT;
      if (chunk < nchunk) {
        const int64_t k0 = chunk * 8;
        const int valid = static_cast<int>(K - k0 < 8 ? K - k0 : 8);
        int32_t qi[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) qi[j] = (j < valid) ? quant_elem<TX>(v[c][j], s, r, true) : 0;
        store8<false>(q, row, k0, ldq, K, vec_out, 0, qi);
      }
    }
  } else {
    for (int64_t c = tid; c < nchunk; c += NT) {
      const int64_t k0 = c * 8;
      const int valid = static_cast<int>(K - k0 < 8 ? K - k0 : 8);
      float t[8];
      load8(xr + k0, t, vec_in != 0, valid);
      int32_t qi[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) qi[j] = (j < valid) ? quant_elem<TX>(t[j], s, r, true) : 0;
      store8<false>(q, row, k0, ldq, K, vec_out, 0, qi);
    }
  }
}

// Packs a row-major int8 [rows, K] matrix into 16x64 tiles.  One thread per
// 16-byte lane slot.  layout 1 maps packed row p to source row p/2 (p even)
// or rows/2 + p/2 (p odd): the gate/up "interleave" order of
// _pack_gateup_tensors (llama/lightweight_runner.py:81-92) applied to a
// split-packed [gate; up] source.
__global__ __launch_bounds__(256) void pack_rows_kernel(const int8_t* __restrict__ src,
                                                         int64_t rows, int64_t K, int64_t ld,
                                                         int layout, int vec, int64_t KB,
                                                         int64_t nslots,
                                                         int8_t* __restrict__ dst) {
  const int64_t slot = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (slot >= nslots) return;
  const int64_t tile = slot >> 6;
  const int lane = static_cast<int>(slot & 63);
  const int64_t rb = tile / KB;
  const int64_t kb = tile - rb * KB;
  const int64_t prow = rb * 16 + (lane & 15);
  const int64_t k0 = kb * 64 + (lane >> 4) * 16;
  u32x4 out = {0u, 0u, 0u, 0u};
  if (prow < rows && k0 < K) {
    int64_t srow = prow;
    if (layout == 1) srow = (prow & 1) ? (rows / 2 + (prow >> 1)) : (prow >> 1);
    const int8_t* p = src + srow * ld + k0;
    const int64_t valid = K - k0 < 16 ? K - k0 : 16;
    if (vec && valid == 16) {
      out = *reinterpret_cast<const u32x4*>(p);
    } else {
      uint8_t b[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) b[j] = (j < valid) ? static_cast<uint8_t>(p[j]) : 0u;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        out[j] = static_cast<uint32_t>(b[4 * j]) | (static_cast<uint32_t>(b[4 * j + 1]) << 8) |
                 (static_cast<uint32_t>(b[4 * j + 2]) << 16) |
                 (static_cast<uint32_t>(b[4 * j + 3]) << 24);
      }
    }
  }
  reinterpret_cast<u32x4*>(dst)[slot] = out;
}

// Row-major int8 copy [rows, K] -> [rows, ldd] with zero columns K..ldd-1.
// One thread per 16-byte destination chunk.
__global__ __launch_bounds__(256) void pad_rows_kernel(const int8_t* __restrict__ src,
                                                        int64_t rows, int64_t K, int64_t ld,
                                                        int8_t* __restrict__ dst, int64_t ldd) {
  const int64_t chunks_per_row = ldd / 16;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= rows * chunks_per_row) return;
  const int64_t r = idx / chunks_per_row;
  const int64_t k0 = (idx - r * chunks_per_row) * 16;
  uint8_t b[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) b[j] = (k0 + j < K) ? static_cast<uint8_t>(src[r * ld + k0 + j]) : 0u;
  u32x4 out;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    out[j] = static_cast<uint32_t>(b[4 * j]) | (static_cast<uint32_t>(b[4 * j + 1]) << 8) |
             (static_cast<uint32_t>(b[4 * j + 2]) << 16) | (static_cast<uint32_t>(b[4 * j + 3]) << 24);
  }
  *reinterpret_cast<u32x4*>(dst + r * ldd + k0) = out;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

template <typename TX, bool PACKED, bool DYN, int REG, int NT>
void quant_launch_reg(dim3 g, hipStream_t st, const TX* x, int64_t ldx, int64_t rows,
                      int64_t K, int vec_in, const float* scale_in, int64_t scale_stride,
                      int8_t* q, int64_t ldq, int64_t ncols_out, int vec_out, int64_t KB,
                      float* scales_out) {
  hipLaunchKernelGGL((quant_rows_kernel<TX, PACKED, DYN, REG, NT>), g, dim3(NT), 0, st, x, ldx,
                     rows, K, vec_in, scale_in, scale_stride, q, ldq, ncols_out, vec_out, KB,
                     scales_out);
}

template <typename TX, bool PACKED, bool DYN, int NT>
void quant_launch_nt(dim3 g, hipStream_t st, int64_t chunks, const TX* x, int64_t ldx,
                     int64_t rows, int64_t K, int vec_in, const float* scale_in,
                     int64_t scale_stride, int8_t* q, int64_t ldq, int64_t ncols_out,
                     int vec_out, int64_t KB, float* scales_out) {
  const int64_t per = ceil_div(chunks, NT);
#define W8A8_QUANT_REG(R)                                                                     \
  quant_launch_reg<TX, PACKED, DYN, R, NT>(g, st, x, ldx, rows, K, vec_in, scale_in,          \
                                           scale_stride, q, ldq, ncols_out, vec_out, KB,      \
                                           scales_out)
  if (per <= 1)
    W8A8_QUANT_REG(1);
  else if (per <= 2)
    W8A8_QUANT_REG(2);
  else if (per <= 4)
    W8A8_QUANT_REG(4);
  else if (per <= kRegChunksMax)
    W8A8_QUANT_REG(kRegChunksMax);
  else
    W8A8_QUANT_REG(0);
#undef W8A8_QUANT_REG
}

// Few rows (decode) leave most of the GPU idle, so each row's latency is what
// counts: wide rows then get up to 1024 threads (16 wavefronts share each
// CU's SIMDs and hide each other's load latency).  Many rows keep 256
// threads per row.
template <typename TX, bool PACKED, bool DYN>
void quant_launch(dim3 g, hipStream_t st, int64_t chunks, const TX* x, int64_t ldx,
                  int64_t rows, int64_t K, int vec_in, const float* scale_in,
                  int64_t scale_stride, int8_t* q, int64_t ldq, int64_t ncols_out, int vec_out,
                  int64_t KB, float* scales_out) {
  if constexpr (!PACKED) {
    if (rows <= kGemvMaxRows && chunks > kQuantThreads) {
      if (chunks > 2 * kQuantThreads)
        return quant_launch_nt<TX, PACKED, DYN, 4 * kQuantThreads>(
            g, st, chunks, x, ldx, rows, K, vec_in, scale_in, scale_stride, q, ldq, ncols_out,
            vec_out, KB, scales_out);
      return quant_launch_nt<TX, PACKED, DYN, 2 * kQuantThreads>(
          g, st, chunks, x, ldx, rows, K, vec_in, scale_in, scale_stride, q, ldq, ncols_out,
          vec_out, KB, scales_out);
    }
  }
  quant_launch_nt<TX, PACKED, DYN, kQuantThreads>(g, st, chunks, x, ldx, rows, K, vec_in,
                                                  scale_in, scale_stride, q, ldq, ncols_out,
                                                  vec_out, KB, scales_out);
}

template <typename TX>
hipError_t quant_dispatch(const TX* x, int64_t ldx, int64_t rows, int64_t K,
                          const float* scale_in, int64_t scale_stride, int8_t* q, int64_t ldq,
                          int64_t ncols_out, bool packed, float* scales_out, hipStream_t st) {
  const int vec_in = aligned16(x) && (ldx % 8 == 0) && (K % 8 == 0);
  const int vec_out = aligned8(q) && (ldq % 8 == 0);
  const int64_t KB = ceil_div(K, kTileK);
  const int64_t grid = packed ? ceil_div(rows, kTileRows) * kTileRows : rows;
  if (grid == 0) return hipSuccess;
  const int64_t chunks = packed ? KB * 8 : ceil_div(ncols_out > K ? ncols_out : K, 8);
  const bool dyn = scale_in == nullptr;
  dim3 g(static_cast<unsigned>(grid));
  if (packed) {
    if (dyn)
      quant_launch<TX, true, true>(g, st, chunks, x, ldx, rows, K, vec_in, scale_in,
                                   scale_stride, q, ldq, ncols_out, vec_out, KB, scales_out);
    else
      quant_launch<TX, true, false>(g, st, chunks, x, ldx, rows, K, vec_in, scale_in,
                                    scale_stride, q, ldq, ncols_out, vec_out, KB, scales_out);
  } else {
    if (dyn)
      quant_launch<TX, false, true>(g, st, chunks, x, ldx, rows, K, vec_in, scale_in,
                                    scale_stride, q, ldq, ncols_out, vec_out, KB, scales_out);
    else
      quant_launch<TX, false, false>(g, st, chunks, x, ldx, rows, K, vec_in, scale_in,
                                     scale_stride, q, ldq, ncols_out, vec_out, KB, scales_out);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_quant_rows(const void* x, int x_dtype, int64_t ldx, int64_t rows, int64_t K,
                             const float* scale_in, int64_t scale_stride, int8_t* q,
                             int64_t ldq, int64_t ncols_out, bool packed, float* scales_out,
                             hipStream_t st) {
  switch (x_dtype) {
    case kF32:
      return quant_dispatch(static_cast<const float*>(x), ldx, rows, K, scale_in, scale_stride,
                            q, ldq, ncols_out, packed, scales_out, st);
    case kF16:
      return quant_dispatch(static_cast<const __half*>(x), ldx, rows, K, scale_in, scale_stride,
                            q, ldq, ncols_out, packed, scales_out, st);
    case kBF16:
      return quant_dispatch(static_cast<const __hip_bfloat16*>(x), ldx, rows, K, scale_in,
                            scale_stride, q, ldq, ncols_out, packed, scales_out, st);
    default:
      return hipErrorInvalidValue;
  }
}

template <typename TX, int NT>
void quant_parts_launch(dim3 g, hipStream_t st, int64_t chunks, const TX* x, int64_t ldx,
                        int64_t K, int vec_in, const float* parts, int64_t nparts, int8_t* q,
                        int64_t ldq, int vec_out, float* scales) {
  const int64_t per = ceil_div(chunks, NT);
#define W8A8_PARTS_REG(R)                                                                     \
  hipLaunchKernelGGL((quant_rows_parts_kernel<TX, R, NT>), g, dim3(NT), 0, st, x, ldx, K,       \
                     vec_in, parts, nparts, q, ldq, vec_out, scales)
  if (per <= 1)
    W8A8_PARTS_REG(1);
  else if (per <= 2)
    W8A8_PARTS_REG(2);
  else if (per <= 4)
    W8A8_PARTS_REG(4);
  else if (per <= kRegChunksMax)
    W8A8_PARTS_REG(kRegChunksMax);
  else
    W8A8_PARTS_REG(0);
#undef W8A8_PARTS_REG
}

template <typename TX>
hipError_t quant_parts_dispatch(const TX* x, int64_t ldx, int64_t rows, int64_t K,
                                const float* parts, int64_t nparts, int8_t* q, int64_t ldq,
                                float* scales, hipStream_t st) {
  const int vec_in = aligned16(x) && (ldx % 8 == 0) && (K % 8 == 0);
  const int vec_out = aligned8(q) && (ldq % 8 == 0);
  const int64_t chunks = ceil_div(K, 8);
  const dim3 g(static_cast<unsigned>(rows));
  // Few rows (decode) get wide workgroups, as in quant_launch.
  if (rows <= kGemvMaxRows && chunks > 2 * kQuantThreads)
    quant_parts_launch<TX, 4 * kQuantThreads>(g, st, chunks, x, ldx, K, vec_in, parts, nparts, q,
                                              ldq, vec_out, scales);
  else if (rows <= kGemvMaxRows && chunks > kQuantThreads)
    quant_parts_launch<TX, 2 * kQuantThreads>(g, st, chunks, x, ldx, K, vec_in, parts, nparts, q,
                                              ldq, vec_out, scales);
  else
    quant_parts_launch<TX, kQuantThreads>(g, st, chunks, x, ldx, K, vec_in, parts, nparts, q,
                                          ldq, vec_out, scales);
  return hipGetLastError();
}

hipError_t launch_quant_rows_parts(const void* x, int x_dtype, int64_t ldx, int64_t rows,
                                   int64_t K, const float* parts, int64_t nparts, int8_t* q,
                                   int64_t ldq, float* scales_out, hipStream_t st) {
  if (rows == 0) return hipSuccess;
  switch (x_dtype) {
    case kF32:
      return quant_parts_dispatch(static_cast<const float*>(x), ldx, rows, K, parts, nparts, q,
                                  ldq, scales_out, st);
    case kF16:
      return quant_parts_dispatch(static_cast<const __half*>(x), ldx, rows, K, parts, nparts, q,
                                  ldq, scales_out, st);
    case kBF16:
      return quant_parts_dispatch(static_cast<const __hip_bfloat16*>(x), ldx, rows, K, parts,
                                  nparts, q, ldq, scales_out, st);
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_pack_rows(const int8_t* src, int64_t rows, int64_t K, int64_t ld, int layout,
                            int8_t* dst, hipStream_t st) {
  const int64_t KB = ceil_div(K, kTileK);
  const int64_t nslots = ceil_div(rows, kTileRows) * KB * kTileVec;
  if (nslots == 0) return hipSuccess;
  const int vec = aligned16(src) && (ld % 16 == 0);
  const int64_t blocks = ceil_div(nslots, 256);
  hipLaunchKernelGGL(pack_rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                     src, rows, K, ld, layout, vec, KB, nslots, dst);
  return hipGetLastError();
}

hipError_t launch_pad_rows(const int8_t* src, int64_t rows, int64_t K, int64_t ld, int8_t* dst,
                           int64_t ldd, hipStream_t st) {
  const int64_t total = rows * (ldd / 16);
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(pad_rows_kernel, dim3(static_cast<unsigned>(ceil_div(total, 256))), dim3(256),
                     0, st, src, rows, K, ld, dst, ldd);
  return hipGetLastError();
}

}  // namespace w8a8
