// Decode W8A8 linear with the per-token quantization fused in (M <= 8).
//
// One launch replaces quantize_symmetric(x, scale_from_absmax(|x|max)) +
// int8 GEMV + dequant epilogue (nanopointllm/compression/w8a8.py:46-50,
// 33-43, 118-139) for the decode call sites (llama/paged_attention.py:97-124,
// llama/lightweight_runner.py:38-54, 329-379).
//
// Design: a persistent grid of one 16-wavefront workgroup per CU.
//   1. Each wavefront issues its first weight loads (they do not depend on x).
//   2. While they are in flight the workgroup quantizes all M rows of x into
//      LDS (row absmax on the raw 16-bit patterns, binary16 scale, the
//      division-free exact quantizer), laid out as half MFMA A fragments:
//      8 rows x 64 K per k-block, so lane (i, g) reads row i, k 16g..16g+15
//      with one conflict-free ds_read_b128.
//   3. Workgroup b then streams 16-output weight blocks b, b+G, b+2G, ...; its
//      16 wavefronts split K, each keeping two chunks of CH 1 KiB fragments in
//      flight across block boundaries.  Per block, the per-wave 16x16 int32
//      partials go through one of two LDS buffers, one barrier, and the fused
//      epilogue (dequant / SiLU*mul / int8 requant) of the GEMV.
// Quantizing x once per CU costs M*K*~10 VALU ops per CU; for decode shapes
// that hides behind the weight loads already in flight, and it saves the
// separate quantization launch and its round trip through memory.
#include "w8a8_internal.h"

namespace w8a8 {

namespace {

constexpr int kFusedWaves = 16;
constexpr int kFusedThreads = kFusedWaves * 64;
constexpr int kFusedCH = 4;
constexpr int kFusedMaxRows = 8;
constexpr int kFusedMaxKB = 192;  // K <= 12288
// Max 16-byte x chunks a thread holds during quantization (1 row: 12288/8/1024).
constexpr int kFusedMaxChunks = 12;

struct FusedParams {
  const void* x;
  int64_t ldx;
  const i32x4* w;
  const float* sw;
  const float* bias;
  void* y;
  int64_t ldy;
  float* sx_out;
  float out_scale;
  int M;
  int N;
  int K;
  int KB;
  int NB;
  int G;
};

__device__ inline i32x4 mfma_16x16x64(i32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// |x| of a packed pair of 16-bit floats, as unsigned integers.  For
// non-negative binary16 / bfloat16 values the bit patterns order like the
// values, so the integer max is the absmax.
__device__ inline uint32_t abs_lo(uint32_t v) { return v & 0x7fffu; }
__device__ inline uint32_t abs_hi(uint32_t v) { return (v >> 16) & 0x7fffu; }

template <typename TX>
__device__ inline float bits_to_f32(uint32_t b16) {
  return to_f32(__builtin_bit_cast(TX, static_cast<uint16_t>(b16)));
}

template <int EPI, typename TX, typename TY, typename TH>
__global__ __launch_bounds__(kFusedThreads) void gemv_fused_kernel(FusedParams p) {
  // A fragments: [kb][g][row < 8][16 bytes]
  __shared__ __attribute__((aligned(16))) int8_t a_lds[kFusedMaxKB * 512];
  __shared__ int32_t red[2][kFusedWaves][256];
  __shared__ uint32_t amax_w[kFusedWaves];
  __shared__ float row_s[kFusedMaxRows];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int KB = p.KB;
  const int M = p.M;

  // This wave's k-block range; all waves use the same trip count kbw.
  const int kbw = (KB + kFusedWaves - 1) / kFusedWaves;
  const int kb0 = min(wave * kbw, KB);
  const int kb1 = min(kb0 + kbw, KB);
  const bool has_range = kb0 < kb1;
  const int nch = (kbw + kFusedCH - 1) / kFusedCH;
  const int n_mine = (p.NB - static_cast<int>(blockIdx.x) + p.G - 1) / p.G;
  const int total = n_mine * nch;

  auto load = [&](i32x4(&buf)[kFusedCH], int j, int c) {
    const int64_t nb = static_cast<int64_t>(blockIdx.x) + static_cast<int64_t>(j) * p.G;
    const i32x4* base = p.w + nb * KB * 64 + lane;
#pragma unroll
    for (int i = 0; i < kFusedCH; ++i) {
      int kb = kb0 + c * kFusedCH + i;
      kb = kb < kb1 ? kb : kb1 - 1;
      buf[i] = __builtin_nontemporal_load(base + static_cast<int64_t>(kb) * 64);
    }
  };

  i32x4 cur[kFusedCH], nxt[kFusedCH];
  if (has_range && total > 0) load(cur, 0, 0);

  // ---------------------------------------------------------- quantize x
  // Rows are spread over power-of-two groups of TPR >= 128 threads.
  const int mpad = M <= 1 ? 1 : (M <= 2 ? 2 : (M <= 4 ? 4 : 8));
  const int tpr = kFusedThreads / mpad;
  const int row = tid / tpr;
  const int j0 = tid - row * tpr;
  const int nchunk = KB * 8;  // 8-element chunks per padded row
  const bool row_live = row < M;
  const uint16_t* xr =
      static_cast<const uint16_t*>(p.x) + static_cast<int64_t>(row_live ? row : 0) * p.ldx;
  u32x4 raw[kFusedMaxChunks];
  uint32_t am = 0;
#pragma unroll
  for (int i = 0; i < kFusedMaxChunks; ++i) {
    const int c = j0 + i * tpr;
    if (row_live && c < nchunk && c * 8 < p.K) {
      raw[i] = *reinterpret_cast<const u32x4*>(xr + static_cast<int64_t>(c) * 8);
    } else {
      raw[i] = u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) am = max(am, max(abs_lo(raw[i][q]), abs_hi(raw[i][q])));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) am = max(am, static_cast<uint32_t>(__shfl_xor(static_cast<int>(am), off)));
  if (lane == 0) amax_w[wave] = am;
  __syncthreads();
  if (tid < M) {
    const int wpr = tpr / 64;  // waves per row
    uint32_t m = 0;
    for (int v = 0; v < wpr; ++v) m = max(m, amax_w[tid * wpr + v]);
    const float s = scale_from_absmax(bits_to_f32<TX>(m));
    row_s[tid] = s;
    if (blockIdx.x == 0 && p.sx_out != nullptr) p.sx_out[tid] = s;
  }
  __syncthreads();
  if (row_live) {
    const float s = row_s[row];
    const float r = 1.0f / s;
#pragma unroll
    for (int i = 0; i < kFusedMaxChunks; ++i) {
      const int c = j0 + i * tpr;
      if (c < nchunk) {
        int32_t qi[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          qi[2 * q] = quant1_h(bits_to_f32<TX>(raw[i][q] & 0xffffu), s, r);
          qi[2 * q + 1] = quant1_h(bits_to_f32<TX>(raw[i][q] >> 16), s, r);
        }
        const int k = c * 8;
        const int off = (((k >> 6) * 4 + ((k & 63) >> 4)) * 8 + row) * 16 + (k & 15);
        *reinterpret_cast<u32x2*>(a_lds + off) =
            u32x2{pack4_i8(qi[0], qi[1], qi[2], qi[3]), pack4_i8(qi[4], qi[5], qi[6], qi[7])};
      }
    }
  }
  __syncthreads();

  // ------------------------------------------------------- stream weights
  const bool a_live = li < M;
  const int a_off = (lg * 8 + li) * 16;
  i32x4 acc = i32x4{0, 0, 0, 0};
  int j = 0, c = 0;
  for (int step = 0; step < total; ++step) {
    int jn = j, cn = c + 1;
    if (cn == nch) {
      cn = 0;
      jn = j + 1;
    }
    if (has_range && step + 1 < total) load(nxt, jn, cn);
    if (has_range) {
#pragma unroll
      for (int i = 0; i < kFusedCH; ++i) {
        const int kb = kb0 + c * kFusedCH + i;
        if (kb < kb1) {
          const i32x4 a = a_live ? *reinterpret_cast<const i32x4*>(a_lds + kb * 512 + a_off)
                                 : i32x4{0, 0, 0, 0};
          acc = mfma_16x16x64(a, cur[i], acc);
        }
      }
    }
    if (cn == 0) {
      // Block j done: reduce the wave partials and run the epilogue.
      const int par = j & 1;
#pragma unroll
      for (int r = 0; r < 4; ++r) red[par][wave][(4 * lg + r) * 16 + li] = acc[r];
      acc = i32x4{0, 0, 0, 0};
      __syncthreads();
      const int64_t nb = static_cast<int64_t>(blockIdx.x) + static_cast<int64_t>(j) * p.G;
      if constexpr (EPI == kEpiI32 || EPI == kEpiDequant) {
        if (tid < 256) {
          const int m = tid >> 4;
          const int64_t n = nb * 16 + (tid & 15);
          if (m < M && n < p.N) {
            int32_t s = 0;
#pragma unroll
            for (int w = 0; w < kFusedWaves; ++w) s += red[par][w][tid];
            TY* y = static_cast<TY*>(p.y) + static_cast<int64_t>(m) * p.ldy + n;
            if constexpr (EPI == kEpiI32) {
              *y = s;
            } else {
              *y = from_f32<TY>(dequant1(s, row_s[m], p.sw[n], p.bias, n));
            }
          }
        }
      } else {
        if (tid < 128) {
          const int m = tid >> 3;
          const int cc = tid & 7;
          const int64_t n_out = nb * 8 + cc;
          if (m < M && n_out < p.N / 2) {
            const int base = m * 16 + 2 * cc;
            int32_t sg = 0, su = 0;
#pragma unroll
            for (int w = 0; w < kFusedWaves; ++w) {
              sg += red[par][w][base];
              su += red[par][w][base + 1];
            }
            const int64_t ng = nb * 16 + 2 * cc;
            const float sxm = row_s[m];
            const float g = to_f32(from_f32<TH>(dequant1(sg, sxm, p.sw[ng], p.bias, ng)));
            const float u = to_f32(from_f32<TH>(dequant1(su, sxm, p.sw[ng + 1], p.bias, ng + 1)));
            const TH h = from_f32<TH>(silu_mul<TH>(g, u));
            TY* y = static_cast<TY*>(p.y) + static_cast<int64_t>(m) * p.ldy + n_out;
            if constexpr (EPI == kEpiSilu) {
              *y = h;
            } else {
              *y = static_cast<int8_t>(quant1(to_f32(h), p.out_scale));
            }
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kFusedCH; ++i) cur[i] = nxt[i];
    j = jn;
    c = cn;
  }
}

int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <int EPI, typename TX, typename TY, typename TH>
hipError_t launch_f(const FusedParams& p, hipStream_t st) {
  hipLaunchKernelGGL((gemv_fused_kernel<EPI, TX, TY, TH>), dim3(p.G), dim3(kFusedThreads), 0, st,
                     p);
  return hipGetLastError();
}

template <typename TX>
hipError_t dispatch_f(const FusedParams& p, int epi, int y_dtype, int h_dtype, hipStream_t st) {
  switch (epi) {
    case kEpiI32:
      return launch_f<kEpiI32, TX, int32_t, float>(p, st);
    case kEpiDequant:
      if (y_dtype == kF16) return launch_f<kEpiDequant, TX, __half, float>(p, st);
      if (y_dtype == kBF16) return launch_f<kEpiDequant, TX, __hip_bfloat16, float>(p, st);
      if (y_dtype == kF32) return launch_f<kEpiDequant, TX, float, float>(p, st);
      return hipErrorInvalidValue;
    case kEpiSilu:
      if (y_dtype == kF16) return launch_f<kEpiSilu, TX, __half, __half>(p, st);
      if (y_dtype == kBF16) return launch_f<kEpiSilu, TX, __hip_bfloat16, __hip_bfloat16>(p, st);
      return hipErrorInvalidValue;
    case kEpiSiluQ8:
      if (h_dtype == kF16) return launch_f<kEpiSiluQ8, TX, int8_t, __half>(p, st);
      if (h_dtype == kBF16) return launch_f<kEpiSiluQ8, TX, int8_t, __hip_bfloat16>(p, st);
      return hipErrorInvalidValue;
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace

// Used for single-row decode only: measured on MI355X, quantizing x once per
// CU in this persistent kernel beats the separate quantization launch at
// M = 1, but its per-CU quantization work (M*K elements) and per-block
// barriers make it slower than quantize + gemv_kernel from M = 4 up.
bool fused_gemv_supported(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K) {
  return (x_dtype == kF16 || x_dtype == kBF16) && M == 1 && K >= 8 &&
         K % 8 == 0 && ceil_div(K, kTileK) <= kFusedMaxKB && ldx % 8 == 0 &&
         (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

hipError_t launch_gemv_fused(const void* x, int x_dtype, int64_t ldx, const LinearOperands& op,
                             float* sx_out, hipStream_t st) {
  FusedParams p;
  p.x = x;
  p.ldx = ldx;
  p.w = reinterpret_cast<const i32x4*>(op.w);
  p.sw = op.sw;
  p.bias = op.bias;
  p.y = op.y;
  p.ldy = op.ldy;
  p.sx_out = sx_out;
  p.out_scale = op.out_scale;
  p.M = static_cast<int>(op.M);
  p.N = static_cast<int>(op.N);
  p.K = static_cast<int>(op.K);
  p.KB = static_cast<int>(ceil_div(op.K, kTileK));
  p.NB = static_cast<int>(ceil_div(op.N, kTileRows));
  p.G = static_cast<int>(p.NB < cu_count() ? p.NB : cu_count());
  if (p.NB == 0 || p.M == 0) return hipSuccess;
  if (x_dtype == kF16) return dispatch_f<__half>(p, op.epi, op.y_dtype, op.h_dtype, st);
  if (x_dtype == kBF16) return dispatch_f<__hip_bfloat16>(p, op.epi, op.y_dtype, op.h_dtype, st);
  return hipErrorInvalidValue;
}

}  // namespace w8a8
