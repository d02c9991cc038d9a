// Prefill-regime W8A8 GEMM (M > 64): y = epi(xq @ wq^T) with int8 MFMA.
//
// Replaces the prefill/mixed projections (llama/paged_attention.py:1349-1352,
// 1488; llama/lightweight_runner.py:320-404) for the int8 contract of
// integer_linear_per_output_reference (nanopointllm/compression/w8a8.py:118-139).
//
// Design (MFMA-bound): 256-thread workgroups own a 128 x 128 output tile; the
// four wavefronts form a 2 x 2 grid of 64 x 64 sub-tiles (4 x 4
// v_mfma_i32_16x16x64_i8 fragments, 64 accumulator VGPRs each).  Both operands
// are in the packed 16x64 tile layout, so one k-step (64) of the workgroup
// tile is 16 fragments of 1 KiB: each wavefront copies four of them with
// coalesced global_load_dwordx4 into registers one step ahead, and the LDS
// stage is double-buffered so one barrier per k-step suffices.  Fragments are
// read back with conflict-free ds_read_b128 (lane l reads bytes 16l..16l+15).
// Workgroups are mapped XCD-major: consecutive tiles of the same weight
// column block land on the same XCD and share its L2.
#include "w8a8_internal.h"

namespace w8a8 {

namespace {

struct GemmParams {
  const i32x4* a;
  const float* sx;
  const i32x4* w;
  const float* sw;
  const float* bias;
  void* y;
  int64_t ldy;
  float out_scale;
  int M;
  int N;
  int MB;
  int NB;
  int KB;
  int tiles_m;
  int tiles;
  int per_xcd;
};

constexpr int kXcds = 8;
constexpr int kBMF = 8;  // 16-row fragments per workgroup tile (128 rows)
constexpr int kBNF = 8;  // 16-col fragments per workgroup tile (128 cols)

__device__ inline i32x4 mfma_16x16x64(i32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

template <int EPI, typename TY, typename TH>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmParams p) {
  __shared__ i32x4 lds[2][kBMF + kBNF][64];

  // XCD-major tile mapping: workgroup b runs on XCD b % 8.
  const int b = blockIdx.x;
  const int tile = (b % kXcds) * p.per_xcd + b / kXcds;
  if (tile >= p.tiles) return;
  const int tm = tile % p.tiles_m;
  const int tn = tile / p.tiles_m;
  const int mb0 = tm * kBMF;
  const int nb0 = tn * kBNF;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int KB = p.KB;

  // Fragment f = 4q + wave of each k-step: f < 8 are activation blocks
  // mb0 + f, f >= 8 weight blocks nb0 + f - 8.
  const i32x4* src[4];
  bool ok[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int f = 4 * q + wave;
    if (f < kBMF) {
      ok[q] = mb0 + f < p.MB;
      src[q] = p.a + static_cast<int64_t>(ok[q] ? mb0 + f : 0) * KB * 64 + lane;
    } else {
      ok[q] = nb0 + f - kBMF < p.NB;
      src[q] = p.w + static_cast<int64_t>(ok[q] ? nb0 + f - kBMF : 0) * KB * 64 + lane;
    }
  }

  i32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

  i32x4 st[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) st[q] = (ok[q] && KB > 0) ? src[q][0] : i32x4{0, 0, 0, 0};
#pragma unroll
  for (int q = 0; q < 4; ++q) lds[0][4 * q + wave][lane] = st[q];
  __syncthreads();

  for (int kb = 0; kb < KB; ++kb) {
    const int cur = kb & 1;
    const bool more = kb + 1 < KB;
    if (more) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        st[q] = ok[q] ? src[q][static_cast<int64_t>(kb + 1) * 64] : i32x4{0, 0, 0, 0};
    }
    i32x4 af[4], bf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = lds[cur][wm * 4 + i][lane];
#pragma unroll
    for (int j = 0; j < 4; ++j) bf[j] = lds[cur][kBMF + wn * 4 + j][lane];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma_16x16x64(af[i], bf[j], acc[i][j]);
    if (more) {
#pragma unroll
      for (int q = 0; q < 4; ++q) lds[cur ^ 1][4 * q + wave][lane] = st[q];
    }
    __syncthreads();
  }

  // Epilogue.  Fragment (i, j), register r: row (mb0 + 4wm + i)*16 + 4lg + r,
  // column (nb0 + 4wn + j)*16 + li.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t n = static_cast<int64_t>(nb0 + wn * 4 + j) * 16 + li;
    const bool n_ok = n < p.N;
    float swn = 0.0f;
    if constexpr (EPI != kEpiI32) swn = n_ok ? p.sw[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = (mb0 + wm * 4 + i) * 16 + 4 * lg + r;
        const bool m_ok = m < p.M;
        if constexpr (EPI == kEpiI32) {
          if (m_ok && n_ok) static_cast<TY*>(p.y)[static_cast<int64_t>(m) * p.ldy + n] = acc[i][j][r];
        } else if constexpr (EPI == kEpiDequant) {
          if (m_ok && n_ok) {
            static_cast<TY*>(p.y)[static_cast<int64_t>(m) * p.ldy + n] =
                from_f32<TY>(dequant1(acc[i][j][r], p.sx[m], swn, p.bias, n));
          }
        } else {
          // Interleaved gate/up: even column = gate, odd column = up of
          // output n / 2.  Every lane dequantizes its own column; the even
          // lane takes the up value from its odd neighbour.
          const float sxm = m_ok ? p.sx[m] : 0.0f;
          const float v = (m_ok && n_ok) ? to_f32(from_f32<TH>(dequant1(acc[i][j][r], sxm, swn,
                                                                        p.bias, n)))
                                         : 0.0f;
          const float u = __shfl_xor(v, 1);
          if ((li & 1) == 0 && m_ok && n_ok) {
            const TH h = from_f32<TH>(silu_mul<TH>(v, u));
            TY* y = static_cast<TY*>(p.y) + static_cast<int64_t>(m) * p.ldy + n / 2;
            if constexpr (EPI == kEpiSilu) {
              *y = h;
            } else {
              *y = static_cast<int8_t>(quant1(to_f32(h), p.out_scale));
            }
          }
        }
      }
    }
  }
}

template <int EPI, typename TY, typename TH>
hipError_t launch_t(const GemmParams& p, hipStream_t st) {
  const int grid = p.per_xcd * kXcds;
  hipLaunchKernelGGL((gemm_kernel<EPI, TY, TH>), dim3(grid), dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(const LinearOperands& op, hipStream_t st) {
  GemmParams p;
  p.a = reinterpret_cast<const i32x4*>(op.a);
  p.sx = op.sx;
  p.w = reinterpret_cast<const i32x4*>(op.w);
  p.sw = op.sw;
  p.bias = op.bias;
  p.y = op.y;
  p.ldy = op.ldy;
  p.out_scale = op.out_scale;
  p.M = static_cast<int>(op.M);
  p.N = static_cast<int>(op.N);
  p.MB = static_cast<int>(ceil_div(op.M, kTileRows));
  p.NB = static_cast<int>(ceil_div(op.N, kTileRows));
  p.KB = static_cast<int>(ceil_div(op.K, kTileK));
  p.tiles_m = static_cast<int>(ceil_div(p.MB, kBMF));
  const int tiles_n = static_cast<int>(ceil_div(p.NB, kBNF));
  p.tiles = p.tiles_m * tiles_n;
  p.per_xcd = static_cast<int>(ceil_div(p.tiles, kXcds));
  if (p.tiles == 0) return hipSuccess;
  switch (op.epi) {
    case kEpiI32:
      return launch_t<kEpiI32, int32_t, float>(p, st);
    case kEpiDequant:
      if (op.y_dtype == kF16) return launch_t<kEpiDequant, __half, float>(p, st);
      if (op.y_dtype == kBF16) return launch_t<kEpiDequant, __hip_bfloat16, float>(p, st);
      if (op.y_dtype == kF32) return launch_t<kEpiDequant, float, float>(p, st);
      return hipErrorInvalidValue;
    case kEpiSilu:
      if (op.y_dtype == kF16) return launch_t<kEpiSilu, __half, __half>(p, st);
      if (op.y_dtype == kBF16) return launch_t<kEpiSilu, __hip_bfloat16, __hip_bfloat16>(p, st);
      return hipErrorInvalidValue;
    case kEpiSiluQ8:
      if (op.h_dtype == kF16) return launch_t<kEpiSiluQ8, int8_t, __half>(p, st);
      if (op.h_dtype == kBF16) return launch_t<kEpiSiluQ8, int8_t, __hip_bfloat16>(p, st);
      return hipErrorInvalidValue;
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace w8a8
