// Dense 16-bit GEMV for the LM head at decode batches: y = x @ w^T (+ bias)
// with binary16 or bfloat16 x, w and y, binary32 accumulation
// (v_mfma_f32_16x16x32_{f16,bf16}).
//
// Replaces the LM head's F.linear at decode batches
// (llama/lightweight_runner.py:675-681: lm_head of the final-norm rows, a
// plain 16-bit nn.Linear, not a W8A8 linear).  The weight stays in the
// module's own row-major [N, K] layout.
//
// Design (HBM-bound: every weight byte is read once, 2 bytes per MAC per row
// of x):
//   * G = min(ceil(N/16), CUs) persistent workgroups of 16 wavefronts; block
//     nb of 16 weight rows goes to workgroup nb % G.
//   * Wavefront w owns a contiguous range of K-steps.  Its x fragments for
//     those steps are loaded once and stay in registers.
//   * Weights stream through a ring of register buffers with buffer loads
//     whose range ends at the block's last row: rows past N and columns past
//     K read zeros.
//   * Each load instruction reads 8 weight rows x 128 contiguous bytes,
//     whole cache lines, through an MFMA tile whose columns are (weight row,
//     K half) pairs and whose rows are (x row, K half) pairs (see
//     gemv_dense_halves_kernel); rows 9-16 of x take a second A operand.
//     Cold LM head 32003 x 4096 at M = 8, graphs: 43 us (6.0 TB/s) against
//     50 us for the usual operand layout (16 rows x 64 bytes per load) and
//     58 us for torch's F.linear on the same GPU.
//   * Each wavefront's binary32 partials go to LDS at the end of the block;
//     after one barrier, one thread per output adds each wavefront's two K
//     halves, the wavefronts in order and the bias, and rounds once to the
//     output type.  Two LDS buffers alternate between blocks, so one barrier
//     per block suffices.
// The summation order is fixed (per K half: MFMA over 32 columns, the
// wavefront's steps in order; then the two halves, then wavefronts 0..15),
// the same for every row and batch size, so the result is deterministic and
// row m's values do not depend on the other rows of the batch.
#include <type_traits>
#include <utility>

#include "w8a8_internal.h"

namespace w8a8 {

namespace {

constexpr int kDenseWaves = 16;
constexpr int kDenseThreads = kDenseWaves * 64;
constexpr int kBufferWord3 = 0x00020000;  // gfx9 raw buffer, 32-bit data format
constexpr int kCacheNT = 2;               // nontemporal: each weight byte is read once
constexpr int kOutside = 0x7ffffff0;      // an offset beyond every range

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct DenseParams {
  const void* x;
  int64_t ldx;
  const void* w;
  int64_t ldw;
  const void* bias;
  void* y;
  int64_t ldy;
  int M;
  int N;
  int K;
  int NB;
  int G;
};

// f(integral_constant<int, I>) for I = 0 .. N-1, unrolled at compile time.
template <typename F, int... I>
__device__ inline void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <typename T>
__device__ inline f32x4 mfma_f32_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (std::is_same<T, __half>::value) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a),
                                                  __builtin_bit_cast(h8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, a),
                                                   __builtin_bit_cast(b8, b), c, 0, 0, 0);
  }
}

// Each weight load covers whole 128-byte lines.  A K-step is 64 columns;
// weight load q (rows 8q .. 8q+7 of the block) gives lane l row 8q + l%8 at
// columns 64s + 32h + 8g .. +7 (h = (l/8)%2, g = l/16), so the 8 lanes of a
// row read its 128 contiguous bytes.  That is the B operand
// of an MFMA whose 16 columns are (row, half h) pairs; its A operand (lane l:
// x row l%8, half (l%16)/8, columns 64s + 32 half + 8g .. +7) pairs x row m
// and half h in its row m + 8h.  Output (m + 8h, r + 8h) of the 16 x 16 tile
// is then row m's partial over half h of the step with weight row r; the
// mixed-half outputs are discarded.  The epilogue adds each wavefront's two
// halves, then the wavefronts in order.  RG groups of 8 x rows (RG = 2: rows
// 8 .. 15 in a second A operand against the same weight fragments, with the
// same arithmetic per row).  XS: 64-column K-steps per wavefront; CS: K-steps
// per ring step; RING: ring buffers.
template <typename T, int RG, int XS, int CS, int RING>
__global__ __launch_bounds__(kDenseThreads) void gemv_dense_halves_kernel(DenseParams p) {
  static_assert(XS % CS == 0, "whole ring steps per block");
  constexpr int kStepK = 64;
  constexpr int kHalf = 128 * RG;  // partials of one half: 8 RG rows x 16 outputs
  __shared__ float red[2][kDenseWaves][2 * kHalf];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lg = lane >> 4;
  const int K = p.K;
  const int ks0 = wave * XS;

  // x fragments (A operand): row 8g + (lane % 16) % 8, half (lane % 16) / 8.
  u32x4 xf[RG][XS];
  {
    const int nrec = __builtin_amdgcn_readfirstlane(
        static_cast<int>((p.M - 1) * p.ldx * 2) + K * 2);
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.x), 0, nrec, kBufferWord3);
    const int m = lane & 7;
    const int half = (lane >> 3) & 1;
#pragma unroll
    for (int g = 0; g < RG; ++g)
#pragma unroll
      for (int s = 0; s < XS; ++s) {
        const int k = (ks0 + s) * kStepK + 32 * half + 8 * lg;
        const int row = 8 * g + m;
        const int off =
            row < p.M && k < K ? static_cast<int>(row * p.ldx * 2) + k * 2 : kOutside;
        xf[g][s] =
            __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
      }
  }

  // Weight lanes: row 8q + lane%8, columns 32 ((lane/8)%2) + 8 (lane/16).
  const int wrow = lane & 7;
  const int wcol = 32 * ((lane >> 3) & 1) + 8 * lg;
  constexpr int nch = XS / CS;
  const int n_mine = (p.NB - static_cast<int>(blockIdx.x) + p.G - 1) / p.G;
  const int total = n_mine * nch;
  int lj = 0, lc = 0;  // next step to load
  auto issue = [&](u32x4(&buf)[2 * CS]) {
    const bool past = lj >= n_mine;
    const int sj = __builtin_amdgcn_readfirstlane(past ? n_mine - 1 : lj);
    const int64_t nb = static_cast<int64_t>(blockIdx.x) + static_cast<int64_t>(sj) * p.G;
    const int rows = static_cast<int>(min<int64_t>(16, p.N - nb * 16));
    const int nrec = __builtin_amdgcn_readfirstlane(
        past ? 0 : static_cast<int>((rows - 1) * p.ldw * 2) + K * 2);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(static_cast<const uint16_t*>(p.w) + nb * 16 * p.ldw), 0, nrec,
        kBufferWord3);
#pragma unroll
    for (int i = 0; i < CS; ++i) {
      const int k = (ks0 + lc * CS + i) * kStepK + wcol;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int off = k < K ? static_cast<int>((8 * q + wrow) * p.ldw * 2) + k * 2 : kOutside;
        buf[2 * i + q] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, kCacheNT));
      }
    }
    const int nc = lc + 1;
    const bool wrap = nc == nch;
    lj += wrap ? 1 : 0;
    lc = wrap ? 0 : nc;
  };

  u32x4 rb[RING][2 * CS];
#pragma unroll
  for (int u = 0; u < RING - 1; ++u) issue(rb[u]);

  f32x4 acc[RG][2];
#pragma unroll
  for (int g = 0; g < RG; ++g) acc[g][0] = acc[g][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // Lane l holds tile rows 4(l/16) .. +3 (x row m, half l/32) and column
  // l%16 (weight row l%8 of half (l/8)%2): its outputs are kept when the
  // halves agree.
  const bool keep = (lane >> 5) == ((lane >> 3) & 1);
  const int half_out = lane >> 5;
  int j = 0;
  auto step = [&](auto chunk, const u32x4(&cur)[2 * CS], u32x4(&freed)[2 * CS], int t) {
    constexpr int C = decltype(chunk)::value;
    issue(freed);
    const bool live = t < total;
    if (live) {
#pragma unroll
      for (int i = 0; i < CS; ++i) {
#pragma unroll
        for (int g = 0; g < RG; ++g)
#pragma unroll
          for (int q = 0; q < 2; ++q)
            acc[g][q] = mfma_f32_16x16x32<T>(xf[g][C * CS + i], cur[2 * i + q], acc[g][q]);
      }
    }
    if constexpr (C == nch - 1) {
      if (live) {
        const int par = j & 1;
        if (keep) {
#pragma unroll
          for (int g = 0; g < RG; ++g)
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int m = 8 * g + ((4 * lg + r) & 7);
                red[par][wave][half_out * kHalf + m * 16 + 8 * q + wrow] = acc[g][q][r];
              }
        }
#pragma unroll
        for (int g = 0; g < RG; ++g) acc[g][0] = acc[g][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        __syncthreads();
        if (tid < kHalf) {
          const int m = tid >> 4;
          const int n_local = tid & 15;
          const int64_t n =
              (static_cast<int64_t>(blockIdx.x) + static_cast<int64_t>(j) * p.G) * 16 + n_local;
          if (m < p.M && n < p.N) {
            float s = __fadd_rn(red[par][0][tid], red[par][0][kHalf + tid]);
#pragma unroll
            for (int w = 1; w < kDenseWaves; ++w)
              s = __fadd_rn(s, __fadd_rn(red[par][w][tid], red[par][w][kHalf + tid]));
            if (p.bias != nullptr) s = __fadd_rn(s, to_f32(static_cast<const T*>(p.bias)[n]));
            static_cast<T*>(p.y)[m * p.ldy + n] = from_f32<T>(s);
          }
        }
        ++j;
      }
    }
  };
  constexpr int kPeriod = RING * nch;
  for (int t = 0; t < total; t += kPeriod) {
    static_for<kPeriod>([&](auto u) {
      constexpr int U = decltype(u)::value;
      step(std::integral_constant<int, U % nch>{}, rb[U % RING], rb[(U + RING - 1) % RING],
           t + U);
    });
  }
}

template <typename T>
hipError_t launch_dense_t(const DenseParams& p, hipStream_t st) {
  const dim3 grid(p.G), block(kDenseThreads);
  // Register budget (128 per lane): the x fragments of RG x XS steps and RING
  // buffers of 2 CS weight fragments.  Up to 4096 columns: 4 steps of 64 per
  // wavefront; up to 8192: 8.  Rows 9-16 double the x fragments, so their
  // rings are shorter.
  const bool short_k = p.K <= kDenseWaves * 4 * 64;
  if (p.M <= 8) {
    if (short_k)
      hipLaunchKernelGGL((gemv_dense_halves_kernel<T, 1, 4, 2, 4>), grid, block, 0, st, p);
    else
      hipLaunchKernelGGL((gemv_dense_halves_kernel<T, 1, 8, 1, 4>), grid, block, 0, st, p);
  } else if (short_k) {
    hipLaunchKernelGGL((gemv_dense_halves_kernel<T, 2, 4, 2, 3>), grid, block, 0, st, p);
  } else {
    hipLaunchKernelGGL((gemv_dense_halves_kernel<T, 2, 8, 1, 2>), grid, block, 0, st, p);
  }
  return hipGetLastError();
}

}  // namespace

int64_t dense_gemv_max_k() { return static_cast<int64_t>(kDenseWaves) * 8 * 64; }

hipError_t launch_gemv_dense(const void* x, int64_t ldx, const void* w, int64_t ldw,
                             const void* bias, void* y, int64_t ldy, int dtype, int64_t M,
                             int64_t N, int64_t K, hipStream_t st) {
  DenseParams p;
  p.x = x;
  p.ldx = ldx;
  p.w = w;
  p.ldw = ldw;
  p.bias = bias;
  p.y = y;
  p.ldy = ldy;
  p.M = static_cast<int>(M);
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.NB = static_cast<int>(ceil_div(N, kTileRows));
  p.G = static_cast<int>(p.NB < cu_count() ? p.NB : cu_count());
  if (dtype == kF16) return launch_dense_t<__half>(p, st);
  if (dtype == kBF16) return launch_dense_t<__hip_bfloat16>(p, st);
  return hipErrorInvalidValue;
}

}  // namespace w8a8
