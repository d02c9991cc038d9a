// Prefill-regime W8A8 GEMM (M > 64, or M > 16 with M * N >= 32 * 12288):
// y = epi(xq @ wq^T) with int8 MFMA.
//
// Replaces the prefill/mixed projections (llama/paged_attention.py:1349-1352,
// 1488; llama/lightweight_runner.py:320-404) for the int8 contract of
// integer_linear_per_output_reference (nanopointllm/compression/w8a8.py:118-139).
//
// Design (MFMA-bound), chosen by measurement on MI355X:
//   * v_mfma_i32_32x32x32_i8, which sustains ~2x the int8 rate of the
//     16x16x64 form (4.4 vs 2.7 POPS in a register-only loop).
//   * Every wavefront owns BC adjacent 32x32 output blocks; the workgroup
//     tile is a WM x WN grid of them: 128x256 (16 wavefronts of 32x64) when
//     there are enough such tiles to fill every CU twice, else 128x128 (16
//     wavefronts of 32x32), else 64x64 with 4 wavefronts (4 workgroups per CU)
//     when 128x128 tiles would not cover every CU.  Many resident wavefronts
//     per SIMD hide the LDS and memory latency better than larger per-wave
//     tiles did; the 32x64 block halves the activation reads from LDS.
//   * Both operands are in the packed 16x64 tile layout, so a k-step (64) of
//     the workgroup tile is (BM + BN)/16 fragments of 1 KiB.  Each wavefront
//     copies its share with global_load_lds_dwordx4 straight into a 3- or
//     4-stage LDS ring (lane l lands at slot base + 16*l, the fragment layout),
//     keeping STG - 1 k-steps in flight; explicit vmcnt waits and one barrier
//     per k-step order the ring.  A 32x32x32 operand is the lane slots of two
//     adjacent 16-row tiles, read with ds_read_b128 as four contiguous
//     256-byte runs.
//   * Workgroups are mapped XCD-major: consecutive tiles of the same weight
//     column block land on the same XCD and share its L2.
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
  const uint32_t* rq_mult;
  const int32_t* rq_shift;
  const int32_t* rq_bias;
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

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

__device__ inline i32x16 mfma_32x32x32(i32x4 a, i32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// Waits until at most n of this wave's vector-memory loads (the LDS-DMA
// fragment copies) are outstanding.  gfx9 s_waitcnt: vmcnt in bits [3:0] and
// [15:14], expcnt [6:4] and lgkmcnt [11:8] left at their maxima.
template <int n>
__device__ inline void wait_vmcnt() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier for the LDS ring.  The wave's own LDS reads complete
// first (lgkmcnt(0)), so a later LDS-DMA write into the slot they read cannot
// overtake them; unlike __syncthreads it does not drain outstanding loads.
__device__ inline void ring_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// WM x WN wavefronts, each owning BC 32x32 blocks side by side (BM = 32 WM,
// BN = 32 WN BC), with an STG-deep LDS ring.
// The second launch bound is waves per SIMD: OCC workgroups of WM x WN
// wavefronts over the CU's 4 SIMDs, so the register budget admits OCC
// workgroups per CU.
template <int WM, int WN, int BC, int STG, int OCC, int EPI, typename TY, typename TH>
__global__ __launch_bounds__(WM * WN * 64, OCC * WM * WN / 4) void gemm_kernel(GemmParams p) {
  constexpr int NW = WM * WN;
  constexpr int BMF = 2 * WM;       // 16-row activation tiles per k-step
  constexpr int BNF = 2 * WN * BC;  // 16-row weight tiles per k-step
  constexpr int F = BMF + BNF;
  // Fragment copies per wave per k-step: LPW for the first F - (LPW-1) NW
  // waves, LPW - 1 for the rest.
  constexpr int LPW = (F + NW - 1) / NW;
  __shared__ i32x4 lds[STG][F][64];

  // XCD-major tile mapping: workgroup b runs on XCD b % 8.
  const int b = blockIdx.x;
  const int tile = (b % kXcds) * p.per_xcd + b / kXcds;
  if (tile >= p.tiles) return;
  const int mb0 = (tile % p.tiles_m) * BMF;
  const int nb0 = (tile / p.tiles_m) * BNF;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int KB = p.KB;

  // Fragment f = q*NW + wave of each k-step: f < BMF are activation blocks
  // mb0 + f, the rest weight blocks nb0 + f - BMF.  Blocks past the operand
  // are clamped to its last block: their products only reach accumulator
  // rows or columns that the epilogue never stores.
  const bool full = (LPW - 1) * NW + wave < F;  // wave-uniform
  const i32x4* src[LPW];
#pragma unroll
  for (int q = 0; q < LPW; ++q) {
    const int f = min(q * NW + wave, F - 1);
    if (f < BMF) {
      src[q] = p.a + static_cast<int64_t>(min(mb0 + f, p.MB - 1)) * KB * 64 + lane;
    } else {
      src[q] = p.w + static_cast<int64_t>(min(nb0 + f - BMF, p.NB - 1)) * KB * 64 + lane;
    }
  }
  auto issue = [&](int kb, int slot) {
#pragma unroll
    for (int q = 0; q < LPW; ++q)
      if (q < LPW - 1 || full)
        __builtin_amdgcn_global_load_lds(
            static_cast<const void*>(src[q] + static_cast<int64_t>(kb) * 64),
            (lds_void*)(&lds[slot][q * NW + wave][0]), 16, 0, 0);
  };

  i32x16 acc[BC];
#pragma unroll
  for (int j = 0; j < BC; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0;

#pragma unroll
  for (int s = 0; s < STG - 1; ++s)
    if (s < KB) issue(s, s);

  // 32x32x32 operands of k-half h: lane l takes 16 bytes of row l%32 of a
  // 16-row tile pair at k 32h + 16(l/32): slot (l%16) + 16(2h + l/32) of
  // tile (l%32)/16.
  const int fhalf = (lane >> 4) & 1;
  for (int kb = 0; kb < KB; ++kb) {
    // Stage kb has landed once only the later stages' loads may remain.
    if (kb + STG - 2 < KB) {
      if (full) {
        wait_vmcnt<LPW * (STG - 2)>();
      } else {
        wait_vmcnt<(LPW - 1) * (STG - 2)>();
      }
    } else {
      wait_vmcnt<0>();
    }
    ring_barrier();
    // Every wave has finished reading the slot of stage kb-1: refill it.
    if (kb + STG - 1 < KB) issue(kb + STG - 1, (kb + STG - 1) % STG);
    const int slot = kb % STG;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int fslot = (lane & 15) + 16 * (2 * h + (lane >> 5));
      const i32x4 af = lds[slot][2 * wm + fhalf][fslot];
      i32x4 bf[BC];
#pragma unroll
      for (int j = 0; j < BC; ++j) bf[j] = lds[slot][BMF + 2 * (wn * BC + j) + fhalf][fslot];
#pragma unroll
      for (int j = 0; j < BC; ++j) acc[j] = mfma_32x32x32(af, bf[j], acc[j]);
    }
  }

  // Epilogue.  Register r of block j in lane l holds row (mb0 + 2wm)*16 +
  // 8(r/4) + 4(l/32) + r%4 and column (nb0 + 2(wn BC + j))*16 + l%32.
  // When the output tile fits in the LDS ring, the values go to LDS first and
  // leave as 16-byte row chunks (a lane's own values are 2 rows x 32 columns
  // apart, so stored directly they make short partial-line writes).
  constexpr int BM = 32 * WM;
  constexpr int BN = 32 * WN * BC;
  constexpr bool kHalfCols = EPI == kEpiSilu || EPI == kEpiSiluQ8;  // one output per gate/up pair
  constexpr int BNO = kHalfCols ? BN / 2 : BN;
  constexpr int kOutBytes = static_cast<int>(sizeof(TY));
  constexpr bool kStage = BM * BNO * kOutBytes <= STG * F * 1024 && (BNO * kOutBytes) % 16 == 0;
  [[maybe_unused]] TY* const stile = reinterpret_cast<TY*>(&lds[0][0][0]);
  if constexpr (kStage) ring_barrier();  // every wave is done reading the ring
  // Writes output (m, n_out) of tile-local row ml and column nlo.
  auto put = [&](int ml, int nlo, bool ok, int64_t m, int64_t n_out, TY v) {
    if constexpr (kStage) {
      stile[ml * BNO + nlo] = v;
    } else {
      if (ok) static_cast<TY*>(p.y)[m * p.ldy + n_out] = v;
    }
  };
#pragma unroll
  for (int j = 0; j < BC; ++j) {
    const int nl = 32 * (wn * BC + j) + (lane & 31);
    const int64_t n = static_cast<int64_t>(nb0) * 16 + nl;
    const bool n_ok = n < p.N;
    float swn = 0.0f;
    if constexpr (EPI != kEpiI32 && EPI != kEpiRequant) swn = n_ok ? p.sw[n] : 0.0f;
    uint32_t rq_mult = 0;
    int32_t rq_shift = 0, rq_bias = 0;
    if constexpr (EPI == kEpiRequant) {
      if (n_ok) {
        rq_mult = p.rq_mult[n];
        rq_shift = p.rq_shift[n];
        rq_bias = p.rq_bias != nullptr ? p.rq_bias[n] : 0;
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ml = 32 * wm + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      const int m = mb0 * 16 + ml;
      const bool m_ok = m < p.M;
      const bool ok = m_ok && n_ok;
      const int32_t a = acc[j][r];
      if constexpr (EPI == kEpiI32) {
        put(ml, nl, ok, m, n, a);
      } else if constexpr (EPI == kEpiDequant) {
        const float sxm = m_ok ? p.sx[m] : 0.0f;
        put(ml, nl, ok, m, n, from_f32<TY>(dequant1(a, sxm, swn, ok ? p.bias : nullptr, n)));
      } else if constexpr (EPI == kEpiRequant) {
        put(ml, nl, ok, m, n, static_cast<int8_t>(requant1(a, rq_bias, rq_mult, rq_shift)));
      } else if constexpr (EPI == kEpiBf16Exact) {
        const float sxm = m_ok ? p.sx[m] : 0.0f;
        put(ml, nl, ok, m, n,
            __builtin_bit_cast(TY, dequant_bf16_exact(a, f16_bits(sxm), f16_bits(swn))));
      } else {
        // Interleaved gate/up: even column = gate, odd column = up of output
        // n / 2.  Every lane dequantizes its own column; the even lane takes
        // the up value from its odd neighbour.
        const float sxm = m_ok ? p.sx[m] : 0.0f;
        const float v = ok ? to_f32(from_f32<TH>(dequant1(a, sxm, swn, p.bias, n))) : 0.0f;
        const float u = __shfl_xor(v, 1);
        if ((lane & 1) == 0) {
          const TH h = from_f32<TH>(silu_mul<TH>(v, u));
          if constexpr (EPI == kEpiSilu) {
            put(ml, nl / 2, ok, m, n / 2, h);
          } else {
            put(ml, nl / 2, ok, m, n / 2, static_cast<int8_t>(quant1(to_f32(h), p.out_scale)));
          }
        }
      }
    }
  }
  if constexpr (kStage) {
    __syncthreads();
    constexpr int EV = 16 / kOutBytes;  // outputs per 16-byte chunk
    constexpr int CPR = BNO / EV;       // chunks per tile row
    constexpr int NT = NW * 64;
    constexpr int RPP = NT / CPR;       // tile rows per pass
    static_assert(NT % CPR == 0, "threads cover whole rows");
    const int64_t n_out_total = kHalfCols ? p.N / 2 : p.N;
    const int64_t n0 = kHalfCols ? static_cast<int64_t>(nb0) * 8 : static_cast<int64_t>(nb0) * 16;
    const bool vec_ok =
        ((reinterpret_cast<uintptr_t>(p.y) | static_cast<uintptr_t>(p.ldy * kOutBytes)) & 15) == 0;
#pragma unroll
    for (int base = 0; base < BM; base += RPP) {
      const int ml = base + static_cast<int>(threadIdx.x) / CPR;
      const int nlo = (static_cast<int>(threadIdx.x) % CPR) * EV;
      const int64_t m = static_cast<int64_t>(mb0) * 16 + ml;
      const int64_t n = n0 + nlo;
      if (ml < BM && m < p.M && n < n_out_total) {
        TY* dst = static_cast<TY*>(p.y) + m * p.ldy + n;
        const TY* src = stile + ml * BNO + nlo;
        if (vec_ok && n + EV <= n_out_total) {
          *reinterpret_cast<i32x4*>(dst) = *reinterpret_cast<const i32x4*>(src);
        } else {
          for (int e = 0; e < EV; ++e)
            if (n + e < n_out_total) dst[e] = src[e];
        }
      }
    }
  }
}

// Launches one tile configuration for the problem in p (tile counts are
// filled in here).
template <int WM, int WN, int BC, int STG, int OCC, int EPI, typename TY, typename TH>
hipError_t launch_cfg(GemmParams p, hipStream_t st) {
  p.tiles_m = static_cast<int>(ceil_div(p.MB, 2 * WM));
  const int tiles_n = static_cast<int>(ceil_div(p.NB, 2 * WN * BC));
  p.tiles = p.tiles_m * tiles_n;
  p.per_xcd = static_cast<int>(ceil_div(p.tiles, kXcds));
  if (p.tiles == 0) return hipSuccess;
  hipLaunchKernelGGL((gemm_kernel<WM, WN, BC, STG, OCC, EPI, TY, TH>), dim3(p.per_xcd * kXcds),
                     dim3(WM * WN * 64), 0, st, p);
  return hipGetLastError();
}

// Tile configurations, chosen by tile count (measured on MI355X, random data,
// cold weights, LLaMA-7B projections at M = 256..2048):
//   * 128x256, 16 waves of 32x64 blocks, 3-stage ring, 2 workgroups per CU,
//     when there are at least ~0.82 tiles per workgroup slot (2 per CU): each
//     MFMA moves 1.5 KiB of operands through LDS instead of 2, 3-12% faster.
//     Just past one full round of slots (1 to 1.16 tiles per slot) the few
//     tiles of the second round cost more than that saves, and the 128x128
//     tile is kept;
//   * else 128x128, 16 waves of 32x32, 4 stages, 2 per CU, when those cover
//     every CU;
//   * else 64x64, 4 waves, 4 per CU.
template <int EPI, typename TY, typename TH>
hipError_t launch_t(const GemmParams& p, hipStream_t st) {
  // (The integer-requant epilogue needs more registers than two workgroups
  // per CU leave it, so it keeps the 128x128 tile.)
  if constexpr (EPI != kEpiRequant) {
    const int64_t wide_tiles = ceil_div(p.MB, 8) * ceil_div(p.NB, 16);
    const int64_t slots = static_cast<int64_t>(cu_count()) * 2;
    const bool short_second_round = wide_tiles > slots && wide_tiles * 100 < slots * 116;
    if (wide_tiles * 100 >= slots * 82 && !short_second_round)
      return launch_cfg<4, 4, 2, 3, 2, EPI, TY, TH>(p, st);
  }
  const int64_t big_tiles = ceil_div(p.MB, 8) * ceil_div(p.NB, 8);
  if (big_tiles >= cu_count()) return launch_cfg<4, 4, 1, 4, 2, EPI, TY, TH>(p, st);
  return launch_cfg<2, 2, 1, 4, 4, EPI, TY, TH>(p, st);
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
  p.rq_mult = op.rq_mult;
  p.rq_shift = op.rq_shift;
  p.rq_bias = op.rq_bias;
  p.M = static_cast<int>(op.M);
  p.N = static_cast<int>(op.N);
  p.MB = static_cast<int>(ceil_div(op.M, kTileRows));
  p.NB = static_cast<int>(ceil_div(op.N, kTileRows));
  p.KB = static_cast<int>(ceil_div(op.K, kTileK));
  p.tiles_m = p.tiles = p.per_xcd = 0;
  if (p.MB == 0 || p.NB == 0) return hipSuccess;
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
    case kEpiRequant:
      return launch_t<kEpiRequant, int8_t, float>(p, st);
    case kEpiBf16Exact:
      return launch_t<kEpiBf16Exact, __hip_bfloat16, float>(p, st);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace w8a8
