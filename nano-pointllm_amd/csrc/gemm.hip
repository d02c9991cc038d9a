// Prefill-regime W8A8 GEMM (M > 64, or M > 32 with N > 12288 and K > 4096):
// y = epi(xq @ wq^T) with int8 MFMA.
//
// Replaces the prefill/mixed projections (llama/paged_attention.py:1349-1352,
// 1488; llama/lightweight_runner.py:320-404) for the int8 contract of
// integer_linear_per_output_reference (nanopointllm/compression/w8a8.py:118-139).
//
// Design (MFMA-bound), chosen by measurement on MI355X (gemm_kernel; the
// weights-direct gemm_wd_kernel further below keeps the weights out of LDS):
//   * v_mfma_i32_16x16x64_i8.  Its operand is exactly one packed 16x64
//     fragment (lane l holds 16 bytes of row l%16), read with one contiguous
//     ds_read_b128.  On random int8 data it sustains more than the 32x32x32
//     form: 3.3 against 3.0 POPS from LDS alone, and 15-25% more in this
//     kernel on LLaMA-7B shapes (the matrix pipes slow down with the
//     data-dependent switching of their inputs).
//   * Every wavefront owns a BR x BC grid of 16x16 output blocks; the
//     workgroup tile is a WM x WN grid of wavefronts: 128x256 (8 wavefronts
//     of 64x64) when there are enough such tiles to fill every CU twice, else
//     128x128 (16 wavefronts of 32x32), else 64x64 (4 wavefronts of 32x32,
//     4 workgroups per CU) when 128x128 tiles would not cover every CU; past
//     64 rows, 64x32 (4 wavefronts of 32x16) when those fill one round; and
//     112x96 (14 wavefronts of 16x48) or 128x96 (8 of 32x48), one per CU,
//     when one round of those fills the CUs.  The full rule is at launch_t.
//   * Both operands are in the packed 16x64 tile layout, so a k-step (64) of
//     the workgroup tile is (BM + BN)/16 fragments of 1 KiB.  Each wavefront
//     copies its share with global_load_lds_dwordx4 straight into a 3- or
//     4-stage LDS ring (lane l lands at slot base + 16*l, the fragment layout),
//     keeping STG - 1 k-steps in flight; explicit vmcnt waits and one barrier
//     per k-step order the ring.
//   * Workgroups are mapped XCD-major: consecutive tiles of the same weight
//     column block land on the same XCD and share its L2.
#include "w8a8_internal.h"

#include <utility>

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
  float* absmax_parts;  // kEpiSilu: [M][NB] per-block row |h|max (nullable)
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

typedef __attribute__((address_space(3))) void lds_void;

// C layout: lane l, register r holds row 4(l/16) + r (activation) and column
// l%16 (weight row) of the 16x16 block.
__device__ inline i32x4 mfma_16x16x64(i32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
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

// Stores a workgroup's output tile through the epilogue EPI: a WM x WN grid
// of wavefronts, each holding BR x BC 16x16 blocks of int32 accumulators.
// Register r of block (i, j) in lane l holds tile row 16(wm BR + i) +
// 4(l/16) + r and tile column 16(wn BC + j) + l%16.  When the output tile
// fits in the STAGE_BYTES of LDS at `stage` (whose operand reads every wave
// has finished once the first barrier below passes), the values go to LDS
// first and leave as 16-byte row chunks (stored directly, 16 lanes cover only
// 16 columns of a row: short partial-line writes).
template <int WM, int WN, int BR, int BC, int STAGE_BYTES, int EPI, typename TY, typename TH>
__device__ inline void store_tile(const GemmParams& p, i32x4 (&acc)[BR][BC], int wm, int wn,
                                  int mb0, int nb0, int lane, void* stage) {
  constexpr int BM = 16 * WM * BR;
  constexpr int BN = 16 * WN * BC;
  constexpr bool kHalfCols = EPI == kEpiSilu || EPI == kEpiSiluQ8;  // one output per gate/up pair
  constexpr int BNO = kHalfCols ? BN / 2 : BN;
  constexpr int kOutBytes = static_cast<int>(sizeof(TY));
  constexpr bool kStage = BM * BNO * kOutBytes <= STAGE_BYTES && (BNO * kOutBytes) % 16 == 0;
  [[maybe_unused]] TY* const stile = static_cast<TY*>(stage);
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
  for (int i = 0; i < BR; ++i)
#pragma unroll
  for (int j = 0; j < BC; ++j) {
    const int nl = 16 * (wn * BC + j) + (lane & 15);
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
    if constexpr (kHalfCols) {
      // kEpiSilu with absmax_parts: |h| of this lane's output for row pair r / 2.
      [[maybe_unused]] float habs[2] = {0.0f, 0.0f};
      // Interleaved gate/up: even column = gate, odd column = up of output
      // n / 2.  Every lane dequantizes its own column at rows r and r + 1;
      // then the even lane forms output row r from its gate and the odd
      // lane's up, and the odd lane output row r + 1 from the even lane's
      // gate and its own up, so each SiLU is evaluated by one lane.
      const bool odd = (lane & 1) != 0;
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        const int ml0 = 16 * (wm * BR + i) + 4 * (lane >> 4) + r;
        float v[2];
        bool vok[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int64_t m = static_cast<int64_t>(mb0) * 16 + ml0 + e;
          const bool m_ok = m < p.M;
          vok[e] = m_ok && n_ok;
          const float sxm = m_ok ? p.sx[m] : 0.0f;
          v[e] = vok[e] ? to_f32(from_f32<TH>(dequant1(acc[i][j][r + e], sxm, swn, p.bias, n)))
                        : 0.0f;
        }
        const float x = __shfl_xor(odd ? v[0] : v[1], 1);
        const float g = odd ? x : v[0];
        const float u = odd ? v[1] : x;
        const int ml = ml0 + (odd ? 1 : 0);
        const int64_t m = static_cast<int64_t>(mb0) * 16 + ml;
        const bool ok = odd ? vok[1] : vok[0];
        const TH h = from_f32<TH>(silu_mul<TH>(g, u));
        if constexpr (EPI == kEpiSilu) {
          put(ml, nl / 2, ok, m, n / 2, h);
          if (ok) habs[r >> 1] = fabsf(to_f32(h));
        } else {
          put(ml, nl / 2, ok, m, n / 2, static_cast<int8_t>(quant1(to_f32(h), p.out_scale)));
        }
      }
      if constexpr (EPI == kEpiSilu) {
        if (p.absmax_parts != nullptr) {
          // Lanes of one parity in a 16-lane group hold the same output row
          // (even lanes row r, odd lanes row r + 1) over the 8 outputs of
          // packed block nb: reduce over them, then one store per row.
          const int64_t nb = static_cast<int64_t>(nb0) + wn * BC + j;
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            float v = habs[h2];
#pragma unroll
            for (int off = 2; off < 16; off <<= 1) v = fmaxf(v, __shfl_xor(v, off));
            const int64_t m = static_cast<int64_t>(mb0) * 16 + 16 * (wm * BR + i) +
                              4 * (lane >> 4) + 2 * h2 + (lane & 1);
            if ((lane & 15) < 2 && m < p.M && nb < p.NB) p.absmax_parts[m * p.NB + nb] = v;
          }
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ml = 16 * (wm * BR + i) + 4 * (lane >> 4) + r;
        const int64_t m = static_cast<int64_t>(mb0) * 16 + ml;
        const bool m_ok = m < p.M;
        const bool ok = m_ok && n_ok;
        const int32_t a = acc[i][j][r];
        if constexpr (EPI == kEpiI32) {
          put(ml, nl, ok, m, n, a);
        } else if constexpr (EPI == kEpiDequant) {
          const float sxm = m_ok ? p.sx[m] : 0.0f;
          put(ml, nl, ok, m, n, from_f32<TY>(dequant1(a, sxm, swn, ok ? p.bias : nullptr, n)));
        } else if constexpr (EPI == kEpiRequant) {
          put(ml, nl, ok, m, n, static_cast<int8_t>(requant1(a, rq_bias, rq_mult, rq_shift)));
        } else {
          static_assert(EPI == kEpiBf16Exact, "epilogue");
          const float sxm = m_ok ? p.sx[m] : 0.0f;
          put(ml, nl, ok, m, n,
              __builtin_bit_cast(TY, dequant_bf16_exact(a, f16_bits(sxm), f16_bits(swn))));
        }
      }
    }
  }
  if constexpr (kStage) {
    __syncthreads();
    constexpr int EV = 16 / kOutBytes;  // outputs per 16-byte chunk
    constexpr int CPR = BNO / EV;       // chunks per tile row
    constexpr int NT = WM * WN * 64;
    constexpr int RPP = NT / CPR;       // tile rows per pass; threads past RPP * CPR idle
    static_assert(RPP >= 1, "a pass covers at least one tile row");
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
      if (static_cast<int>(threadIdx.x) < RPP * CPR && ml < BM && m < p.M && n < n_out_total) {
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

// WM x WN wavefronts, each owning BR x BC blocks of 16x16 (BM = 16 WM BR,
// BN = 16 WN BC), with an STG-deep LDS ring whose stages hold KT k-blocks
// (64 K each) of both operands.
// The second launch bound is waves per SIMD: OCC workgroups of WM x WN
// wavefronts over the CU's 4 SIMDs, so the register budget admits OCC
// workgroups per CU.
template <int WM, int WN, int BR, int BC, int STG, int OCC, int KT, int EPI, typename TY,
          typename TH>
__global__ __launch_bounds__(WM * WN * 64, OCC * WM * WN / 4) void gemm_kernel(GemmParams p) {
  constexpr int NW = WM * WN;
  constexpr int BMF = WM * BR;  // 16-row activation tiles per k-block
  constexpr int BNF = WN * BC;  // 16-row weight tiles per k-block
  constexpr int F = BMF + BNF;
  constexpr int FS = F * KT;    // fragments per stage
  // Fragment copies per wave per stage: LPW for the first FS - (LPW-1) NW
  // waves, LPW - 1 for the rest.
  constexpr int LPW = (FS + NW - 1) / NW;
  __shared__ i32x4 lds[STG][FS][64];

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
  const int NS = static_cast<int>(ceil_div(KB, KT));  // ring stages over K

  // Fragment f = q*NW + wave of a stage is k-block f / F of the stage; of
  // that k-block, g = f % F < BMF are activation blocks mb0 + g, the rest
  // weight blocks nb0 + g - BMF.  Blocks past the operand are clamped to its
  // last block: their products only reach accumulator rows or columns that
  // the epilogue never stores.  K-blocks past KB (the last stage of a K that
  // is not a multiple of 64 KT) reload block KB - 1 and are not multiplied.
  const bool full = (LPW - 1) * NW + wave < FS;  // wave-uniform
  const i32x4* src[LPW];
  int kk_of[LPW];
#pragma unroll
  for (int q = 0; q < LPW; ++q) {
    const int f = min(q * NW + wave, FS - 1);
    const int g = f % F;
    kk_of[q] = f / F;
    if (g < BMF) {
      src[q] = p.a + static_cast<int64_t>(min(mb0 + g, p.MB - 1)) * KB * 64 + lane;
    } else {
      src[q] = p.w + static_cast<int64_t>(min(nb0 + g - BMF, p.NB - 1)) * KB * 64 + lane;
    }
  }
  auto issue = [&](int stage, int slot) {
#pragma unroll
    for (int q = 0; q < LPW; ++q)
      if (q < LPW - 1 || full) {
        const int kb = min(stage * KT + kk_of[q], KB - 1);
        __builtin_amdgcn_global_load_lds(
            static_cast<const void*>(src[q] + static_cast<int64_t>(kb) * 64),
            (lds_void*)(&lds[slot][q * NW + wave][0]), 16, 0, 0);
      }
  };

  i32x4 acc[BR][BC];
#pragma unroll
  for (int i = 0; i < BR; ++i)
#pragma unroll
    for (int j = 0; j < BC; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0;

#pragma unroll
  for (int s = 0; s < STG - 1; ++s)
    if (s < NS) issue(s, s);

  for (int st = 0; st < NS; ++st) {
    // Stage st has landed once only the later stages' loads may remain.
    if (st + STG - 2 < NS) {
      if (full) {
        wait_vmcnt<LPW * (STG - 2)>();
      } else {
        wait_vmcnt<(LPW - 1) * (STG - 2)>();
      }
    } else {
      wait_vmcnt<0>();
    }
    ring_barrier();
    // Every wave has finished reading the slot of stage st-1: refill it.
    if (st + STG - 1 < NS) issue(st + STG - 1, (st + STG - 1) % STG);
    const int slot = st % STG;
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      if (KT == 1 || st * KT + kk < KB) {
        i32x4 af[BR], bf[BC];
#pragma unroll
        for (int i = 0; i < BR; ++i) af[i] = lds[slot][kk * F + wm * BR + i][lane];
#pragma unroll
        for (int j = 0; j < BC; ++j) bf[j] = lds[slot][kk * F + BMF + wn * BC + j][lane];
#pragma unroll
        for (int i = 0; i < BR; ++i)
#pragma unroll
          for (int j = 0; j < BC; ++j) acc[i][j] = mfma_16x16x64(af[i], bf[j], acc[i][j]);
      }
    }
  }

  store_tile<WM, WN, BR, BC, STG * FS * 1024, EPI, TY, TH>(p, acc, wm, wn, mb0, nb0, lane,
                                                           &lds[0][0][0]);
}

// Workgroup barrier with the wave's LDS reads complete, through the builtin
// s_waitcnt, so the compiler's own wait insertion knows they are (an inline
// asm wait is opaque to it, and it would then wait for the newer reads of
// the next k-block too).  The empty asm statements keep LDS accesses on
// their side of the barrier.
__device__ inline void ring_barrier_tracked() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt at their maxima
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// f(integral_constant<int, I>) for I = 0 .. N-1, unrolled at compile time.
template <typename F, int... I>
__device__ inline void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ inline __amdgpu_buffer_rsrc_t dma_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}

// 16 bytes per lane from the buffer at voffset into LDS at lds + 16 * lane
// (buffer_load_dwordx4 ... lds).
__device__ inline void dma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voffset, 0, 0, 0);
}

// Weights-direct GEMM: NW wavefronts, each owning all A 16-row activation
// blocks of the tile and B 16-row weight blocks of its own (tile 16A x
// 16 NW B).  A weight fragment is used by exactly one wavefront, so it goes
// from global memory straight into registers (the packed fragment is the
// MFMA operand image) through a ring of D + 1 register sets, D k-blocks ahead;
// only the activation fragments, which every wavefront reads, pass through
// LDS: buffer_load ... lds copies into an S-slot ring, and each wavefront
// reads k-block t+1 into registers during k-block t's MFMAs.  Per k-block a
// wavefront reads A KiB from LDS for A x B MFMAs, against (BR + BC) KiB for
// BR x BC in gemm_kernel.  One barrier per k-block.
template <int NW, int A, int B, int D, int EPI, typename TY, typename TH>
__global__ __launch_bounds__(NW * 64, NW / 4) void gemm_wd_kernel(GemmParams p) {
  static_assert(D >= 2 && NW % 4 == 0, "prefetch depth and wavefront count");
  constexpr int S = D <= 2 ? 2 : (D <= 4 ? 4 : 8);  // ring slots: a power of two >= D
  constexpr int BS = D + 1;                          // weight register sets
  constexpr int LPW = (A + NW - 1) / NW;             // activation copies per wavefront
  constexpr int BM = 16 * A;
  constexpr int BN = 16 * NW * B;
  constexpr bool kHalfCols = EPI == kEpiSilu || EPI == kEpiSiluQ8;
  constexpr int kRing = S * A * 1024;
  constexpr int kOut = BM * (kHalfCols ? BN / 2 : BN) * static_cast<int>(sizeof(TY));
  constexpr int kLds = kRing > kOut ? kRing : kOut;
  __shared__ i32x4 lds[kLds / 16];
  auto ring = reinterpret_cast<i32x4 (*)[A][64]>(lds);

  const int b = blockIdx.x;
  const int tile = (b % kXcds) * p.per_xcd + b / kXcds;
  if (tile >= p.tiles) return;
  const int mb0 = (tile % p.tiles_m) * A;
  const int nb0 = (tile / p.tiles_m) * (NW * B);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int KB = p.KB;

  // Activation block q * NW + wave of the tile (clamped to the last block:
  // its products reach only rows the epilogue never stores).
  const bool full = (LPW - 1) * NW + wave < A;
  const __amdgpu_buffer_rsrc_t arsrc = dma_rsrc(p.a + static_cast<int64_t>(mb0) * KB * 64);
  uint32_t aoff[LPW];
#pragma unroll
  for (int q = 0; q < LPW; ++q) {
    const int f = min(q * NW + wave, A - 1);
    aoff[q] = static_cast<uint32_t>((min(mb0 + f, p.MB - 1) - mb0) * KB * 1024 + lane * 16);
  }
  const i32x4* bsrc[B];
#pragma unroll
  for (int j = 0; j < B; ++j)
    bsrc[j] = p.w + static_cast<int64_t>(min(nb0 + wave * B + j, p.NB - 1)) * KB * 64 + lane;

  i32x4 breg[BS][B];
  i32x4 af[2][A];
  i32x4 acc[A][B];
#pragma unroll
  for (int i = 0; i < A; ++i)
#pragma unroll
    for (int j = 0; j < B; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

  auto issue = [&](int kb, auto set_c) __attribute__((always_inline)) {
    constexpr int set = decltype(set_c)::value;
#pragma unroll
    for (int q = 0; q < LPW; ++q)
      if (q < LPW - 1 || full)
        dma16(arsrc, &ring[kb & (S - 1)][q * NW + wave][0], aoff[q] + static_cast<uint32_t>(kb) * 1024);
#pragma unroll
    for (int j = 0; j < B; ++j) breg[set][j] = bsrc[j][static_cast<int64_t>(kb) * 64];
  };
  // Loads per wavefront per k-block.
  constexpr int kLoadsFull = LPW + B;
  constexpr int kLoadsPart = LPW - 1 + B;

  static_for<D>([&](auto i) __attribute__((always_inline)) {
    if (decltype(i)::value < KB) issue(decltype(i)::value, i);
  });
  // k-block 0 has landed once only k-blocks 1 .. D-1 may be in flight.
  if (D - 1 < KB) {
    if (full) wait_vmcnt<kLoadsFull * (D - 1)>(); else wait_vmcnt<kLoadsPart * (D - 1)>();
  } else {
    wait_vmcnt<0>();
  }
  ring_barrier_tracked();
#pragma unroll
  for (int i = 0; i < A; ++i) af[0][i] = ring[0][i][lane];

  // k-block kb: make kb+1's activations visible and read them, refill the
  // slot and register set kb+1 leaves behind with k-block kb+D, then kb's
  // MFMAs.  STEADY: kb + 1 < KB is known.
  auto step = [&](int kb, auto set_c, auto cur_c, auto steady_c) __attribute__((always_inline)) {
    constexpr int set = decltype(set_c)::value;
    constexpr int nset = (set + D) % BS;
    constexpr int cur = decltype(cur_c)::value;
    constexpr bool steady = decltype(steady_c)::value;
    if (steady || kb + 1 < KB) {
      // k-block kb+1 has landed once only kb+2 .. kb+D-1 may be in flight.
      if (kb + D - 1 < KB) {
        if (full) wait_vmcnt<kLoadsFull * (D - 2)>(); else wait_vmcnt<kLoadsPart * (D - 2)>();
      } else {
        wait_vmcnt<0>();
      }
      ring_barrier_tracked();
      // Slot (kb+D) & (S-1) held k-block kb+D-S <= kb-1, read before the barrier.
      if (kb + D < KB) issue(kb + D, std::integral_constant<int, nset>{});
#pragma unroll
      for (int i = 0; i < A; ++i) af[cur ^ 1][i] = ring[(kb + 1) & (S - 1)][i][lane];
    }
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
      for (int j = 0; j < B; ++j) acc[i][j] = mfma_16x16x64(af[cur][i], breg[set][j], acc[i][j]);
  };
  // Unrolled by U, a multiple of the register-set count and of 2, so every
  // set and buffer index is static.
  constexpr int U = (BS % 2 == 0) ? BS : 2 * BS;
  int kb = 0;
  for (; kb + U < KB; kb += U) {
    static_for<U>([&](auto i) __attribute__((always_inline)) {
      constexpr int I = decltype(i)::value;
      step(kb + I, std::integral_constant<int, I % BS>{}, std::integral_constant<int, I % 2>{},
           std::true_type{});
    });
  }
  static_for<U>([&](auto i) __attribute__((always_inline)) {
    constexpr int I = decltype(i)::value;
    if (kb + I < KB)
      step(kb + I, std::integral_constant<int, I % BS>{}, std::integral_constant<int, I % 2>{},
           std::false_type{});
  });

  store_tile<1, NW, A, B, kLds, EPI, TY, TH>(p, acc, 0, wave, mb0, nb0, lane, lds);
}

// Launches the weights-direct kernel for the problem in p.
template <int NW, int A, int B, int D, int EPI, typename TY, typename TH>
hipError_t launch_wd(GemmParams p, hipStream_t st) {
  const int64_t tiles_m = ceil_div(p.MB, A);
  const int64_t tiles = tiles_m * ceil_div(p.NB, NW * B);
  if (tiles == 0) return hipSuccess;
  if (ceil_div(tiles, kXcds) * kXcds > INT32_MAX) return hipErrorInvalidConfiguration;
  p.tiles_m = static_cast<int>(tiles_m);
  p.tiles = static_cast<int>(tiles);
  p.per_xcd = static_cast<int>(ceil_div(tiles, kXcds));
  hipLaunchKernelGGL((gemm_wd_kernel<NW, A, B, D, EPI, TY, TH>), dim3(p.per_xcd * kXcds),
                     dim3(NW * 64), 0, st, p);
  return hipGetLastError();
}

// Launches one tile configuration for the problem in p (tile counts are
// filled in here).
template <int WM, int WN, int BR, int BC, int STG, int OCC, int KT, int EPI, typename TY,
          typename TH>
hipError_t launch_cfg(GemmParams p, hipStream_t st) {
  const int64_t tiles_m = ceil_div(p.MB, WM * BR);
  const int64_t tiles = tiles_m * ceil_div(p.NB, WN * BC);
  if (tiles == 0) return hipSuccess;
  if (ceil_div(tiles, kXcds) * kXcds > INT32_MAX) return hipErrorInvalidConfiguration;
  p.tiles_m = static_cast<int>(tiles_m);
  p.tiles = static_cast<int>(tiles);
  p.per_xcd = static_cast<int>(ceil_div(tiles, kXcds));
  hipLaunchKernelGGL((gemm_kernel<WM, WN, BR, BC, STG, OCC, KT, EPI, TY, TH>),
                     dim3(p.per_xcd * kXcds), dim3(WM * WN * 64), 0, st, p);
  return hipGetLastError();
}

// Tile configurations, chosen by tile count (measured on MI355X, random data,
// cold weights, LLaMA-7B projections at M = 256..2048).  A launch is fastest
// when its tiles fill one round of workgroup slots (2 per CU) as closely as
// possible, and when several rounds are needed, with the widest tile:
//   * first the one-workgroup-per-CU tiles taken when one round of them fills
//     the CUs (gemm_tile_choice): 112x256 weights-direct (gemm_wd_kernel,
//     packed QKV at M = 449..560), then 112x96 and 128x96 (O and down at
//     M = 465..640);
//   * past 64 rows (M > 64), 64x32 tiles (4 waves of 32x16, a 3-stage ring of
//     four k-blocks, 2 workgroups per CU) when they fit in one round and
//     number at least half the CUs: O and down at M = 65..128 13-16% faster
//     than the tiles below, 4-10% at M = 160..256, N = 2048 14%; beyond one
//     round (N = 8192 past M = 128) they lose;
//   * 128x128 tiles, when they fit in one round: 16 waves of 32x32, a
//     4-stage ring of one k-block (64 K), 2 workgroups per CU, when there
//     are more of them than CUs; else (one tile per CU or less, where every
//     k-step's barrier and memory latency is exposed) ring stages of several
//     k-blocks cut the barriers and keep more bytes in flight: 64x64 (4 waves
//     of 32x32, a 2-stage ring of four k-blocks, 2 per CU) when those tiles
//     fit in one round, else 128x128 with a 4-stage ring of two k-blocks,
//     one per CU (8-14% faster on O and down at M = 560..1024, 15-20% at
//     M = 384, with weights streamed from HBM).  With at most one 64x64 tile
//     per CU, 32x32 tiles of one wave (a 3-stage ring of four k-blocks, 3 per
//     CU by LDS) spread the work over more CUs when they fit in one round:
//     9-13% faster on QKV at M = 64;
//   * else the widest of 128x192, 128x224 and 128x256 whose tiles still fit
//     in one round, trying the narrowest first (8 waves of 32x96, 32x112 or
//     64x64, 3-stage ring): 128x224 takes gate/up at M = 560 in 495 tiles,
//     8% faster than 430 tiles of 128x256;
//   * else (several rounds) 128x256, except just past one round of those
//     (1 to 1.25 tiles per slot), where the few tiles of the second round cost
//     more than the wider tile saves and 128x128 is kept, and except from two
//     full rounds of 256x256 tiles (one per CU, 16 waves of 64x64, 2-stage
//     ring of two k-blocks) when those add no row padding: the square tile
//     reads a third fewer operand bytes per MAC (2048 x 22016 x 4096: 1.94
//     against 1.71 POPS; 8192^3: 2.03 against 1.99), while at 1.3-1.5 rounds
//     it gains nothing.
template <int EPI, typename TY, typename TH>
hipError_t launch_t(const GemmParams& p, hipStream_t st) {
  switch (gemm_tile_choice(p.MB, p.NB, cu_count())) {
    case kGemmTinyDeep:
      return launch_cfg<1, 1, 2, 2, 3, 4, 4, EPI, TY, TH>(p, st);
    case kGemmSmallDeep:
      return launch_cfg<2, 2, 2, 2, 2, 2, 4, EPI, TY, TH>(p, st);
    case kGemmBigDeep:
      return launch_cfg<4, 4, 2, 2, 4, 1, 2, EPI, TY, TH>(p, st);
    case kGemmBig:
      return launch_cfg<4, 4, 2, 2, 4, 2, 1, EPI, TY, TH>(p, st);
    case kGemmW192:
      return launch_cfg<4, 2, 2, 6, 3, 2, 1, EPI, TY, TH>(p, st);
    case kGemmW224:
      return launch_cfg<4, 2, 2, 7, 3, 2, 1, EPI, TY, TH>(p, st);
    case kGemmW256Sq:
      return launch_cfg<4, 4, 4, 4, 2, 1, 2, EPI, TY, TH>(p, st);
    case kGemmMid:
      return launch_cfg<2, 2, 2, 1, 3, 2, 4, EPI, TY, TH>(p, st);
    case kGemmWd7x2:
      return launch_wd<8, 7, 2, 4, EPI, TY, TH>(p, st);
    case kGemmT112x96:
      return launch_cfg<7, 2, 1, 3, 3, 1, 3, EPI, TY, TH>(p, st);
    case kGemmT128x96:
      return launch_cfg<4, 2, 2, 3, 2, 1, 4, EPI, TY, TH>(p, st);
    default:
      return launch_cfg<2, 4, 4, 4, 3, 2, 1, EPI, TY, TH>(p, st);
  }
}

}  // namespace

int gemm_tile_choice(int64_t MB, int64_t NB, int64_t cus) {
  // The 112 x 256 weights-direct tile when one round of it (one workgroup per
  // CU) fills at least 85% of the CUs with at least 85% of the tile rows in
  // use (the packed QKV at M = 449..560).  A 144 x 64 weights-direct tile for
  // O and down at the same M measured slower than the 128 x 128 deep ring
  // (27.2 vs 23.5 us and 59.6 vs 51.3 us with the fp16 epilogue), so those
  // keep the LDS-ring tiles.
  if (MB > 4) {
    const int64_t tm = ceil_div(MB, 7);
    const int64_t tiles = tm * ceil_div(NB, 16);
    if (tiles <= cus && 100 * tiles >= 85 * cus && 100 * MB >= 85 * tm * 7) return kGemmWd7x2;
  }
  // Narrow tiles (96 columns) when one round of them, at least four tile rows
  // deep, fills at least 80% of the CUs with at least 85% of the tile rows in
  // use: O and down (N = 4096) at M = 465..640, where 128x128 tiles leave 96
  // of 256 CUs idle.  Measured at M = 560 (fp16 epilogue): 112x96 takes O in
  // 20.8 against 23.6 us and down in 48.1 against 58.5 us; at M = 567 (36
  // row blocks) 128x96 takes O in 21.6 against 23.8 us.  The 14 wavefronts of
  // 112x96 each own a 16-row strip.
  if (MB > 4) {
    auto one_round = [&](int64_t rows, int64_t cols) {
      const int64_t tm = ceil_div(MB, rows);
      const int64_t tiles = tm * ceil_div(NB, cols);
      return tm >= 4 && tiles <= cus && 100 * tiles >= 80 * cus && 100 * MB >= 85 * tm * rows;
    };
    if (one_round(7, 6)) return kGemmT112x96;
    if (one_round(8, 6)) return kGemmT128x96;
  }
  const int64_t slots = cus * 2;
  const int64_t tiles_m = ceil_div(MB, 8);  // 128-row tiles
  const int64_t big_tiles = tiles_m * ceil_div(NB, 8);
  if (big_tiles <= slots) {
    const int64_t mid_tiles = ceil_div(MB, 4) * ceil_div(NB, 2);
    if (MB > 4 && 2 * mid_tiles >= cus && mid_tiles <= slots) return kGemmMid;
    if (big_tiles > cus) return kGemmBig;
    const int64_t small_tiles = ceil_div(MB, 4) * ceil_div(NB, 4);
    if (small_tiles <= cus && ceil_div(MB, 2) * ceil_div(NB, 2) <= 3 * cus) return kGemmTinyDeep;
    if (small_tiles <= slots) return kGemmSmallDeep;
    return kGemmBigDeep;
  }
  if (tiles_m * ceil_div(NB, 12) <= slots) return kGemmW192;
  if (tiles_m * ceil_div(NB, 14) <= slots) return kGemmW224;
  const int64_t wide_tiles = tiles_m * ceil_div(NB, 16);
  const bool short_second_round = wide_tiles > slots && wide_tiles * 100 < slots * 125;
  if (short_second_round) return kGemmBig;
  const int64_t sq_tiles_m = ceil_div(MB, 16);
  if (sq_tiles_m * ceil_div(NB, 16) >= 2 * cus && sq_tiles_m * 2 == tiles_m) return kGemmW256Sq;
  return kGemmW256;
}

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
  p.absmax_parts = op.absmax_parts;
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
