// Decode-regime W8A8 GEMV (M <= 32, or M <= 64 with N <= 12288):
// y[m, n] = epi(sum_k xq[m, k] * wq[n, k]).
//
// Replaces the F.linear call sites of the decode path
// (llama/paged_attention.py:97-124, llama/lightweight_runner.py:38-54,
// 329-379) for the int8 contract of integer_linear_per_output_reference
// (nanopointllm/compression/w8a8.py:118-139).
//
// Design (HBM-bound): one workgroup per NBW 16-output blocks of packed
// weights.  Its WAVES wavefronts split K into contiguous k-block ranges, so each wave
// streams a contiguous slab of the block's 16 x K packed tile column with
// fully coalesced 1 KiB global_load_dwordx4 (one MFMA B fragment per load),
// double-buffered CH fragments deep in registers.  The activation fragment of
// each k-block (16 rows x 64 int8) comes from the L2-resident quantized
// activations and serves the NBW blocks' fragments of that k-block (past 16
// rows the activation bytes outnumber the weight bytes, so sharing them across
// blocks cuts the L2 traffic NBW-fold).  v_mfma_i32_16x16x64_i8 does the int8 dot products (16 cycles of
// the matrix pipe per KiB of weights, so the VALU stays free), then the
// per-wave 16x16 int32 partial tiles are summed through LDS and the fused
// epilogue (dequant / SiLU*mul / int8 requant) writes the outputs.
#include "w8a8_internal.h"

namespace w8a8 {

namespace {

struct GemvParams {
  const int8_t* xq;
  int64_t ldq;
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
  int KB;
  int NB;
};

__device__ inline i32x4 mfma_16x16x64(i32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

template <int WAVES, int MT, int CH, int NBW, int EPI, typename TY, typename TH>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(GemvParams p) {
  constexpr int NT = WAVES * 64;
  constexpr int TB = MT * 256;  // int32 partials of one block per wave
  __shared__ int32_t red[WAVES][NBW * TB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int64_t nb0 = static_cast<int64_t>(blockIdx.x) * NBW;
  const int KB = p.KB;
  const int kb_begin = (KB * wave) / WAVES;
  const int kb_end = (KB * (wave + 1)) / WAVES;

  // Blocks past the last one (a partial group) re-read the last block: their
  // products are never stored.
  const i32x4* wt[NBW];
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    const int64_t nb = nb0 + j < p.NB ? nb0 + j : p.NB - 1;
    wt[j] = p.w + nb * KB * 64 + lane;
  }
  const int8_t* arow[MT];
  bool alive[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + li;
    alive[mt] = m < p.M;
    arow[mt] = p.xq + static_cast<int64_t>(alive[mt] ? m : 0) * p.ldq + lg * 16;
  }

  i32x4 acc[NBW][MT];
#pragma unroll
  for (int j = 0; j < NBW; ++j)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[j][mt] = i32x4{0, 0, 0, 0};

  i32x4 wb0[NBW][CH], wb1[NBW][CH];
  i32x4 ab0[MT][CH], ab1[MT][CH];

  // Loads CH k-blocks starting at kc.  Indices past the wave's range are
  // clamped to its last k-block (an in-bounds, cache-hot address); their
  // MFMAs are skipped in compute().
  auto load = [&](i32x4(&wb)[NBW][CH], i32x4(&ab)[MT][CH], int kc) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int kb = (kc + c < kb_end) ? kc + c : kb_end - 1;
#pragma unroll
      for (int j = 0; j < NBW; ++j)
        wb[j][c] = __builtin_nontemporal_load(wt[j] + static_cast<int64_t>(kb) * 64);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        ab[mt][c] = alive[mt] ? *reinterpret_cast<const i32x4*>(arow[mt] + kb * 64)
                              : i32x4{0, 0, 0, 0};
      }
    }
  };
  auto compute = [&](const i32x4(&wb)[NBW][CH], const i32x4(&ab)[MT][CH], int kc) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      if (kc + c < kb_end) {
#pragma unroll
        for (int j = 0; j < NBW; ++j)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[j][mt] = mfma_16x16x64(ab[mt][c], wb[j][c], acc[j][mt]);
      }
    }
  };

  if (kb_begin < kb_end) {
    load(wb0, ab0, kb_begin);
    for (int kc = kb_begin; kc < kb_end; kc += 2 * CH) {
      const bool second = kc + CH < kb_end;
      if (second) load(wb1, ab1, kc + CH);
      compute(wb0, ab0, kc);
      if (second) {
        if (kc + 2 * CH < kb_end) load(wb0, ab0, kc + 2 * CH);
        compute(wb1, ab1, kc + CH);
      }
    }
  }

  // C layout of v_mfma_i32_16x16x64_i8: lane (li, lg), register r holds
  // row 4*lg + r (activation row) and column li (output within the block).
#pragma unroll
  for (int j = 0; j < NBW; ++j)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        red[wave][j * TB + mt * 256 + (4 * lg + r) * 16 + li] = acc[j][mt][r];
    }
  __syncthreads();

  if constexpr (EPI == kEpiI32 || EPI == kEpiDequant || EPI == kEpiRequant ||
                EPI == kEpiBf16Exact) {
    for (int e = tid; e < NBW * TB; e += NT) {
      const int m = ((e % TB) >> 8) * 16 + ((e & 255) >> 4);
      const int64_t nb = nb0 + e / TB;
      const int64_t n = nb * 16 + (e & 15);
      if (m >= p.M || nb >= p.NB || n >= p.N) continue;
      int32_t s = 0;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) s += red[w][e];
      TY* y = static_cast<TY*>(p.y) + static_cast<int64_t>(m) * p.ldy + n;
      if constexpr (EPI == kEpiI32) {
        *y = s;
      } else if constexpr (EPI == kEpiRequant) {
        *y = static_cast<int8_t>(
            requant1(s, p.rq_bias != nullptr ? p.rq_bias[n] : 0, p.rq_mult[n], p.rq_shift[n]));
      } else if constexpr (EPI == kEpiBf16Exact) {
        *y = __builtin_bit_cast(TY, dequant_bf16_exact(s, f16_bits(p.sx[m]), f16_bits(p.sw[n])));
      } else {
        *y = from_f32<TY>(dequant1(s, p.sx[m], p.sw[n], p.bias, n));
      }
    }
  } else {
    // Interleaved gate/up: packed rows 2c (gate) and 2c+1 (up) of this block
    // produce output column nb*8 + c.
    const int64_t n_out_total = p.N / 2;
    // NBW * MT * 128 and NT are multiples of 64, so every wavefront runs the
    // same trip count and the shuffles below run in uniform control flow.
    for (int e = tid; e < NBW * MT * 128; e += NT) {
      const int j = e / (MT * 128);
      const int mt = (e % (MT * 128)) >> 7;
      const int i = (e & 127) >> 3;
      const int c = e & 7;
      const int m = mt * 16 + i;
      const int64_t nb = nb0 + j;
      const int64_t n_out = nb * 8 + c;
      float habs = 0.0f;
      if (m < p.M && nb < p.NB && n_out < n_out_total) {
        const int base = j * TB + mt * 256 + i * 16 + 2 * c;
        int32_t sg = 0, su = 0;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
          sg += red[w][base];
          su += red[w][base + 1];
        }
        const int64_t ng = nb * 16 + 2 * c;
        const float sxm = p.sx[m];
        const float g = to_f32(from_f32<TH>(dequant1(sg, sxm, p.sw[ng], p.bias, ng)));
        const float u = to_f32(from_f32<TH>(dequant1(su, sxm, p.sw[ng + 1], p.bias, ng + 1)));
        const TH h = from_f32<TH>(silu_mul<TH>(g, u));
        TY* y = static_cast<TY*>(p.y) + static_cast<int64_t>(m) * p.ldy + n_out;
        if constexpr (EPI == kEpiSilu) {
          *y = h;
          habs = fabsf(to_f32(h));
        } else {
          *y = static_cast<int8_t>(quant1(to_f32(h), p.out_scale));
        }
      }
      if constexpr (EPI == kEpiSilu) {
        if (p.absmax_parts != nullptr) {
          // Row m's 8 outputs of this block sit in 8 consecutive lanes.
#pragma unroll
          for (int off = 1; off < 8; off <<= 1) habs = fmaxf(habs, __shfl_xor(habs, off));
          if (c == 0 && m < p.M && nb < p.NB)
            p.absmax_parts[static_cast<int64_t>(m) * p.NB + nb] = habs;
        }
      }
    }
  }
}

template <int WAVES, int MT, int CH, int EPI, typename TY, typename TH, int NBW = 1>
hipError_t launch_cfg(const GemvParams& p, int64_t nblocks, hipStream_t st) {
  hipLaunchKernelGGL((gemv_kernel<WAVES, MT, CH, NBW, EPI, TY, TH>),
                     dim3(static_cast<unsigned>(ceil_div(nblocks, NBW))), dim3(WAVES * 64), 0,
                     st, p);
  return hipGetLastError();
}

// Launch shape.  Few output blocks (O / down: 256 blocks for 256 CUs) get
// 16 wavefronts per block so every CU keeps ~64 KiB of weight loads in
// flight; many blocks (QKV, gate/up) use 4 wavefronts and several resident
// blocks per CU.  Past 16 rows many blocks are taken three per workgroup (8
// wavefronts, one k-block per step), so each activation fragment serves
// three weight fragments: measured on MI355X (quantize + GEMV, LLaMA-7B),
// QKV at M = 17 / 24 / 32 in 14.2 / 14.9 / 15.8 us against 17.5 / 19.8 /
// 22.3 with one block per workgroup, gate/up 21.0 / 22.7 / 24.5 against
// 27.0 / 32.0 / 37.1, QKV at M = 48 / 64 18.7 / 20.6 against 27.5 / 33.1.
template <int EPI, typename TY, typename TH>
hipError_t launch_mt(const GemvParams& p, int64_t nblocks, hipStream_t st) {
  const bool few = nblocks <= 512;
  if (p.M <= 16)
    return few ? launch_cfg<16, 1, 4, EPI, TY, TH>(p, nblocks, st)
               : launch_cfg<4, 1, 8, EPI, TY, TH>(p, nblocks, st);
  if (p.M <= 32)
    return few ? launch_cfg<8, 2, 4, EPI, TY, TH>(p, nblocks, st)
               : launch_cfg<8, 2, 1, EPI, TY, TH, 3>(p, nblocks, st);
  return few ? launch_cfg<8, 4, 2, EPI, TY, TH>(p, nblocks, st)
             : launch_cfg<8, 4, 1, EPI, TY, TH, 3>(p, nblocks, st);
}

}  // namespace

hipError_t launch_gemv(const LinearOperands& op, hipStream_t st) {
  GemvParams p;
  p.xq = op.a;
  p.ldq = op.lda;
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
  p.KB = static_cast<int>(ceil_div(op.K, kTileK));
  const int64_t nblocks = ceil_div(op.N, kTileRows);
  p.NB = static_cast<int>(nblocks);
  if (op.M <= 0 || nblocks == 0) return hipSuccess;
  if (fused_gemv_i8_supported(op.M, op.N, op.K, op.lda, op.epi)) return launch_gemv_fused_i8(op, st);
  switch (op.epi) {
    case kEpiI32:
      return launch_mt<kEpiI32, int32_t, float>(p, nblocks, st);
    case kEpiDequant:
      if (op.y_dtype == kF16) return launch_mt<kEpiDequant, __half, float>(p, nblocks, st);
      if (op.y_dtype == kBF16) return launch_mt<kEpiDequant, __hip_bfloat16, float>(p, nblocks, st);
      if (op.y_dtype == kF32) return launch_mt<kEpiDequant, float, float>(p, nblocks, st);
      return hipErrorInvalidValue;
    case kEpiSilu:
      if (op.y_dtype == kF16) return launch_mt<kEpiSilu, __half, __half>(p, nblocks, st);
      if (op.y_dtype == kBF16)
        return launch_mt<kEpiSilu, __hip_bfloat16, __hip_bfloat16>(p, nblocks, st);
      return hipErrorInvalidValue;
    case kEpiSiluQ8:
      if (op.h_dtype == kF16) return launch_mt<kEpiSiluQ8, int8_t, __half>(p, nblocks, st);
      if (op.h_dtype == kBF16) return launch_mt<kEpiSiluQ8, int8_t, __hip_bfloat16>(p, nblocks, st);
      return hipErrorInvalidValue;
    case kEpiRequant:
      return launch_mt<kEpiRequant, int8_t, float>(p, nblocks, st);
    case kEpiBf16Exact:
      return launch_mt<kEpiBf16Exact, __hip_bfloat16, float>(p, nblocks, st);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace w8a8
