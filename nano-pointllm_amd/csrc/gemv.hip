// Decode-regime W8A8 GEMV (M <= 32, or M <= 64 with N <= 12288):
// y[m, n] = epi(sum_k xq[m, k] * wq[n, k]).  gemv_kernel below serves every
// shape; at 17..64 rows with K <= 4096 the persistent gemv_rows_kernel
// (further below) takes over.
//
// Replaces the F.linear call sites of the decode path
// (llama/paged_attention.py:97-124, llama/lightweight_runner.py:38-54,
// 329-379) for the int8 contract of integer_linear_per_output_reference
// (nanopointllm/compression/w8a8.py:118-139).
//
// gemv_kernel (HBM-bound): one workgroup per NBW 16-output blocks of packed
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
  // kEpiDequant (gemv_kernel only, nullable): the residual-add epilogue and
  // its RMSNorm chunk sums (LinearOperands::res / ss_parts).
  const void* res;
  int64_t ld_res;
  float* ss_parts;
  int64_t ld_parts;
  int M;
  int N;
  int KB;
  int NB;
  int G;  // gemv_rows_kernel: workgroups, balanced_grid(NB)
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

  // Residual-add epilogue: the residual of this thread's first output is
  // requested before the weights, so the epilogue does not wait a memory
  // round trip for it (later outputs, when a thread has several, load then).
  [[maybe_unused]] TY res_first{};
  if constexpr (EPI == kEpiDequant) {
    if (p.res != nullptr && tid < NBW * TB) {
      const int m = ((tid % TB) >> 8) * 16 + ((tid & 255) >> 4);
      const int64_t nb = nb0 + tid / TB;
      const int64_t n = nb * 16 + (tid & 15);
      if (m < p.M && nb < p.NB && n < p.N) res_first = static_cast<const TY*>(p.res)[m * p.ld_res + n];
    }
  }

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
      if constexpr (EPI == kEpiDequant) {
        if (p.res != nullptr) {
          // Residual-add epilogue: the chunk sums need every lane, so no lane
          // leaves before them (NBW * TB and NT are multiples of 64).
          const bool ok = m < p.M && nb < p.NB && n < p.N;
          float v = 0.0f;
          if (ok) {
            int32_t s = 0;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) s += red[w][e];
            const TY r = e == tid ? res_first : static_cast<const TY*>(p.res)[m * p.ld_res + n];
            const TY o = add_rounded(from_f32<TY>(dequant1(s, p.sx[m], p.sw[n], p.bias, n)), r);
            static_cast<TY*>(p.y)[static_cast<int64_t>(m) * p.ldy + n] = o;
            v = to_f32(o);
          }
          if (p.ss_parts != nullptr) {
            const float cs = chunk_sumsq8(v);
            if ((e & 7) == 0 && ok) p.ss_parts[m * p.ld_parts + (n >> 3)] = cs;
          }
          continue;
        }
      }
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

// Batched decode, 17..64 rows with K <= 4096 (gemv_rows_kernel): a
// persistent grid of at most one 16-wavefront workgroup per CU
// (G = balanced_grid(NB)); workgroup b takes 16-output blocks b, b + G,
// b + 2G, ...  Wavefront w owns
// the k-blocks [w kbw, (w + 1) kbw) of every block (kbw = ceil(KB / 16) <=
// KBW = 4), so it loads the x fragments of its k-range (MT row tiles of 16
// rows x 64 K, 16 bytes per lane) into registers once and keeps them for the
// whole launch: every x byte crosses from L2 into the CU once, and the weight
// stream never waits on an activation load.  The weights stream through a
// ring of RING register buffers of CH fragments (one step = CH k-blocks of
// one block, RING - 1 steps in flight), loaded with raw buffer loads whose
// range ends at the wavefront's last k-block (zeros past it, no memory
// access).  Per block the wavefront partials go through one of two LDS
// buffers, one barrier, and the epilogue.  Measured on MI355X against
// gemv_kernel (int8 x, LLaMA-7B shapes, cold weights): QKV at M = 17 / 32 /
// 64 in 10.8 / 11.9 / 16.6 us against 11.0 / 12.4 / 17.0, gate/up + SiLU*mul
// at M = 17 / 32 in 17.6 / 19.0 against 18.1 / 21.4, O at M = 32 / 64 in
// 7.4 / 10.7 against 7.9 / 12.0, and gate/up at M = 48 / 64 in 22.9 / 24.8
// against 26.2 / 27.3 on the GEMM after a packing pass (x in fragment
// loads; with x in whole lines and the quantization in front, gate/up at
// M = 48 / 64 takes 24.2 / 25.4 us here against 26.5 / 27.2 on the GEMM).
constexpr int kRowsWaves = 16;
constexpr int kRowsThreads = kRowsWaves * 64;
constexpr int kRowsMaxBlocks = 64;  // blocks per workgroup: N <= 1024 * CUs
constexpr int kRowsKBW = 4;         // k-blocks per wavefront: K <= 4096
constexpr int kBufferWord3 = 0x00020000;
constexpr int kCacheNT = 2;         // weights: nontemporal (read once)

template <typename F, int... I>
__device__ inline void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
constexpr int gcd_i(int a, int b) { return b == 0 ? a : gcd_i(b, a % b); }

// Requires p.G workgroups of kRowsThreads, M <= 16 MT, KB <= 16 KBW, at most
// kRowsMaxBlocks blocks per workgroup and (M - 1) * ldq + 64 KB < 2^31; xq
// readable and zero past K up to 64 KB bytes per row.  Epilogues: int32,
// dequant, SiLU*mul (with the per-block row maxima) and its int8 requant.
template <int MT, int CH, int RING, int EPI, typename TY, typename TH>
__global__ __launch_bounds__(kRowsThreads) void gemv_rows_kernel(GemvParams p) {
  static_assert(EPI == kEpiI32 || EPI == kEpiDequant || EPI == kEpiSilu || EPI == kEpiSiluQ8,
                "gemv_rows_kernel epilogue");
  constexpr int KBW = kRowsKBW;
  constexpr int NCH = KBW / CH;  // steps per block
  static_assert(NCH * CH == KBW && RING >= 2, "ring shape");
  // Unrolled by U steps, a multiple of RING and of NCH, so every ring slot
  // and chunk index is static.
  constexpr int U = RING * NCH / gcd_i(RING, NCH);
  constexpr int TB = MT * 256;  // int32 partials of one block per wavefront
  constexpr bool kHalfCols = EPI == kEpiSilu || EPI == kEpiSiluQ8;
  __shared__ int32_t red[2][kRowsWaves][TB];
  __shared__ float ops_lds[kRowsMaxBlocks * 32];  // per block: 16 scales, 16 biases
  __shared__ float row_s[MT * 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave-uniform, so the step bookkeeping stays in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int KB = p.KB;
  const int M = p.M;
  const int kbw = (KB + kRowsWaves - 1) / kRowsWaves;
  const int kb0 = min(wave * kbw, KB);
  const int kb1 = min(kb0 + kbw, KB);
  const int n_mine = (p.NB - static_cast<int>(blockIdx.x) + p.G - 1) / p.G;
  const int total = n_mine * NCH;

  // x fragment (mt, i): rows 16 mt + li, bytes 64 (kb0 + i) + 16 lg, the A
  // operand of k-block kb0 + i.  It is read from memory in whole 128-byte
  // lines, not in the fragment's 16 rows x 64 bytes: line c of the wave's
  // range (k-blocks kb0 + 2c, kb0 + 2c + 1) of 8 rows per load, lane l taking
  // row l / 8 and bytes 16 (l % 8).  A load of half lines costs the CU's
  // memory pipeline about as much as one of whole lines, so this halves the
  // cost of x (measured on MI355X: 256 KiB of L2-resident rows per CU, as at
  // M = 64, in 4.7 against 8.2 us; with 192 KiB of cold weights behind them,
  // 13.5 against 16.4 us).  The lines go through this wavefront's own slice
  // of the partial buffers (free until the first block's epilogue, behind the
  // barrier below), two passes of one line per row, and come back as
  // fragments.  The descriptor's range ends with row M-1's 64 KB bytes; rows
  // past M and lines past the wave's range get an offset beyond it and read
  // zeros without a memory access; the second k-block of a line may lie past
  // the wave's range (its fragment is never multiplied).
  i32x4 xa[MT][KBW];
  static_assert(KBW == 4, "two lines per row");
  u32x4 xl[2][2 * MT];
  {
    const int xrec = __builtin_amdgcn_readfirstlane(static_cast<int>((M - 1) * p.ldq) + KB * 64);
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(p.xq), 0, xrec, kBufferWord3);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int g = 0; g < 2 * MT; ++g) {
        const int m = 8 * g + (lane >> 3);
        const int kb = kb0 + 2 * c;
        const int off = (m < M && kb < kb1)
                            ? static_cast<int>(m * p.ldq) + kb * 64 + (lane & 7) * 16
                            : 0x7ffffff0;
        xl[c][g] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
      }
  }
  // The epilogue operands of all this workgroup's blocks (one per thread) and
  // the row scales go to LDS up front: a load at epilogue time would wait
  // for every weight load in flight (vmcnt counts loads in issue order).
  float op_s = 0.0f, op_b = 0.0f, sxr = 0.0f;
  const int op_j = tid >> 4;
  if constexpr (EPI != kEpiI32) {
    const int64_t n =
        (static_cast<int64_t>(blockIdx.x) + static_cast<int64_t>(op_j) * p.G) * 16 + (tid & 15);
    if (op_j < n_mine && n < p.N) {
      op_s = p.sw[n];
      if (p.bias != nullptr) op_b = p.bias[n];
    }
    if (tid < M) sxr = p.sx[tid];
  }

  i32x4 rb[RING][CH];
  // Loads step t (block t / NCH, chunk C = t % NCH) into buf.  A step past
  // the wave's blocks gets an empty range (zeros, no memory access).
  auto issue = [&](i32x4(&buf)[CH], int t, auto c_c) __attribute__((always_inline)) {
    constexpr int C = decltype(c_c)::value;
    const int j = t / NCH;
    const bool past = j >= n_mine;
    const int sj = __builtin_amdgcn_readfirstlane(past ? n_mine - 1 : j);
    const int nrec = __builtin_amdgcn_readfirstlane(past ? 0 : kb1 * 1024);
    const int64_t nb = static_cast<int64_t>(blockIdx.x) + static_cast<int64_t>(sj) * p.G;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<i32x4*>(p.w + nb * KB * 64), 0, nrec, kBufferWord3);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int off = (kb0 + C * CH + i) * 1024 + lane * 16;
      buf[i] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCacheNT));
    }
  };
  static_for<RING - 1>([&](auto u) __attribute__((always_inline)) {
    constexpr int I = decltype(u)::value;
    issue(rb[I], I, std::integral_constant<int, I % NCH>{});
  });
  if (op_j < n_mine) {
    ops_lds[op_j * 32 + (tid & 15)] = op_s;
    ops_lds[op_j * 32 + 16 + (tid & 15)] = op_b;
  }
  if (tid < M) row_s[tid] = sxr;
  {
    // x lines -> fragments through the wavefront's slice (MT x 2 KiB) of red:
    // line slot g holds 8 rows x 128 bytes in lane order.  Fragment (mt, 2c +
    // h) of lane l is row 16 mt + li = 8 g + r (g = 2 mt + li / 8) at bytes
    // 64 h + 16 lg of the line: lane 8 r + 4 h + lg of slot g.
    int8_t* slice = reinterpret_cast<int8_t*>(&red[0][0][0]) + wave * (MT * 2048);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
      for (int g = 0; g < 2 * MT; ++g)
        *reinterpret_cast<u32x4*>(slice + g * 1024 + lane * 16) = xl[c][g];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          xa[mt][2 * c + h] = *reinterpret_cast<const i32x4*>(
              slice + (2 * mt + (li >> 3)) * 1024 + (8 * (li & 7) + 4 * h + lg) * 16);
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
  }
  // Every wavefront is done with its slice before any epilogue writes red.
  __syncthreads();

  i32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = i32x4{0, 0, 0, 0};
  const bool has_bias = p.bias != nullptr;

  // Block j's epilogue over the partials in red[par].
  auto finish = [&](int j, int par) __attribute__((always_inline)) {
    const int64_t nb = static_cast<int64_t>(blockIdx.x) + static_cast<int64_t>(j) * p.G;
    const float* ops = ops_lds + j * 32;
    if constexpr (!kHalfCols) {
      // Partial index e = 16 m + column; 16 m < TB.
      for (int e = tid; e < TB; e += kRowsThreads) {
        const int m = e >> 4;
        const int r = e & 15;
        const int64_t n = nb * 16 + r;
        if (m < M && n < p.N) {
          int32_t s = 0;
#pragma unroll
          for (int w = 0; w < kRowsWaves; ++w) s += red[par][w][e];
          TY* y = static_cast<TY*>(p.y) + static_cast<int64_t>(m) * p.ldy + n;
          if constexpr (EPI == kEpiI32) {
            *y = s;
          } else {
            *y = from_f32<TY>(dequant1b(s, row_s[m], ops[r], has_bias, ops[16 + r]));
          }
        }
      }
    } else {
      // Interleaved gate/up: packed rows 2c (gate) and 2c+1 (up) of the block
      // give output column 8 nb + c.  Thread e2 takes row e2 / 4 and the
      // outputs 2 (e2 % 4) and 2 (e2 % 4) + 1, reading their four partials
      // at once; TB / 4 is a multiple of 64, so whole wavefronts take part
      // and the shuffles below run in uniform control flow.
      const int64_t n_out_total = p.N / 2;
      if (tid < TB / 4) {
        const int e2 = tid;
        const int m = e2 >> 2;
        const int cc0 = (e2 & 3) * 2;
        const int base = m * 16 + 2 * cc0;
        i32x4 s = {0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < kRowsWaves; ++w) s += *reinterpret_cast<const i32x4*>(&red[par][w][base]);
        float habs = 0.0f;
        if (m < M) {
          const float sxm = row_s[m];
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            const int cc = cc0 + h2;
            const int64_t n_out = nb * 8 + cc;
            if (n_out < n_out_total) {
              const float g = to_f32(from_f32<TH>(
                  dequant1b(s[2 * h2], sxm, ops[2 * cc], has_bias, ops[16 + 2 * cc])));
              const float u = to_f32(from_f32<TH>(
                  dequant1b(s[2 * h2 + 1], sxm, ops[2 * cc + 1], has_bias, ops[17 + 2 * cc])));
              const TH h = from_f32<TH>(silu_mul<TH>(g, u));
              TY* y = static_cast<TY*>(p.y) + static_cast<int64_t>(m) * p.ldy + n_out;
              if constexpr (EPI == kEpiSilu) {
                *y = h;
                habs = fmaxf(habs, fabsf(to_f32(h)));
              } else {
                *y = static_cast<int8_t>(quant1(to_f32(h), p.out_scale));
              }
            }
          }
        }
        if constexpr (EPI == kEpiSilu) {
          if (p.absmax_parts != nullptr) {
            // Row m's 8 outputs of this block sit in 4 consecutive lanes.
            habs = fmaxf(habs, __shfl_xor(habs, 1));
            habs = fmaxf(habs, __shfl_xor(habs, 2));
            if ((e2 & 3) == 0 && m < M) p.absmax_parts[static_cast<int64_t>(m) * p.NB + nb] = habs;
          }
        }
      }
    }
  };

  for (int t0 = 0; t0 < total; t0 += U) {
    static_for<U>([&](auto u) __attribute__((always_inline)) {
      constexpr int I = decltype(u)::value;
      constexpr int slot = I % RING;
      constexpr int C = I % NCH;
      const int t = t0 + I;
      // Refill the buffer the previous step used, then this step's MFMAs.
      issue(rb[(I + RING - 1) % RING], t + RING - 1, std::integral_constant<int, (I + RING - 1) % NCH>{});
      const bool live = t < total;
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        if (live && kb0 + C * CH + i < kb1) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma_16x16x64(xa[mt][C * CH + i], rb[slot][i], acc[mt]);
        }
      }
      if (live && C == NCH - 1) {
        // Block j done.  Two partial buffers: a wavefront writing block j+2's
        // partials has passed block j+1's barrier, so every thread has
        // finished block j's epilogue.  The barrier waits for LDS traffic
        // only; the weight loads in flight keep streaming across it.
        const int j = t / NCH;
        const int par = j & 1;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) red[par][wave][mt * 256 + (4 * lg + r) * 16 + li] = acc[mt][r];
          acc[mt] = i32x4{0, 0, 0, 0};
        }
        __syncthreads();
        finish(j, par);
      }
    });
  }
}

template <int MT, int CH, int RING, int EPI, typename TY, typename TH>
hipError_t launch_rows(const GemvParams& p, hipStream_t st) {
  hipLaunchKernelGGL((gemv_rows_kernel<MT, CH, RING, EPI, TY, TH>), dim3(p.G), dim3(kRowsThreads),
                     0, st, p);
  return hipGetLastError();
}

// Ring shape by row tiles: two (M <= 32) stream steps of four k-blocks, three
// in flight, or of two when a CU has a single block (O at M = 32: 7.4
// against 8.1 us); four (M <= 64) one k-block per step, four in flight, to
// keep the registers of the 16 x fragments.
template <int EPI, typename TY, typename TH>
hipError_t launch_rows_m(const GemvParams& p, hipStream_t st) {
  if (p.M <= 32)
    return p.NB > p.G ? launch_rows<2, 4, 3, EPI, TY, TH>(p, st)
                      : launch_rows<2, 2, 4, EPI, TY, TH>(p, st);
  return launch_rows<4, 1, 4, EPI, TY, TH>(p, st);
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

// Whether launch_gemv takes gemv_rows_kernel: 17..64 rows, K <= 4096,
// row-major activations with leading dimension lda, the int32 / dequant /
// SiLU*mul epilogues.
bool gemv_rows_supported(int64_t M, int64_t N, int64_t K, int64_t lda, int epi) {
  if (!(M > 16 && M <= kGemvMaxRows && K >= 1 && N >= 1)) return false;
  if (!(epi == kEpiI32 || epi == kEpiDequant || epi == kEpiSilu || epi == kEpiSiluQ8)) return false;
  const int64_t kb = ceil_div(K, kTileK);
  if (kb > kRowsWaves * kRowsKBW || lda < kb * kTileK) return false;
  if ((M - 1) * lda + kb * kTileK >= (int64_t{1} << 31)) return false;
  const int64_t nb = ceil_div(N, kTileRows);
  const int64_t g = nb < cu_count() ? nb : cu_count();
  return ceil_div(nb, g) <= kRowsMaxBlocks;
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
  p.res = op.res;
  p.ld_res = op.ld_res;
  p.ss_parts = op.ss_parts;
  p.ld_parts = op.ld_parts;
  p.M = static_cast<int>(op.M);
  p.N = static_cast<int>(op.N);
  p.KB = static_cast<int>(ceil_div(op.K, kTileK));
  const int64_t nblocks = ceil_div(op.N, kTileRows);
  p.NB = static_cast<int>(nblocks);
  p.G = balanced_grid(nblocks);  // gate/up at M = 17..64: 0.3-0.5 us faster
  if (op.M <= 0 || nblocks == 0) return hipSuccess;
  if (fused_gemv_i8_supported(op.M, op.N, op.K, op.lda, op.epi)) return launch_gemv_fused_i8(op, st);
  if (op.res == nullptr && gemv_rows_supported(op.M, op.N, op.K, op.lda, op.epi)) {
    switch (op.epi) {
      case kEpiI32:
        return launch_rows_m<kEpiI32, int32_t, float>(p, st);
      case kEpiDequant:
        if (op.y_dtype == kF16) return launch_rows_m<kEpiDequant, __half, float>(p, st);
        if (op.y_dtype == kBF16) return launch_rows_m<kEpiDequant, __hip_bfloat16, float>(p, st);
        if (op.y_dtype == kF32) return launch_rows_m<kEpiDequant, float, float>(p, st);
        return hipErrorInvalidValue;
      case kEpiSilu:
        if (op.y_dtype == kF16) return launch_rows_m<kEpiSilu, __half, __half>(p, st);
        if (op.y_dtype == kBF16)
          return launch_rows_m<kEpiSilu, __hip_bfloat16, __hip_bfloat16>(p, st);
        return hipErrorInvalidValue;
      case kEpiSiluQ8:
        if (op.h_dtype == kF16) return launch_rows_m<kEpiSiluQ8, int8_t, __half>(p, st);
        if (op.h_dtype == kBF16) return launch_rows_m<kEpiSiluQ8, int8_t, __hip_bfloat16>(p, st);
        return hipErrorInvalidValue;
      default:
        return hipErrorInvalidValue;
    }
  }
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
