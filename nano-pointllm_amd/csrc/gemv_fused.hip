// Decode W8A8 linear with the per-token quantization fused in (M <= 8).
//
// One launch replaces quantize_symmetric(x, scale_from_absmax(|x|max)) +
// int8 GEMV + dequant epilogue (nanopointllm/compression/w8a8.py:46-50,
// 33-43, 118-139) for the decode call sites (llama/paged_attention.py:97-124,
// llama/lightweight_runner.py:38-54, 329-379).
//
// Design: a persistent grid of one 16-wavefront workgroup per CU.
//   1. Each thread loads its x chunks and one epilogue operand (a weight scale
//      or bias of this workgroup's output blocks, kept in LDS); once x has
//      arrived each wavefront issues its first step of weight loads (they do
//      not depend on x).
//   2. While those are in flight the workgroup quantizes all M rows of x into
//      LDS (row absmax on the raw 16-bit patterns, binary16 scale, the
//      division-free exact quantizer), laid out as half MFMA A fragments:
//      8 rows x 64 K per k-block, so lane (i, g) reads row i, k 16g..16g+15
//      with one conflict-free ds_read_b128.
//   3. Workgroup b then streams 16-output weight blocks b, b+G, b+2G, ...; its
//      16 wavefronts split K.  Each keeps two steps of CH 1 KiB fragments in
//      flight in a three-buffer register ring that runs across block
//      boundaries; loads are raw buffer loads whose descriptor range ends at
//      the wave's last k-block, so the ring never reads past its share.  Per
//      block, the per-wave 16x16 int32 partials go through one of two LDS
//      buffers, one barrier (LDS counter only: the ring keeps streaming), and
//      the fused epilogue (dequant / SiLU*mul / int8 requant).
// Quantizing x once per CU costs M*K*~10 VALU ops per CU; for decode shapes
// that hides behind the weight loads already in flight, and it saves the
// separate quantization launch and its round trip through memory.
// gemv_split_kernel (below) serves the shapes with one output block per CU
// (o_proj, down): there half the wavefronts stream the block's weights from
// entry while the other half quantize one row each.
#include <atomic>
#include <type_traits>

#include "w8a8_internal.h"

namespace w8a8 {

namespace {

constexpr int kFusedWaves = 16;
constexpr int kFusedThreads = kFusedWaves * 64;
constexpr int kFusedCH = 4;
// Weight ring steps issued before x is quantized (the others follow it).
constexpr int kFusedPreSteps = 1;
// Raw buffer loads: descriptor word 3 of gfx9 (32-bit data format), the
// nontemporal cache policy (each weight byte is read once: 6% faster than the
// default policy on gate/up at M = 8) and the bytes of one 16 x 64 packed
// k-block.
constexpr int kBufferWord3 = 0x00020000;
constexpr int kCacheNT = 2;
constexpr int kBlockBytes = 1024;
constexpr int kFusedMaxRows = 8;
constexpr int kFusedMaxKB = 192;  // K <= 12288
// 9 to 16 rows: full 16-row A fragments in LDS, so K is capped lower.
constexpr int kFusedMaxRows16 = 16;
constexpr int kFusedMaxKB16 = 96;  // K <= 6144
constexpr int kFusedI8MinKB = 129;  // int8 x: K > 8192
constexpr int kFusedMaxBlocks = 64;  // 16-row output blocks per workgroup
static_assert(kFusedMaxBlocks * 16 == kFusedThreads, "one epilogue operand per thread");
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
  const float* sx_in;  // int8 x: its per-row scales
  // RMSNorm prologue (NORM kernels only): x <- dtype(x + residual) when a
  // residual is given (written to residual_out by workgroup 0), then
  // x <- dtype(w * dtype(x / sqrt(mean(x^2) + eps))) (written to x_out, when
  // given, by workgroup 0).
  const void* residual;
  int64_t ld_res;
  void* residual_out;
  int64_t ld_res_out;
  const void* norm_w;
  float eps;
  void* x_out;
  int64_t ld_xout;
  float* absmax_parts;  // kEpiSilu: [M][NB] per-block row |h|max (nullable)
  // kEpiDequant (nullable): the residual-add epilogue and its RMSNorm chunk
  // sums (LinearOperands::res / ss_parts).
  const void* add_res;
  int64_t ld_add_res;
  float* ss_out;
  int64_t ld_ss_out;
  // NORM kernels (nullable): the RMSNorm sums of squares of x per 8-column
  // chunk, as the residual-add epilogue of the launch that produced x wrote
  // them; x is then taken as the summed rows (no residual) and the sums
  // replace the workgroup's own.
  const float* ss_in;
  int64_t ld_ss_in;
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

// Start-up timeline (diagnostic builds with W8A8_TIMELINE only; the library
// proper compiles none of it).  Thread 0 of each workgroup notes the 100 MHz
// real-time counter in LDS at fixed points of the launch (kStamp* below) and
// copies them to g_stamps at the end; w8a8_timeline_read fetches the last
// launch's values.
#if W8A8_TIMELINE
constexpr int kStampsPerWg = 16;
constexpr int kStampEntry = 0;      // kernel entry
constexpr int kStampXReady = 1;     // wavefront 0 has x and its absmax
constexpr int kStampPrologue = 2;   // quantization done, ring issued, barrier passed
constexpr int kStampFirstData = 3;  // the first weight step's MFMAs issued (its data arrived)
constexpr int kStampBlock0 = 4;     // 4 + j: epilogue of block j done (j < 11)
constexpr int kStampEnd = 15;       // main loop done
constexpr int kTimelineMaxWg = 1024;
__device__ unsigned long long g_stamps[kTimelineMaxWg * kStampsPerWg];
#define W8A8_STAMP(slot, i)                                             \
  do {                                                                  \
    if (threadIdx.x == 0) (slot)[(i)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define W8A8_STAMP(slot, i) \
  do {                      \
  } while (0)
#endif

// |x| of 16-bit floats as unsigned integers (the sign bit cleared): for
// non-negative binary16 / bfloat16 values the bit patterns order like the
// values, so the integer max is the absmax.
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// Sums the per-wave partials of output block nb and writes its outputs.
// `ops` holds the block's 16 weight scales followed by its 16 biases.
// NW: wavefronts whose partials red[0 .. NW-1] hold.
template <int EPI, typename TY, typename TH, bool RES, int NW = kFusedWaves>
__device__ inline void epilogue(const FusedParams& p, const int32_t (*red)[256],
                                const float* row_s, int64_t nb, int tid, const float* ops,
                                const TY* res_pre) {
  const bool has_bias = p.bias != nullptr;
  const int M = p.M;
  if constexpr (RES) {
    // Residual-add epilogue (kEpiDequant, 16-bit output); threads below 256
    // fill whole wavefronts, so the chunk sums run in uniform control flow.
    static_assert(EPI == kEpiDequant, "residual-add epilogue");
    if (tid < 256) {
      const int m = tid >> 4;
      const int64_t n = nb * 16 + (tid & 15);
      const bool ok = m < M && n < p.N;
      float v = 0.0f;
      if (ok) {
        int32_t s = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) s += red[w][tid];
        const int r = tid & 15;
        const TY rv = res_pre != nullptr ? *res_pre
                                         : static_cast<const TY*>(p.add_res)[m * p.ld_add_res + n];
        const TY o = add_rounded(from_f32<TY>(dequant1b(s, row_s[m], ops[r], has_bias, ops[16 + r])),
                                 rv);
        static_cast<TY*>(p.y)[static_cast<int64_t>(m) * p.ldy + n] = o;
        v = to_f32(o);
      }
      if (p.ss_out != nullptr) {
        const float cs = chunk_sumsq8(v);
        if ((tid & 7) == 0 && ok) p.ss_out[m * p.ld_ss_out + (n >> 3)] = cs;
      }
    }
  } else if constexpr (EPI == kEpiI32 || EPI == kEpiDequant) {
    if (tid < 256) {
      const int m = tid >> 4;
      const int64_t n = nb * 16 + (tid & 15);
      if (m < M && n < p.N) {
        int32_t s = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) s += red[w][tid];
        TY* y = static_cast<TY*>(p.y) + static_cast<int64_t>(m) * p.ldy + n;
        if constexpr (EPI == kEpiI32) {
          *y = s;
        } else {
          const int r = tid & 15;
          *y = from_f32<TY>(dequant1b(s, row_s[m], ops[r], has_bias, ops[16 + r]));
        }
      }
    }
  } else {
    // Interleaved gate/up: packed rows 2c (gate) and 2c+1 (up) of the block
    // produce output column nb*8 + c.
    // Threads below 128 fill whole wavefronts, so the shuffles below run in
    // uniform control flow.
    if (tid < 128) {
      const int m = tid >> 3;
      const int cc = tid & 7;
      const int64_t n_out = nb * 8 + cc;
      float habs = 0.0f;
      if (m < M && n_out < p.N / 2) {
        const int base = m * 16 + 2 * cc;
        int32_t sg = 0, su = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          sg += red[w][base];
          su += red[w][base + 1];
        }
        const float sxm = row_s[m];
        const float g = to_f32(from_f32<TH>(dequant1b(sg, sxm, ops[2 * cc], has_bias,
                                                      ops[16 + 2 * cc])));
        const float u = to_f32(from_f32<TH>(dequant1b(su, sxm, ops[2 * cc + 1], has_bias,
                                                      ops[17 + 2 * cc])));
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
          if (cc == 0 && m < M) p.absmax_parts[static_cast<int64_t>(m) * p.NB + nb] = habs;
        }
      }
    }
  }
}

// NORM: the activation prologue of LightweightRMSNorm (residual add and
// RMSNorm, lightweight_runner.py:239-257) runs on the x chunks first, as in
// the reference's fused RMSNorm + packed QKV decode kernel
// (paged_attention.py:163-234); M <= 8 and NCH <= 4 only.
// NCH: 16-byte x chunks each thread holds while quantizing (sized to the
// shape, so small shapes keep their registers for the ring).  RING: register
// buffers of the weight stream; RING - 1 steps are in flight in the main
// loop, kFusedPreSteps of them during the quantization.  ROWS: activation
// rows per A fragment in LDS, 8 (M <= 8, half a fragment; the other half is
// zero) or 16 (M <= 16, K <= 6144).
template <int EPI, typename TX, typename TY, typename TH, int NCH, int RING, int ROWS,
          bool NORM = false, bool RES = false>
__global__ __launch_bounds__(kFusedThreads) void gemv_fused_kernel(FusedParams p) {
  static_assert(NCH <= kFusedMaxChunks && RING >= 2 && kFusedPreSteps < RING,
                "fused kernel shape");
  static_assert(!NORM || (NCH <= 4 && ROWS == kFusedMaxRows), "RMSNorm prologue shape");
  static_assert(ROWS == kFusedMaxRows || ROWS == kFusedMaxRows16, "8 or 16 rows");
  // TX = int8_t: x comes quantized, with per-row scales (no quantization).
  constexpr bool kI8 = std::is_same<TX, int8_t>::value;
  static_assert(!kI8 || ROWS == kFusedMaxRows, "int8 staging holds 8 rows");
  constexpr int kAStride = ROWS * 64;  // LDS bytes of one k-block's A fragment
  static_assert(kFusedMaxKB * 4 <= kFusedThreads, "one int8 x chunk per thread and row");
  // A fragments: [kb][g][row < 8][16 bytes]
  __shared__ __attribute__((aligned(16)))
      int8_t a_lds[ROWS == kFusedMaxRows ? kFusedMaxKB * 512 : kFusedMaxKB16 * 1024];
  __shared__ int32_t red[2][kFusedWaves][256];
  __shared__ uint32_t amax_w[kFusedWaves];
  __shared__ float ss_t[NORM ? kFusedMaxRows : 1][64];  // RMSNorm: per row, 64 tree sums
  __shared__ float row_s[ROWS];
  __shared__ float ops_lds[kFusedMaxBlocks * 32];  // per block: 16 scales, 16 biases
#if W8A8_TIMELINE
  __shared__ unsigned long long stamps[kStampsPerWg];
  if (threadIdx.x < kStampsPerWg) stamps[threadIdx.x] = 0;
#endif
  W8A8_STAMP(stamps, kStampEntry);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave-uniform, so the step bookkeeping below stays in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int KB = p.KB;
  const int M = p.M;

  // This wave's k-block range; all waves use the same trip count kbw.
  const int kbw = (KB + kFusedWaves - 1) / kFusedWaves;
  const int kb0 = min(wave * kbw, KB);
  const int kb1 = min(kb0 + kbw, KB);
  const int nch = (kbw + kFusedCH - 1) / kFusedCH;
  const int n_mine = (p.NB - static_cast<int>(blockIdx.x) + p.G - 1) / p.G;
  const int total = n_mine * nch;

  // The wave's work is a sequence of `total` steps; step (j, c) covers chunk
  // c (CH k-blocks of the wave's range) of its j-th weight block.  Steps are
  // loaded kFusedRing - 1 ahead into a ring of register buffers that the
  // unrolled main loop rotates by name, so no buffer is ever copied (a copy
  // would wait for every load in flight).
  // Every step issues its loads unconditionally, so the compiler's load
  // counting stays exact and it never drains the ring.  Weights are read
  // with buffer loads over the block's packed tile column whose range ends at
  // the wave's last k-block (and is empty for a step past the end): the loads
  // beyond it return zeros without a memory access.
  int lj = 0, lc = 0;  // next step to load
  auto issue = [&](i32x4(&buf)[kFusedCH]) {
    const bool past = lj >= n_mine;
    // The cursor is wave-uniform; say so, or the descriptor would be built in
    // vector registers and every load would become a loop over lanes.
    const int sj = __builtin_amdgcn_readfirstlane(past ? n_mine - 1 : lj);
    const int nrec = __builtin_amdgcn_readfirstlane(past ? 0 : kb1 * kBlockBytes);
    const int64_t nb = static_cast<int64_t>(blockIdx.x) + static_cast<int64_t>(sj) * p.G;
    // A wave without a range has kb0 = kb1 = KB: all its loads are beyond.
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<i32x4*>(p.w + nb * KB * 64), 0, nrec, kBufferWord3);
#pragma unroll
    for (int i = 0; i < kFusedCH; ++i) {
      const int off = (kb0 + lc * kFusedCH + i) * kBlockBytes + lane * 16;
      buf[i] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0,
                                                                               kCacheNT));
    }
    // Branch-free update: a store under a branch here would keep the cursor
    // in scratch memory.
    const int nc = lc + 1;
    const bool wrap = nc == nch;
    lj += wrap ? 1 : 0;
    lc = wrap ? 0 : nc;
  };

  i32x4 rb[RING][kFusedCH];

  // Residual-add epilogue: the residual of this thread's output in the
  // first block is requested before anything else, so that epilogue does not
  // wait behind the weight loads in flight (later blocks load theirs then).
  [[maybe_unused]] TY res0{};
  if constexpr (RES) {
    if (tid < 256) {
      const int m = tid >> 4;
      const int64_t n = static_cast<int64_t>(blockIdx.x) * 16 + (tid & 15);
      if (m < M && n < p.N) res0 = static_cast<const TY*>(p.add_res)[m * p.ld_add_res + n];
    }
  }

  // The epilogue operands of all this workgroup's blocks (n_mine <= 64, one
  // per thread) go to LDS up front: vmcnt counts loads in issue order, so a
  // scale loaded at epilogue time would wait for every weight load in flight.
  float op_s = 0.0f, op_b = 0.0f;
  const int op_j = tid >> 4;
  auto load_ops = [&]() {
    if constexpr (EPI != kEpiI32) {
      const int64_t n =
          (static_cast<int64_t>(blockIdx.x) + static_cast<int64_t>(op_j) * p.G) * 16 + (tid & 15);
      if (op_j < n_mine && n < p.N) {
        op_s = p.sw[n];
        if (p.bias != nullptr) op_b = p.bias[n];
      }
    }
  };
  auto store_ops = [&]() {
    if constexpr (EPI != kEpiI32) {
      if (op_j < n_mine) {
        ops_lds[op_j * 32 + (tid & 15)] = op_s;
        ops_lds[op_j * 32 + 16 + (tid & 15)] = op_b;
      }
    }
  };

  if constexpr (kI8) {
    // ------------------------------------------------ stage int8 x in LDS
    // x is int8 [M, ldx] (M * ldx < 2^30), rows 16-byte aligned and readable
    // (zero past K) up to KB*64 bytes, with per-row scales: each 16-byte
    // chunk goes straight to its slot of the A fragments.  A row has
    // KB*4 <= 768 chunks, so a thread takes at most one chunk of each row.
    // Branch-free buffer loads: the descriptor range ends after row M-1's
    // KB*64 bytes, so rows past M read zeros without a memory access (and a
    // conditional load here would let the compiler wait on each load in turn).
    const int cpr = KB * 4;
    const bool chunk_live = tid < cpr;
    const int xrec = __builtin_amdgcn_readfirstlane(static_cast<int>((M - 1) * p.ldx) + KB * 64);
    const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(p.x), 0, xrec, kBufferWord3);
    const int ldx = static_cast<int>(p.ldx);
    i32x4 v[kFusedMaxRows];
#pragma unroll
    for (int r = 0; r < kFusedMaxRows; ++r) {
      v[r] = __builtin_bit_cast(
          i32x4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, r * ldx + tid * 16, 0, 0));
    }
    load_ops();
    float sxr = 0.0f;
    // The int32 epilogue has no scales (and may be given none).
    if constexpr (EPI != kEpiI32) {
      if (tid < M) sxr = p.sx_in[tid];
    }
    // With nothing to compute on x, the weight stream starts right behind
    // the x loads; the LDS stores below wait for x only.
#pragma unroll
    for (int u = 0; u < RING - 1; ++u) issue(rb[u]);
    __builtin_amdgcn_sched_barrier(0);
    if (tid < M) row_s[tid] = sxr;
    const int k = tid * 16;
    const int off0 = ((k >> 6) * 4 + ((k & 63) >> 4)) * 8 * 16;
#pragma unroll
    for (int r = 0; r < kFusedMaxRows; ++r) {
      if (r < M && chunk_live) *reinterpret_cast<i32x4*>(a_lds + off0 + r * 16) = v[r];
    }
    store_ops();
    __syncthreads();
  } else {
  // ---------------------------------------------------------- quantize x
  // Rows are spread over power-of-two groups of TPR >= 128 threads.
  const int mpad = M <= 1 ? 1 : (M <= 2 ? 2 : (M <= 4 ? 4 : (M <= 8 ? 8 : 16)));
  const int tpr = kFusedThreads / mpad;
  const int row = tid / tpr;
  const int j0 = tid - row * tpr;
  const int nchunk = KB * 8;  // 8-element chunks per padded row
  const bool row_live = row < M;
  // x and the RMSNorm operands.  The NORM kernels use branch-free raw buffer
  // loads: each descriptor's range ends with row M-1's K elements (M * ld * 2
  // < 2^30), and a chunk outside the rows (of a row >= M, or past K) gets an
  // offset beyond every range, so it reads zeros without a memory access.
  // The others load only the chunks inside the row, under a per-lane
  // condition: an out-of-range buffer load still takes its turn in the
  // CU's address unit, and with several chunks per thread past the row (one
  // row of 4096, or down's 11008 at M = 4) those turns delay the x every
  // wavefront waits for (measured on MI355X, graphs of 32 layers: O at
  // M = 1 6.6 against 7.2 us, down at M = 4 12.5 against 13.4 us).
  constexpr int kOutside = 0x7ffffff0;
  const int K = p.K;
  auto rows_rsrc = [&](const void* base, int64_t ld) {
    const int nrec = __builtin_amdgcn_readfirstlane(
        base == nullptr ? 0 : static_cast<int>((M - 1) * ld * 2) + K * 2);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nrec, kBufferWord3);
  };
  auto chunk_off = [&](int c, int64_t ld) {
    return row_live && c * 8 < K ? static_cast<int>(row * ld * 2) + c * 16 : kOutside;
  };
  const __amdgpu_buffer_rsrc_t xrsrc = rows_rsrc(p.x, p.ldx);
  u32x4 raw[NCH];
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      raw[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             xrsrc, chunk_off(j0 + i * tpr, p.ldx), 0, 0));
    }
  } else {
    const uint16_t* xr =
        static_cast<const uint16_t*>(p.x) + static_cast<int64_t>(row_live ? row : 0) * p.ldx;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = j0 + i * tpr;
      raw[i] = u32x4{0u, 0u, 0u, 0u};
      if (row_live && c * 8 < K)
        raw[i] = *reinterpret_cast<const u32x4*>(xr + static_cast<int64_t>(c) * 8);
    }
  }
  // RMSNorm operands, loaded with x (before any weight load is queued); a
  // null residual has an empty range.
  [[maybe_unused]] u32x4 rraw[NORM ? NCH : 1];
  [[maybe_unused]] u32x4 wraw[NORM ? NCH : 1];
  if constexpr (NORM) {
    const __amdgpu_buffer_rsrc_t rrsrc = rows_rsrc(p.residual, p.ld_res);
    const __amdgpu_buffer_rsrc_t wrsrc = rows_rsrc(p.norm_w, 0);
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = j0 + i * tpr;
      rraw[i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rrsrc, chunk_off(c, p.ld_res), 0, 0));
      wraw[i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     wrsrc, row_live && c * 8 < K ? c * 16 : kOutside, 0, 0));
    }
  }
  // With the producer's chunk sums (ss_in): lane l of each wavefront of row
  // `row` takes the sums of chunks 8 l .. 8 l + 7 (zeros past the row), as
  // two 16-byte loads where all four are inside the row and four 4-byte
  // loads for the one ragged quad of a row of K % 32 != 0.
  [[maybe_unused]] float pv[NORM ? 8 : 1];
  if constexpr (NORM) {
    if (p.ss_in != nullptr) {
      const int nck = (K + 7) / 8;
      const int nrec = __builtin_amdgcn_readfirstlane(
          static_cast<int>(((M - 1) * p.ld_ss_in + nck) * 4));
      const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<float*>(p.ss_in), 0, nrec, kBufferWord3);
      const int rbase = static_cast<int>(row * p.ld_ss_in) * 4;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = 8 * lane + 4 * h;
        if (!row_live || c + 4 <= nck) {
          const u32x4 v = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         srsrc, row_live ? rbase + c * 4 : kOutside, 0, 0));
#pragma unroll
          for (int j = 0; j < 4; ++j) pv[4 * h + j] = __uint_as_float(v[j]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            pv[4 * h + j] = c + j < nck ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                                              srsrc, rbase + (c + j) * 4, 0, 0))
                                        : 0.0f;
          }
        }
      }
    }
  }
  load_ops();
  if constexpr (NORM) {
    // Every workgroup normalizes the same rows identically; workgroup 0
    // writes the summed and the normalized rows out.
    const bool writer = blockIdx.x == 0;
    auto pack2 = [](float lo, float hi) {
      return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<TX>(lo))) |
             (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<TX>(hi))) << 16);
    };
    // The binary32 sum of squares takes the order every RMSNorm route shares
    // for K <= 4096: per chunk in element order, tree8_sum over 8
    // consecutive chunks, then one butterfly over the 64 tree sums.  Chunk c
    // of the row is held here by thread c % TPR as its chunk c / TPR, and TPR
    // is a multiple of 64, so lanes 8 j .. 8 j + 7 of a wavefront hold 8
    // consecutive chunks starting at a multiple of 8.
    // Every CU normalizes all M rows, so at M = 8 this arithmetic is a large
    // part of the prologue.  For binary16 rows three steps take one packed or
    // mixed-precision instruction and give the same bits as the binary32
    // sequence of the reference:
    //   dtype(x + residual): binary32 carries 24 >= 2 * 11 + 2 bits, so
    //     rounding the binary32 sum of two binary16 values to binary16 is one
    //     correct rounding, which v_pk_add_f16 computes;
    //   the sum of squares: lo * lo is exact in binary32 for a binary16 lo
    //     (22 significant bits, within the normal range), so
    //     fma(lo, lo, ss) == fl(fl(lo * lo) + ss) (v_fma_mix_f32);
    //   dtype(w * h): the product of two binary16 values is exact in
    //     binary32, so rounding it once is v_pk_mul_f16.
    constexpr bool kHalf = std::is_same<TX, __half>::value;
    using h2 = _Float16 __attribute__((ext_vector_type(2)));
    // By value: __builtin_bit_cast of a vector element lvalue (raw[i][q])
    // reads element 0 whatever the index, so elements go through a scalar.
    auto as_h2 = [](uint32_t u) { return __builtin_bit_cast(h2, u); };
    float sq[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = j0 + i * tpr;
      const bool ok = row_live && c < nchunk && c * 8 < p.K;
      if (p.residual != nullptr) {
        // summed = dtype(x + residual)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if constexpr (kHalf) {
            raw[i][q] = __builtin_bit_cast(uint32_t, as_h2(raw[i][q]) + as_h2(rraw[i][q]));
          } else {
            raw[i][q] = pack2(bits_to_f32<TX>(raw[i][q] & 0xffffu) + bits_to_f32<TX>(rraw[i][q] & 0xffffu),
                              bits_to_f32<TX>(raw[i][q] >> 16) + bits_to_f32<TX>(rraw[i][q] >> 16));
          }
        }
        if (ok && writer) {
          *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p.residual_out) +
                                    static_cast<int64_t>(row) * p.ld_res_out +
                                    static_cast<int64_t>(c) * 8) = raw[i];
        }
      }
      if (p.ss_in == nullptr) {
        float ss = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = bits_to_f32<TX>(raw[i][q] & 0xffffu);
          const float hi = bits_to_f32<TX>(raw[i][q] >> 16);
          if constexpr (kHalf) {
            ss = __builtin_fmaf(lo, lo, ss);
            ss = __builtin_fmaf(hi, hi, ss);
          } else {
            ss = __fadd_rn(ss, __fmul_rn(lo, lo));
            ss = __fadd_rn(ss, __fmul_rn(hi, hi));
          }
        }
        sq[i] = tree8_sum(ss);
      }
    }
    float tot;
    if (p.ss_in == nullptr) {
      if ((lane & 7) == 0 && row_live) {
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
          const int c = j0 + i * tpr;  // the first of the lane group's 8 chunks
          if (c < 512) ss_t[row][c >> 3] = sq[i];
        }
      }
      __syncthreads();
      // Tree sums past the row's chunks are zeros in the other routes:
      // adding them changes nothing, so the unwritten ones read as zero.
      const int ntree = min(64, (tpr * NCH) >> 3);
      tot = wave_sum_xor(lane < ntree ? ss_t[row_live ? row : 0][lane] : 0.0f);
    } else {
      // The same tree and butterfly on the producer's chunk sums, by every
      // wavefront of the row on its own: no barrier, and the weight stream
      // starts as early as in the kernel without the norm.
      tot = wave_sum_xor(tree8_sum_lane(pv));
    }
    const float var = tot / static_cast<float>(p.K);
    const float rstd = 1.0f / sqrtf(__fadd_rn(var, p.eps));
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = j0 + i * tpr;
      const bool ok = row_live && c < nchunk && c * 8 < p.K;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // mul_keep_sign: a -0 element stays -0, as in the prologue kernel.
        if constexpr (kHalf) {
          const h2 h = {static_cast<_Float16>(mul_keep_sign(bits_to_f32<TX>(raw[i][q] & 0xffffu), rstd)),
                        static_cast<_Float16>(mul_keep_sign(bits_to_f32<TX>(raw[i][q] >> 16), rstd))};
          raw[i][q] = __builtin_bit_cast(uint32_t, as_h2(wraw[i][q]) * h);
        } else {
          const float lo = to_f32(from_f32<TX>(mul_keep_sign(bits_to_f32<TX>(raw[i][q] & 0xffffu), rstd)));
          const float hi = to_f32(from_f32<TX>(mul_keep_sign(bits_to_f32<TX>(raw[i][q] >> 16), rstd)));
          raw[i][q] = pack2(mul_keep_sign(bits_to_f32<TX>(wraw[i][q] & 0xffffu), lo),
                            mul_keep_sign(bits_to_f32<TX>(wraw[i][q] >> 16), hi));
        }
      }
      if (ok && writer && p.x_out != nullptr) {
        *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p.x_out) +
                                  static_cast<int64_t>(row) * p.ld_xout +
                                  static_cast<int64_t>(c) * 8) = raw[i];
      }
    }
  }
  // |x| patterns of both halves at once (v_pk_max_u16).
  u16x2 am2 = {0, 0};
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      am2 = __builtin_elementwise_max(am2, __builtin_bit_cast(u16x2, raw[i][q] & 0x7fff7fffu));
  }
  uint32_t am = max(static_cast<uint32_t>(am2[0]), static_cast<uint32_t>(am2[1]));
  // At 3-4 rows (4 wavefronts per row) the LDS-permute butterfly instead of
  // the DPP one: a wavefront that finishes its absmax sooner issues its first
  // weight step while other wavefronts' x loads still queue for the address
  // unit, and the workgroup's barriers then wait on them (O at M = 4: 6.7
  // against 7.2 us; start-up timelines: quantization done at 3.3 against
  // 3.8 us).  Both give the same maximum.
  if (NORM || mpad != 4) {
    am = wave_max_u32(am);
  } else {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
      am = max(am, static_cast<uint32_t>(__shfl_xor(static_cast<int>(am), off)));
  }
  W8A8_STAMP(stamps, kStampXReady);
  // The first weight loads go out once x has arrived (the absmax above waits
  // for it) and stream while x is quantized.  Only kFusedPreSteps steps go out
  // before the quantization: a wave that issues more loads than the CU's
  // memory pipeline holds stalls at the issue, which holds up the barriers of
  // the quantization and with them the whole workgroup.  The rest of the ring
  // is issued once the quantization is done.
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < kFusedPreSteps; ++u) issue(rb[u]);
  store_ops();
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
    for (int i = 0; i < NCH; ++i) {
      const int c = j0 + i * tpr;
      if (c < nchunk) {
        float xv[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          xv[2 * q] = bits_to_f32<TX>(raw[i][q] & 0xffffu);
          xv[2 * q + 1] = bits_to_f32<TX>(raw[i][q] >> 16);
        }
        u32x2 qw;
        if constexpr (NCH <= 8) {
          qw = quant8_dyn(xv, s, r);
        } else {
          // Many chunks per thread leave no registers for the fast path.
          int32_t qi[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) qi[j] = quant1_h(xv[j], s, r);
          qw = u32x2{pack4_i8(qi[0], qi[1], qi[2], qi[3]), pack4_i8(qi[4], qi[5], qi[6], qi[7])};
        }
        const int k = c * 8;
        const int off = (((k >> 6) * 4 + ((k & 63) >> 4)) * ROWS + row) * 16 + (k & 15);
        *reinterpret_cast<u32x2*>(a_lds + off) = qw;
      }
    }
  }
#pragma unroll
  for (int u = kFusedPreSteps; u < RING - 1; ++u) issue(rb[u]);
  __syncthreads();
  }
  W8A8_STAMP(stamps, kStampPrologue);

  // ------------------------------------------------------- stream weights
  const bool a_live = li < M;
  const int a_off = (lg * ROWS + li) * 16;
  i32x4 acc = i32x4{0, 0, 0, 0};
  int j = 0, c = 0;  // step being computed
  auto step = [&](const i32x4(&cur)[kFusedCH], i32x4(&freed)[kFusedCH], int t) {
    issue(freed);
    const bool live = t < total;
#pragma unroll
    for (int i = 0; i < kFusedCH; ++i) {
      const int kb = kb0 + c * kFusedCH + i;
      if (live && kb < kb1) {
        const i32x4 a = a_live ? *reinterpret_cast<const i32x4*>(a_lds + kb * kAStride + a_off)
                               : i32x4{0, 0, 0, 0};
        acc = mfma_16x16x64(a, cur[i], acc);
      }
    }
    const bool last = live && c == nch - 1;
    if (last) {
      // Block j done: reduce the wave partials and run the epilogue.  The
      // barrier waits for LDS traffic only, so the weight loads in flight keep
      // streaming across it.
      const int par = j & 1;
#pragma unroll
      for (int r = 0; r < 4; ++r) red[par][wave][(4 * lg + r) * 16 + li] = acc[r];
      acc = i32x4{0, 0, 0, 0};
      __syncthreads();
      const int64_t nb = static_cast<int64_t>(blockIdx.x) + static_cast<int64_t>(j) * p.G;
      epilogue<EPI, TY, TH, RES>(p, red[par], row_s, nb, tid, ops_lds + j * 32,
                                 j == 0 ? &res0 : nullptr);
#if W8A8_TIMELINE
      if (j < kStampEnd - kStampBlock0) W8A8_STAMP(stamps, kStampBlock0 + j);
#endif
    }
    j += last ? 1 : 0;
    c = last ? 0 : c + 1;
  };
  for (int t = 0; t < total; t += RING) {
#pragma unroll
    for (int u = 0; u < RING; ++u) {
      step(rb[u], rb[(u + RING - 1) % RING], t + u);
#if W8A8_TIMELINE
      if (t + u == 0) W8A8_STAMP(stamps, kStampFirstData);
#endif
    }
  }
  W8A8_STAMP(stamps, kStampEnd);
#if W8A8_TIMELINE
  if (threadIdx.x < kStampsPerWg && blockIdx.x < kTimelineMaxWg)
    g_stamps[blockIdx.x * kStampsPerWg + threadIdx.x] = stamps[threadIdx.x];
#endif
}

// One 16-output block per workgroup (NB <= CUs), 16-bit x, the dequant
// epilogue (o_proj and down at decode): the wavefronts split into two
// groups.  Wavefronts 8-15 issue all of the block's weight loads at entry
// (CAP k-blocks each; they do not depend on x); wavefronts 0-7 fetch row
// `wave` of x (and row `wave` + 8 with ROWS = 16), its absmax and scale, and
// quantize it into the A fragments in LDS.  A wavefront's loads retire in order, so a row never waits behind
// weight loads, and the weights stream from the first cycle instead of
// after the quantization (the kernel above issues its first weight step
// once x has arrived, and every wavefront quantizes a share of all rows).
// After one barrier the weight wavefronts run their MFMAs and hand their
// partials to wavefronts 0-3 for the epilogue.
// CAP: k-blocks per weight wavefront, which is also the number of 16-byte x
// chunks per lane of a row wavefront (K <= CAP * 8 * 64).
constexpr int kSplitXWaves = kFusedMaxRows;
constexpr int kSplitWWaves = kFusedWaves - kSplitXWaves;
constexpr int kSplitCapSmall = 8;   // K <= 4096
constexpr int kSplitCapLarge = 22;  // K <= 11264

template <int EPI, typename TX, typename TY, typename TH, bool RES, int CAP, int ROWS>
__global__ __launch_bounds__(kFusedThreads) void gemv_split_kernel(FusedParams p) {
  static_assert(EPI == kEpiDequant && !std::is_same<TX, int8_t>::value, "o_proj shape");
  constexpr int kSplitMaxKB = CAP * kSplitWWaves;
  static_assert(ROWS == kFusedMaxRows || (ROWS == kFusedMaxRows16 && CAP == kSplitCapSmall),
                "8 rows, or 16 rows of K <= 4096");
  // A fragments: [kb][g][row < 8][16 bytes]
  __shared__ __attribute__((aligned(16))) int8_t a_lds[kSplitMaxKB * ROWS * 64];
  __shared__ int32_t red[kSplitWWaves][256];
  __shared__ float row_s[ROWS];
  __shared__ float ops_lds[32];  // the block's 16 weight scales, then 16 biases

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int KB = p.KB;
  const int M = p.M;
  const int64_t nb = blockIdx.x;
  const bool loader = wave >= kSplitXWaves;

  // ------------------------------------------- weight wavefronts: issue all
  // Wavefront ww takes k-blocks [kb0, kb1); the descriptor's range ends at
  // kb1, so its loads past the range read zeros without a memory access.
  const int ww = wave - kSplitXWaves;
  const int kbw = (KB + kSplitWWaves - 1) / kSplitWWaves;
  const int kb0 = loader ? min(ww * kbw, KB) : 0;
  const int kb1 = loader ? min(kb0 + kbw, KB) : 0;
  // One register array serves both roles (weights, or the row's chunks),
  // so the kernel needs CAP x 4 of them, not twice that.
  u32x4 buf[CAP];
  if (loader) {
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<i32x4*>(p.w + nb * KB * 64), 0,
        __builtin_amdgcn_readfirstlane(kb1 * kBlockBytes), kBufferWord3);
#pragma unroll
    for (int i = 0; i < CAP; ++i) {
      buf[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rsrc, (kb0 + i) * kBlockBytes + lane * 16, 0,
                                             kCacheNT));
    }
  }

  // ---------------------------------------- row wavefronts: quantize row
  [[maybe_unused]] TY res0{};
  const int row = wave;
  const bool row_live = !loader && row < M;
  const int K = p.K;
  u32x4(&raw)[CAP] = buf;
  // The epilogue operands: wavefront 0 (row 0 is always live) holds the
  // block's scales and biases for lanes 0-15, wavefronts 0-3 the residual
  // element of their output (a wavefront w >= M has no output row:
  // 4 w >= M).  They are loaded behind x, unconditionally from clamped
  // addresses: with every load of the wavefront issued on one path, the
  // quantization waits for x only (a conditional load here would make the
  // compiler wait for all of them).
  float op_s = 0.0f, op_b = 0.0f;
  // 9-16 rows: wavefront w also takes row w + 8, loaded behind row w.
  const int row2 = row + kSplitXWaves;
  [[maybe_unused]] u32x4 raw2[ROWS > kFusedMaxRows ? CAP : 1];
  if (row_live) {
    // The row's K elements; chunks past K read zeros (zero int8 columns up
    // to the k-block end).
    const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(static_cast<const uint16_t*>(p.x) + row * p.ldx), 0,
        __builtin_amdgcn_readfirstlane(K * 2), kBufferWord3);
#pragma unroll
    for (int i = 0; i < CAP; ++i) {
      raw[i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, (lane + 64 * i) * 16, 0, 0));
    }
    if constexpr (ROWS > kFusedMaxRows) {
      // Row w + 8, or an empty range past M (the loads stay on one path).
      const __amdgpu_buffer_rsrc_t xrsrc2 = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(static_cast<const uint16_t*>(p.x) + min(row2, M - 1) * p.ldx),
          0, __builtin_amdgcn_readfirstlane(row2 < M ? K * 2 : 0), kBufferWord3);
#pragma unroll
      for (int i = 0; i < CAP; ++i) {
        raw2[i] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc2, (lane + 64 * i) * 16, 0, 0));
      }
    }
    const int64_t n = nb * 16 + (tid & 15);
    const int64_t nc = min(n, static_cast<int64_t>(p.N) - 1);
    if constexpr (RES) {
      const int m = min(tid >> 4, M - 1);
      res0 = static_cast<const TY*>(p.add_res)[m * p.ld_add_res + nc];
    }
    op_s = p.sw[nc];
    // Without a bias the epilogue ignores op_b (a select here would wait
    // for the load).
    op_b = (p.bias != nullptr ? p.bias : p.sw)[nc];
    u16x2 am2 = {0, 0};
#pragma unroll
    for (int i = 0; i < CAP; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        am2 = __builtin_elementwise_max(am2, __builtin_bit_cast(u16x2, raw[i][q] & 0x7fff7fffu));
    }
    const uint32_t am =
        wave_max_u32(max(static_cast<uint32_t>(am2[0]), static_cast<uint32_t>(am2[1])));
    const float s = scale_from_absmax(bits_to_f32<TX>(am));
    const float r = 1.0f / s;
    if (lane == 0) {
      row_s[row] = s;
      if (blockIdx.x == 0 && p.sx_out != nullptr) p.sx_out[row] = s;
    }
    const int nchunk = KB * 8;
#pragma unroll
    for (int i = 0; i < CAP; ++i) {
      const int c = lane + 64 * i;
      if (c < nchunk) {
        float xv[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          xv[2 * q] = bits_to_f32<TX>(raw[i][q] & 0xffffu);
          xv[2 * q + 1] = bits_to_f32<TX>(raw[i][q] >> 16);
        }
        const int k = c * 8;
        const int off = (((k >> 6) * 4 + ((k & 63) >> 4)) * ROWS + row) * 16 + (k & 15);
        *reinterpret_cast<u32x2*>(a_lds + off) = quant8_dyn(xv, s, r);
      }
    }
    if constexpr (ROWS > kFusedMaxRows) {
      if (row2 < M) {
        // The same steps on row w + 8.
        u16x2 bm2 = {0, 0};
#pragma unroll
        for (int i = 0; i < CAP; ++i) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            bm2 = __builtin_elementwise_max(bm2,
                                            __builtin_bit_cast(u16x2, raw2[i][q] & 0x7fff7fffu));
        }
        const uint32_t bm =
            wave_max_u32(max(static_cast<uint32_t>(bm2[0]), static_cast<uint32_t>(bm2[1])));
        const float s2 = scale_from_absmax(bits_to_f32<TX>(bm));
        const float r2 = 1.0f / s2;
        if (lane == 0) {
          row_s[row2] = s2;
          if (blockIdx.x == 0 && p.sx_out != nullptr) p.sx_out[row2] = s2;
        }
#pragma unroll
        for (int i = 0; i < CAP; ++i) {
          const int c = lane + 64 * i;
          if (c < nchunk) {
            float xv[8];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              xv[2 * q] = bits_to_f32<TX>(raw2[i][q] & 0xffffu);
              xv[2 * q + 1] = bits_to_f32<TX>(raw2[i][q] >> 16);
            }
            const int k = c * 8;
            const int off = (((k >> 6) * 4 + ((k & 63) >> 4)) * ROWS + row2) * 16 + (k & 15);
            *reinterpret_cast<u32x2*>(a_lds + off) = quant8_dyn(xv, s2, r2);
          }
        }
      }
    }
  }
  if (tid < 16) {
    ops_lds[tid] = op_s;
    ops_lds[16 + tid] = op_b;
  }
  __syncthreads();

  // ------------------------------------------------ products and epilogue
  if (loader) {
    const int li = lane & 15;
    const int lg = lane >> 4;
    const bool a_live = li < M;
    const int a_off = (lg * ROWS + li) * 16;
    i32x4 acc = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < CAP; ++i) {
      const int kb = kb0 + i;
      if (kb < kb1) {
        const i32x4 a = a_live ? *reinterpret_cast<const i32x4*>(a_lds + kb * (ROWS * 64) + a_off)
                               : i32x4{0, 0, 0, 0};
        acc = mfma_16x16x64(a, __builtin_bit_cast(i32x4, buf[i]), acc);
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) red[ww][(4 * lg + q) * 16 + li] = acc[q];
  }
  __syncthreads();
  epilogue<EPI, TY, TH, RES, kSplitWWaves>(p, red, row_s, nb, tid, ops_lds, &res0);
}

// The o_proj / down shapes gemv_split_kernel takes: M <= 8 with K <= 11264,
// or 9-16 rows of K <= 4096 (O at 9-12 / 16 rows: 7.0 / 6.6 / 8.4 against
// 8.3 / 8.5 / 9.3 us for quantization + gemv_kernel, graphs of 32 layers).
// With the residual add, 13-16 rows measured 0.5-0.9 us slower than the
// two-launch route and keep it (kSplitResMaxRows).
constexpr int kSplitResMaxRows = 12;
bool split_shape(int64_t M, int64_t NB, int64_t KB) {
  return M >= 1 && KB >= 1 &&
         ((M <= kFusedMaxRows && KB <= kSplitCapLarge * kSplitWWaves) ||
          (M <= kFusedMaxRows16 && KB <= kSplitCapSmall * kSplitWWaves)) &&
         NB <= cu_count();
}

template <int EPI, typename TX, typename TY, typename TH, bool RES = false>
hipError_t launch_f(const FusedParams& p, hipStream_t st) {
  if constexpr (EPI == kEpiDequant && !std::is_same<TX, int8_t>::value) {
    if (split_shape(p.M, p.NB, p.KB) && (!RES || p.M <= kSplitResMaxRows)) {
      constexpr int R8 = kFusedMaxRows, R16 = kFusedMaxRows16;
      const dim3 grid(p.NB), block(kFusedThreads);
      if (p.M > R8)
        hipLaunchKernelGGL((gemv_split_kernel<EPI, TX, TY, TH, RES, kSplitCapSmall, R16>), grid,
                           block, 0, st, p);
      else if (p.KB <= kSplitCapSmall * kSplitWWaves)
        hipLaunchKernelGGL((gemv_split_kernel<EPI, TX, TY, TH, RES, kSplitCapSmall, R8>), grid,
                           block, 0, st, p);
      else
        hipLaunchKernelGGL((gemv_split_kernel<EPI, TX, TY, TH, RES, kSplitCapLarge, R8>), grid,
                           block, 0, st, p);
      return hipGetLastError();
    }
  }
  // x chunks per thread: rows spread over 1024 / mpad(M) threads each.
  const int mpad = p.M <= 1 ? 1 : (p.M <= 2 ? 2 : (p.M <= 4 ? 4 : (p.M <= 8 ? 8 : 16)));
  const int per_thread = static_cast<int>(ceil_div(static_cast<int64_t>(p.KB) * 8,
                                                   kFusedThreads / mpad));
  const dim3 grid(p.G), block(kFusedThreads);
  constexpr int R8 = kFusedMaxRows, R16 = kFusedMaxRows16;
  if constexpr (std::is_same<TX, int8_t>::value) {
    hipLaunchKernelGGL((gemv_fused_kernel<EPI, TX, TY, TH, 1, 3, R8, false, RES>), grid, block, 0,
                       st, p);
  } else if (p.M > kFusedMaxRows) {
    if (per_thread <= 8)
      hipLaunchKernelGGL((gemv_fused_kernel<EPI, TX, TY, TH, 8, 3, R16, false, RES>), grid, block,
                         0, st, p);
    else
      hipLaunchKernelGGL((gemv_fused_kernel<EPI, TX, TY, TH, kFusedMaxChunks, 3, R16, false, RES>),
                         grid, block, 0, st, p);
  } else if (per_thread <= 2) {
    hipLaunchKernelGGL((gemv_fused_kernel<EPI, TX, TY, TH, 2, 3, R8, false, RES>), grid, block, 0,
                       st, p);
  } else if (per_thread <= 4) {
    hipLaunchKernelGGL((gemv_fused_kernel<EPI, TX, TY, TH, 4, 3, R8, false, RES>), grid, block, 0,
                       st, p);
  } else {
    hipLaunchKernelGGL((gemv_fused_kernel<EPI, TX, TY, TH, kFusedMaxChunks, 3, R8, false, RES>),
                       grid, block, 0, st, p);
  }
  return hipGetLastError();
}

template <int EPI, typename TX, typename TY, typename TH>
hipError_t launch_norm_f(const FusedParams& p, hipStream_t st) {
  const int mpad = p.M <= 1 ? 1 : (p.M <= 2 ? 2 : (p.M <= 4 ? 4 : 8));
  const int per_thread = static_cast<int>(ceil_div(static_cast<int64_t>(p.KB) * 8,
                                                   kFusedThreads / mpad));
  const dim3 grid(p.G), block(kFusedThreads);
  constexpr int R8 = kFusedMaxRows;
  if (per_thread <= 2)
    hipLaunchKernelGGL((gemv_fused_kernel<EPI, TX, TY, TH, 2, 3, R8, true>), grid, block, 0, st, p);
  else
    hipLaunchKernelGGL((gemv_fused_kernel<EPI, TX, TY, TH, 4, 3, R8, true>), grid, block, 0, st, p);
  return hipGetLastError();
}

template <typename TX>
hipError_t dispatch_norm_f(const FusedParams& p, int epi, int y_dtype, int h_dtype,
                           hipStream_t st) {
  switch (epi) {
    case kEpiI32:
      return launch_norm_f<kEpiI32, TX, int32_t, float>(p, st);
    case kEpiDequant:
      if (y_dtype == kF16) return launch_norm_f<kEpiDequant, TX, __half, float>(p, st);
      if (y_dtype == kBF16) return launch_norm_f<kEpiDequant, TX, __hip_bfloat16, float>(p, st);
      if (y_dtype == kF32) return launch_norm_f<kEpiDequant, TX, float, float>(p, st);
      return hipErrorInvalidValue;
    case kEpiSilu:
      if (y_dtype == kF16) return launch_norm_f<kEpiSilu, TX, __half, __half>(p, st);
      if (y_dtype == kBF16) return launch_norm_f<kEpiSilu, TX, __hip_bfloat16, __hip_bfloat16>(p, st);
      return hipErrorInvalidValue;
    case kEpiSiluQ8:
      if (h_dtype == kF16) return launch_norm_f<kEpiSiluQ8, TX, int8_t, __half>(p, st);
      if (h_dtype == kBF16) return launch_norm_f<kEpiSiluQ8, TX, int8_t, __hip_bfloat16>(p, st);
      return hipErrorInvalidValue;
    default:
      return hipErrorInvalidValue;
  }
}

template <typename TX>
hipError_t dispatch_f(const FusedParams& p, int epi, int y_dtype, int h_dtype, hipStream_t st) {
  switch (epi) {
    case kEpiI32:
      return launch_f<kEpiI32, TX, int32_t, float>(p, st);
    case kEpiDequant:
      if (p.add_res != nullptr) {  // the residual-add epilogue: 16-bit outputs
        if (y_dtype == kF16) return launch_f<kEpiDequant, TX, __half, float, true>(p, st);
        if (y_dtype == kBF16) return launch_f<kEpiDequant, TX, __hip_bfloat16, float, true>(p, st);
        return hipErrorInvalidValue;
      }
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

// Compute units of the current device (cached per device; every thread that
// fills an entry stores the same value).
int cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Persistent workgroups for nb blocks: one per CU when there are no more
// blocks than CUs, else as few as keep the per-workgroup block count at its
// minimum, ceil(nb / CUs), so nearly every workgroup streams the same bytes
// and none runs a last block alone (LLaMA-7B gate/up, 1376 blocks: 230
// workgroups of 6 blocks instead of 96 of 6 and 160 of 5; 16.3 / 16.7 / 17.0
// against 16.6 / 16.8 / 17.2 us at M = 1 / 4 / 8, graphs of 32 layers).
int balanced_grid(int64_t nb) {
  const int64_t cus = cu_count();
  return static_cast<int>(nb <= cus ? nb : ceil_div(nb, ceil_div(nb, cus)));
}

// Decode shapes: up to 8 rows of 16-bit activations, K <= 12288 and at most
// 64 output blocks per workgroup (N <= 1024 * CUs).  Each CU fetches and
// quantizes all M x K activations (the quantization itself takes 0.8 us at
// M = 8, K = 4096; with the x fetch and the barriers the stream reaches full
// rate about 4.5 us into the launch), which only pays off while the CU's
// share of the weights keeps its loads busy for longer: measured on MI355X,
// the fused kernel beats quantization +
// gemv_kernel when a CU streams at least 64 KiB of weights and at least 4
// bytes per activation element it quantizes (LLaMA-7B at M = 8: packed QKV
// and gate/up fused, O and down not, down 25% slower fused; at M <= 4 all four
// fused, O 4-7% faster than quantize + GEMV, down within 1%).  With 9-16 rows
// the quantize + GEMV route pays more per row, and 2 bytes per element
// suffice (packed QKV at M = 13-16: 12-17% faster fused).
// The dequant epilogue at one block per CU (N <= 16 * CUs, K <= 11264 at
// M <= 8, K <= 4096 at 9-16 rows: the o_proj / down shapes) takes
// gemv_split_kernel instead (split_shape): its
// weights stream from the first cycle while half the wavefronts quantize,
// so the CU's share of the weights no longer has to cover the quantization
// (graphs of 32 layers at M = 1 / 4 / 8: O 5.3 / 5.3 / 5.9 against
// 6.6 / 7.2 / 8.1 us, down 9.9 / 10.5 / 11.4 against 11.0 / 13.4 / 14.3 us).
bool fused_gemv_supported(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t N,
                          int64_t K, int epi, bool residual) {
  if (!((x_dtype == kF16 || x_dtype == kBF16) && M >= 1 && M <= kFusedMaxRows16 && K >= 8 &&
        K % 8 == 0 &&
        ceil_div(K, kTileK) <= (M <= kFusedMaxRows ? kFusedMaxKB : kFusedMaxKB16) &&
        ldx % 8 == 0 && M * ldx * 2 < (int64_t{1} << 30) &&
        (reinterpret_cast<uintptr_t>(x) & 15u) == 0))
    return false;
  const int64_t nb = ceil_div(N, kTileRows);
  if (epi == kEpiDequant && split_shape(M, nb, ceil_div(K, kTileK)) &&
      (!residual || M <= kSplitResMaxRows))
    return true;
  const int64_t g = nb < cu_count() ? nb : cu_count();
  const int64_t blocks_per_cu = ceil_div(nb, g);
  const int64_t weight_bytes_per_cu = blocks_per_cu * kTileRows * ceil_div(K, kTileK) * kTileK;
  const int64_t bytes_per_elem = M <= kFusedMaxRows ? 4 : 2;
  return blocks_per_cu <= kFusedMaxBlocks && weight_bytes_per_cu >= (64 << 10) &&
         weight_bytes_per_cu >= bytes_per_elem * M * K;
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
  p.sx_in = nullptr;
  p.residual = nullptr;
  p.ld_res = 0;
  p.residual_out = nullptr;
  p.ld_res_out = 0;
  p.norm_w = nullptr;
  p.eps = 0.0f;
  p.x_out = nullptr;
  p.ld_xout = 0;
  p.absmax_parts = op.absmax_parts;
  p.add_res = op.res;
  p.ld_add_res = op.ld_res;
  p.ss_out = op.ss_parts;
  p.ld_ss_out = op.ld_parts;
  p.ss_in = nullptr;
  p.ld_ss_in = 0;
  p.out_scale = op.out_scale;
  p.M = static_cast<int>(op.M);
  p.N = static_cast<int>(op.N);
  p.K = static_cast<int>(op.K);
  p.KB = static_cast<int>(ceil_div(op.K, kTileK));
  p.NB = static_cast<int>(ceil_div(op.N, kTileRows));
  p.G = balanced_grid(p.NB);
  if (p.NB == 0 || p.M == 0) return hipSuccess;
  if (x_dtype == kF16) return dispatch_f<__half>(p, op.epi, op.y_dtype, op.h_dtype, st);
  if (x_dtype == kBF16) return dispatch_f<__hip_bfloat16>(p, op.epi, op.y_dtype, op.h_dtype, st);
  return hipErrorInvalidValue;
}

// The RMSNorm prologue variant (residual add + RMSNorm + quantization + GEMV
// in one launch) takes the fused decode route's shapes with M <= 8, at most
// four x chunks per thread (K <= 512 * mpad(M)) and K <= 4096 (the row sums
// its squares in the activation prologue kernel's order), a norm weight of x's dtype,
// 16-byte aligned rows for every 16-bit operand, and, with a residual, 2 more
// bytes of weights per CU and activation element (every CU reads x and the
// residual).
bool fused_norm_supported(const void* x, int x_dtype, int64_t ldx, const void* residual,
                          int64_t ld_res, const void* residual_out, int64_t ld_res_out,
                          const void* norm_w, const void* x_out, int64_t ld_xout, int64_t M,
                          int64_t N, int64_t K) {
  // K <= 4096: the prologue kernel's one-chunk-per-thread summation order.
  if (M > kFusedMaxRows || K > 4096 || !fused_gemv_supported(x, x_dtype, ldx, M, N, K))
    return false;
  const int64_t mpad = M <= 1 ? 1 : (M <= 2 ? 2 : (M <= 4 ? 4 : 8));
  if (ceil_div(ceil_div(K, kTileK) * 8, kFusedThreads / mpad) > 4) return false;
  auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
  if (norm_w == nullptr || !a16(norm_w)) return false;
  if (x_out != nullptr && (!a16(x_out) || ld_xout % 8 != 0)) return false;
  if (residual != nullptr) {
    if (!a16(residual) || !a16(residual_out) || ld_res % 8 != 0 || ld_res_out % 8 != 0 ||
        M * ld_res * 2 >= (int64_t{1} << 30))
      return false;
    const int64_t nb = ceil_div(N, kTileRows);
    const int64_t g = nb < cu_count() ? nb : cu_count();
    const int64_t weight_bytes_per_cu = ceil_div(nb, g) * kTileRows * ceil_div(K, kTileK) * kTileK;
    if (weight_bytes_per_cu < 6 * M * K) return false;
  }
  return true;
}

hipError_t launch_gemv_fused_norm(const void* x, int x_dtype, int64_t ldx, const void* residual,
                                  int64_t ld_res, void* residual_out, int64_t ld_res_out,
                                  const void* norm_w, float eps, void* x_out, int64_t ld_xout,
                                  const LinearOperands& op, float* sx_out, hipStream_t st,
                                  const float* ss_in, int64_t ld_ss_in) {
  FusedParams p;
  p.x = x;
  p.ldx = ldx;
  p.w = reinterpret_cast<const i32x4*>(op.w);
  p.sw = op.sw;
  p.bias = op.bias;
  p.y = op.y;
  p.ldy = op.ldy;
  p.sx_out = sx_out;
  p.sx_in = nullptr;
  p.absmax_parts = op.absmax_parts;
  p.residual = residual;
  p.ld_res = ld_res;
  p.residual_out = residual_out;
  p.ld_res_out = ld_res_out;
  p.norm_w = norm_w;
  p.eps = eps;
  p.x_out = x_out;
  p.ld_xout = ld_xout;
  p.add_res = nullptr;
  p.ld_add_res = 0;
  p.ss_out = nullptr;
  p.ld_ss_out = 0;
  p.ss_in = ss_in;
  p.ld_ss_in = ld_ss_in;
  p.out_scale = op.out_scale;
  p.M = static_cast<int>(op.M);
  p.N = static_cast<int>(op.N);
  p.K = static_cast<int>(op.K);
  p.KB = static_cast<int>(ceil_div(op.K, kTileK));
  p.NB = static_cast<int>(ceil_div(op.N, kTileRows));
  p.G = balanced_grid(p.NB);
  if (p.NB == 0 || p.M == 0) return hipSuccess;
  if (x_dtype == kF16) return dispatch_norm_f<__half>(p, op.epi, op.y_dtype, op.h_dtype, st);
  if (x_dtype == kBF16)
    return dispatch_norm_f<__hip_bfloat16>(p, op.epi, op.y_dtype, op.h_dtype, st);
  return hipErrorInvalidValue;
}

// int8 activations (already quantized, per-row scales): the same persistent
// weight stream without the quantization.  It pays where each wavefront
// streams several ring steps per block: for K > 8192 it beats gemv_kernel
// (LLaMA-7B down at M = 1..8: 10.7-10.9 us against 11.2-11.7 us per launch),
// while for K = 4096 the staging of x before the first step costs more than
// the stream gains (O at M = 8: 7.1 against 5.3 us; the x loads wait behind
// every CU's first weight requests).  Also M <= 8, K <= 12288, at most 64
// output blocks per workgroup, rows of at most 2^30 / M bytes, and the
// dequant / SiLU*mul / int8-requant epilogues.
bool fused_gemv_i8_supported(int64_t M, int64_t N, int64_t K, int64_t lda, int epi) {
  const int64_t kb = ceil_div(K, kTileK);
  if (!(M >= 1 && M <= kFusedMaxRows && kb >= kFusedI8MinKB && kb <= kFusedMaxKB &&
        epi <= kEpiSiluQ8 && lda >= kb * kTileK && M * lda < (int64_t{1} << 30)))
    return false;
  const int64_t nb = ceil_div(N, kTileRows);
  const int64_t g = nb < cu_count() ? nb : cu_count();
  return nb >= 1 && ceil_div(nb, g) <= kFusedMaxBlocks;
}

hipError_t launch_gemv_fused_i8(const LinearOperands& op, hipStream_t st) {
  FusedParams p;
  p.x = op.a;
  p.ldx = op.lda;
  p.w = reinterpret_cast<const i32x4*>(op.w);
  p.sw = op.sw;
  p.bias = op.bias;
  p.y = op.y;
  p.ldy = op.ldy;
  p.sx_out = nullptr;
  p.sx_in = op.sx;
  p.residual = nullptr;
  p.ld_res = 0;
  p.residual_out = nullptr;
  p.ld_res_out = 0;
  p.norm_w = nullptr;
  p.eps = 0.0f;
  p.x_out = nullptr;
  p.ld_xout = 0;
  p.absmax_parts = op.absmax_parts;
  p.add_res = op.res;
  p.ld_add_res = op.ld_res;
  p.ss_out = op.ss_parts;
  p.ld_ss_out = op.ld_parts;
  p.ss_in = nullptr;
  p.ld_ss_in = 0;
  p.out_scale = op.out_scale;
  p.M = static_cast<int>(op.M);
  p.N = static_cast<int>(op.N);
  p.K = static_cast<int>(op.K);
  p.KB = static_cast<int>(ceil_div(op.K, kTileK));
  p.NB = static_cast<int>(ceil_div(op.N, kTileRows));
  p.G = balanced_grid(p.NB);
  if (p.NB == 0 || p.M == 0) return hipSuccess;
  return dispatch_f<int8_t>(p, op.epi, op.y_dtype, op.h_dtype, st);
}

}  // namespace w8a8

#if W8A8_TIMELINE
// Diagnostic export of the timeline build: copies the stamps of the last
// fused launch (kStampsPerWg per workgroup, workgroups [0, n_wg)) to host
// memory.  Not part of the C ABI of include/w8a8_gfx950.h.
extern "C" int w8a8_timeline_read(unsigned long long* host_dst, int n_wg) {
  if (host_dst == nullptr || n_wg < 0 || n_wg > w8a8::kTimelineMaxWg) return -1;
  return hipMemcpyFromSymbol(host_dst, HIP_SYMBOL(w8a8::g_stamps),
                             sizeof(unsigned long long) * w8a8::kStampsPerWg * n_wg, 0,
                             hipMemcpyDeviceToHost) == hipSuccess
             ? 0
             : -6;
}
#endif
