// Shared device helpers for the W8A8 linear kernels (gfx950 / CDNA4).
//
// Numerical contract (nanopointllm/compression/w8a8.py:14-62,118-139):
//   * int8 values in [-127, 127], ties-to-even rounding (v_rndne_f32);
//   * scale = max(f32(f16_rne(max(absmax, 2^-14) / 127)), 2^-14) with an
//     IEEE-correct binary32 division (hipcc's default division lowering);
//   * q = clamp(rne(f32(x) / s), -127, 127) with a correct binary32 division;
//   * signed int32 accumulation;
//   * dequant: f32(acc) * s_x, then * s_w, then + bias: three separate binary32
//     roundings, never contracted into an FMA (explicit __fmul_rn/__fadd_rn).
//
// Packed operand layout ("16x64 tiles").  An int8 matrix R[rows][K] is stored
// as tiles of 16 rows x 64 K (1 KiB each).  Tile (rb, kb) sits at byte offset
// (rb * KB + kb) * 1024 with KB = ceil(K / 64).  Inside a tile, bytes
// [16*l, 16*l+16) belong to lane l = r + 16*g and hold R[16*rb + r][64*kb + 16*g
// .. +15].  That is the register image of one operand of
// v_mfma_i32_16x16x64_i8, so a wave fetches a whole fragment with one
// coalesced 1 KiB global_load_dwordx4 (or one global_load_lds_dwordx4 into
// LDS) and reads it back from LDS conflict-free with ds_read_b128.  Rows past
// `rows` and columns past K are zero, so padded work contributes nothing.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

namespace w8a8 {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kScaleMin = 6.103515625e-05f;  // 2^-14, smallest normal binary16
constexpr int kTileRows = 16;
constexpr int kTileK = 64;
constexpr int kTileBytes = kTileRows * kTileK;  // 1024
constexpr int kTileVec = kTileBytes / 16;       // 64 x 16-byte lane slots

// Element-type tags shared with the C ABI (include/w8a8_gfx950.h).
enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2, kI32 = 3, kI8 = 4 };

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------- conversions
__device__ inline float to_f32(float v) { return v; }
__device__ inline float to_f32(__half v) { return __half2float(v); }
__device__ inline float to_f32(__hip_bfloat16 v) {
  return __uint_as_float(static_cast<uint32_t>(__builtin_bit_cast(uint16_t, v)) << 16);
}

template <typename T> __device__ inline T from_f32(float v);
template <> __device__ inline float from_f32<float>(float v) { return v; }
template <> __device__ inline __half from_f32<__half>(float v) { return __float2half_rn(v); }
template <> __device__ inline __hip_bfloat16 from_f32<__hip_bfloat16>(float v) {
  // binary32 -> bfloat16, round to nearest even; NaN stays a quiet NaN.
  uint32_t u = __float_as_uint(v);
  uint16_t b;
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    b = static_cast<uint16_t>((u >> 16) | 0x0040u);
  } else {
    b = static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  }
  return __builtin_bit_cast(__hip_bfloat16, b);
}

// A 16-bit pattern of type TX as binary32.
template <typename TX>
__device__ inline float bits_to_f32(uint32_t b16) {
  return to_f32(__builtin_bit_cast(TX, static_cast<uint16_t>(b16)));
}

// Two binary32 values rounded to the 16-bit type T, packed low then high.
template <typename T>
__device__ inline uint32_t pack2_bits(float lo, float hi) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(lo))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(hi))) << 16);
}

// Loads 8 consecutive elements as binary32.  `vec` selects one (fp16/bf16)
// or two (f32) 16-byte loads; callers guarantee 16-byte alignment then.
template <typename T>
__device__ inline void load8(const T* __restrict__ p, float (&v)[8], bool vec, int valid) {
  if (vec && valid >= 8) {
    if constexpr (sizeof(T) == 2) {
      u32x4 raw = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint16_t lo = static_cast<uint16_t>(raw[j] & 0xffffu);
        uint16_t hi = static_cast<uint16_t>(raw[j] >> 16);
        v[2 * j] = to_f32(__builtin_bit_cast(T, lo));
        v[2 * j + 1] = to_f32(__builtin_bit_cast(T, hi));
      }
    } else {
      u32x4 r0 = reinterpret_cast<const u32x4*>(p)[0];
      u32x4 r1 = reinterpret_cast<const u32x4*>(p)[1];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] = __uint_as_float(r0[j]);
        v[4 + j] = __uint_as_float(r1[j]);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (j < valid) ? to_f32(p[j]) : 0.0f;
  }
}

// --------------------------------------------------------------- quant math
// scale_from_absmax (nanopointllm/compression/w8a8.py:46-50).
__device__ inline float scale_from_absmax(float absmax) {
  float raw = fmaxf(absmax, kScaleMin) / 127.0f;  // IEEE binary32 division
  float s = __half2float(__float2half_rn(raw));
  return fmaxf(s, kScaleMin);
}

// quantize_symmetric (nanopointllm/compression/w8a8.py:33-43) for one value.
__device__ inline int32_t quant1(float x, float s) {
  float q = __builtin_rintf(x / s);  // IEEE binary32 division, ties-to-even
  q = fminf(fmaxf(q, -127.0f), 127.0f);
  return static_cast<int32_t>(q);
}

// quantize_symmetric for a binary16 / bfloat16 input x without a division.
// r is any binary32 approximation of 1/s within a few ulps (v_rcp_f32 is).
// Exactness: with s binary16 and x of at most 11 significant bits, the exact
// quotient z = x/s is either a half-integer k+0.5 or at least 2^-12 away
// from every half-integer (x - (k+0.5)s is a nonzero multiple of
// 2^(e(s)-11) and s < 2^(e(s)+1)), while |x*r - z| <= 128 * 3 * 2^-24 <
// 2^-15 for |z| < 128.  So rint(x*r) == rint(fl32(x/s)) except at exact
// ties, which are detected exactly: c*s is exact for c = floor(x*r) + 0.5,
// and fma(-c, s, x) is zero iff x == c*s.  Ties round to even via rint(c).
// |z| >= 128 always clamps to +-127 on both paths.
__device__ inline int32_t quant1_h(float x, float s, float r) {
  const float y = x * r;
  const float c = floorf(y) + 0.5f;
  const bool tie = __builtin_fmaf(-c, s, x) == 0.0f;
  float q = __builtin_rintf(tie ? c : y);
  q = fminf(fmaxf(q, -127.0f), 127.0f);
  return static_cast<int32_t>(q);
}

__device__ inline uint32_t pack4_i8(int32_t a, int32_t b, int32_t c, int32_t d) {
  return (static_cast<uint32_t>(a) & 0xffu) | ((static_cast<uint32_t>(b) & 0xffu) << 8) |
         ((static_cast<uint32_t>(c) & 0xffu) << 16) | ((static_cast<uint32_t>(d) & 0xffu) << 24);
}

// Quantizes 8 values with a dynamic row scale s (scale_from_absmax of the
// row's |x|max, so |x / s| <= 127.07) and r = 1/s, exactly and faster than
// quant1_h, into two words of 4 int8 each.  t = fma(x, r, 1.5 * 2^23) is
// 1.5 * 2^23 plus the integer nearest to the exact product x*r (ties to
// even): with |x*r| < 128 it stays in [2^23, 2^24), where the ulp is 1, so
// the low byte of its bit pattern is that integer as an int8.  It rounds
// x / s correctly unless x*r lies within 2^-15 of a half-integer
// (|x*r - x/s| <= 127.07 * 2^-24), which the exact remainder
// e = fma(x, r, -(t - 1.5 * 2^23)) detects: |e| >= 0.5 - 2^-14 takes every
// such case (and a few more).  When any lane of the wavefront has one, the 8
// values are redone with quant1_h (a wave-uniform branch).  No clamp is
// needed: |rint(x / s)| <= 127.
__device__ inline u32x2 quant8_dyn(const float (&x)[8], float s, float r) {
  constexpr float kMagic = 0x1.8p23f;
  float t[8];
  float dev = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    t[j] = __builtin_fmaf(x[j], r, kMagic);
    dev = fmaxf(dev, fabsf(__builtin_fmaf(x[j], r, kMagic - t[j])));
  }
  if (__any(dev >= 0.5f - 0x1p-14f)) {
    int32_t q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = quant1_h(x[j], s, r);
    return u32x2{pack4_i8(q[0], q[1], q[2], q[3]), pack4_i8(q[4], q[5], q[6], q[7])};
  }
  u32x2 w;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // v_perm_b32 byte selectors: 0-3 pick bytes of the second operand, 4-7
    // bytes of the first, 12 a zero byte.
    const uint32_t lo = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, t[4 * h + 1]),
                                              __builtin_bit_cast(uint32_t, t[4 * h]), 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, t[4 * h + 3]),
                                              __builtin_bit_cast(uint32_t, t[4 * h + 2]),
                                              0x04000c0cu);
    w[h] = lo | hi;
  }
  return w;
}


// Dequant epilogue (w8a8.py:134-137): three separate binary32 roundings.
// dequant1 with the bias value already loaded (added only when present, so a
// zero result keeps its sign exactly as without a bias).
__device__ inline float dequant1b(int32_t acc, float sx, float sw, bool has_bias, float b) {
  float v = static_cast<float>(acc);
  v = __fmul_rn(v, sx);
  v = __fmul_rn(v, sw);
  if (has_bias) v = __fadd_rn(v, b);
  return v;
}

__device__ inline float dequant1(int32_t acc, float sx, float sw, const float* __restrict__ bias,
                                 int64_t n) {
  float v = static_cast<float>(acc);  // v_cvt_f32_i32: round to nearest even
  v = __fmul_rn(v, sx);
  v = __fmul_rn(v, sw);
  if (bias != nullptr) v = __fadd_rn(v, bias[n]);
  return v;
}

// a * b in binary32, kept a value of its own.  A binary32 multiply feeding a
// 16-bit conversion is otherwise merged by the backend into a mixed-precision
// FMA with a +0 addend, which turns a -0 product into +0; the empty asm (no
// instruction) stops the merge, so the conversion sees the exact product.
__device__ inline float mul_keep_sign(float a, float b) {
  float p = __fmul_rn(a, b);
  asm volatile("" : "+v"(p));
  return p;
}

// SiLU(g) * u on binary16 operands (llama/lightweight_runner.py:358):
// SiLU in binary32, rounded to the activation type, then the product
// (exact in binary32) rounded once.
template <typename T>
__device__ inline float silu_mul(float g, float u) {
  float s = g / (1.0f + expf(-g));
  s = to_f32(from_f32<T>(s));
  // SiLU of a very negative gate is -0, and so is its product.
  return mul_keep_sign(s, u);
}

// INT32 -> A8 requantization of the hardware model
// (architecture_simulator/gtsu_cycle/requant.py:98-119): (acc + bias) *
// multiplier, the magnitude rounded at `shift` with ties to even, the sign
// restored, clipped to [-127, 127].  |acc + bias| <= 2^32 and multiplier <
// 2^32 keep the product below 2^64.  Shifts are clamped to [0, 63].
__host__ __device__ inline int32_t requant1(int32_t acc, int32_t bias, uint32_t multiplier, int shift) {
  const int64_t sum = static_cast<int64_t>(acc) + bias;
  const bool neg = sum < 0;
  const uint64_t mag = static_cast<uint64_t>(neg ? -sum : sum) * multiplier;
  shift = shift < 0 ? 0 : (shift > 63 ? 63 : shift);
  uint64_t t = mag;
  if (shift > 0) {
    t = mag >> shift;
    const uint64_t rem = mag & ((uint64_t{1} << shift) - 1);
    const uint64_t half = uint64_t{1} << (shift - 1);
    t += (rem > half || (rem == half && (t & 1))) ? 1 : 0;
  }
  const int32_t r = static_cast<int32_t>(t < 127 ? t : 127);
  return (neg && mag != 0) ? -r : r;
}

// v >> s rounded to nearest, ties to even (s <= 0: exact left shift).  v <
// 2^54, so s >= 64 rounds to zero.
__host__ __device__ inline uint64_t rne_shift_u64(uint64_t v, int s) {
  if (s <= 0) return v << (-s);
  if (s >= 64) return 0;
  const uint64_t t = v >> s;
  const uint64_t rem = v & ((uint64_t{1} << s) - 1);
  const uint64_t half = uint64_t{1} << (s - 1);
  return t + ((rem > half || (rem == half && (t & 1))) ? 1 : 0);
}

// INT32 x FP16 x FP16 -> BF16 with one rounding of the exact product
// (architecture_simulator/gtsu_cycle/bf16_dequant.py:47-77): round to nearest
// even, subnormal results kept, overflow to infinity, a zero operand gives +0.
// |acc| * 11-bit * 11-bit significands < 2^53 is exact in 64 bits.  A scale
// that is infinite or NaN gives the quiet NaN 0x7fc0 (the model rejects it).
__host__ __device__ inline uint16_t dequant_bf16_exact(int32_t acc, uint16_t sa_bits, uint16_t sw_bits) {
  const int ea = (sa_bits >> 10) & 0x1f, ew = (sw_bits >> 10) & 0x1f;
  if (ea == 0x1f || ew == 0x1f) return 0x7fc0;
  const uint64_t ma = ea ? 1024u + (sa_bits & 0x3ffu) : (sa_bits & 0x3ffu);
  const uint64_t mw = ew ? 1024u + (sw_bits & 0x3ffu) : (sw_bits & 0x3ffu);
  if (acc == 0 || ma == 0 || mw == 0) return 0;
  const int exponent = (ea ? ea - 25 : -24) + (ew ? ew - 25 : -24);
  const uint32_t sign = (acc < 0 ? 1u : 0u) ^ (sa_bits >> 15) ^ (sw_bits >> 15);
  const uint64_t mag = acc < 0 ? uint64_t{0} - static_cast<uint64_t>(static_cast<int64_t>(acc))
                               : static_cast<uint64_t>(acc);
  const uint64_t product = mag * ma * mw;
  const int top = 63 - __builtin_clzll(product);
  int unbiased = top + exponent;
  if (unbiased < -126) {
    const uint64_t frac = rne_shift_u64(product, -(exponent + 133));
    if (frac == 0) return static_cast<uint16_t>(sign << 15);
    if (frac >= 128) return static_cast<uint16_t>((sign << 15) | (1u << 7));
    return static_cast<uint16_t>((sign << 15) | frac);
  }
  uint64_t sig = rne_shift_u64(product, top - 7);
  if (sig >= 256) {
    sig >>= 1;
    ++unbiased;
  }
  if (unbiased > 127) return static_cast<uint16_t>((sign << 15) | 0x7f80u);
  return static_cast<uint16_t>((sign << 15) | (static_cast<uint32_t>(unbiased + 127) << 7) |
                               static_cast<uint32_t>(sig - 128));
}

// Binary16 bit pattern of a binary32 scale (exact for the binary16-
// representable scales of the W8A8 contract).
__device__ inline uint16_t f16_bits(float v) {
  return __builtin_bit_cast(uint16_t, __float2half_rn(v));
}

// ------------------------------------------------------------ raw buffers
// A raw buffer descriptor over [base, base + bytes) (gfx9 word 3: 32-bit
// data format): loads at offsets outside the range return zeros without a
// memory access, so they need no branch.  A null base gets an empty range.
__device__ inline __amdgpu_buffer_rsrc_t raw_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(base), 0, __builtin_amdgcn_readfirstlane(base == nullptr ? 0 : bytes),
      0x00020000);
}

__device__ inline u32x4 load16(__amdgpu_buffer_rsrc_t r, int offset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0));
}

// ------------------------------------------------------ wavefront butterfly
// op over the 64 lanes of a wavefront in the order of the xor butterfly
// v = op(v, shfl_xor(v, d)) for d = 32, 16, 8, 4, 2, 1, every lane ending
// with the result, without LDS round trips.  Partners at distance 32 and 16
// come from v_permlane32_swap / v_permlane16_swap of the value with itself
// (one half of the pair holds the lane's value, the other its partner's), at
// 8 from a DPP rotation by 8 within a row of 16 (lane j reads j ^ 8), at 2
// and 1 from quad permutations.  At 4 a rotation by 4 reads lane j ^ 4 or
// (j ^ 4) ^ 8, which hold the same bits after the level at distance 8: each
// level leaves a lane and its partner with op of the same two values, and op
// must be commutative bit for bit (binary32 +; max of non-negative values).
// Every lane of the wavefront must be active.
template <typename Op>
__device__ inline uint32_t wave_butterfly(uint32_t v, Op op) {
  constexpr int kRowRor8 = 0x128, kRowRor4 = 0x124, kQuadXor2 = 0x4e, kQuadXor1 = 0xb1;
  const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  v = op(a[0], a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = op(b[0], b[1]);
  v = op(v, __builtin_amdgcn_update_dpp(0u, v, kRowRor8, 0xf, 0xf, false));
  v = op(v, __builtin_amdgcn_update_dpp(0u, v, kRowRor4, 0xf, 0xf, false));
  v = op(v, __builtin_amdgcn_update_dpp(0u, v, kQuadXor2, 0xf, 0xf, false));
  v = op(v, __builtin_amdgcn_update_dpp(0u, v, kQuadXor1, 0xf, 0xf, false));
  return v;
}

// Binary32 sum with the bits of the __shfl_xor butterfly.
__device__ inline float wave_sum_xor(float v) {
  return __uint_as_float(wave_butterfly(__float_as_uint(v), [](uint32_t x, uint32_t y) {
    return __float_as_uint(__fadd_rn(__uint_as_float(x), __uint_as_float(y)));
  }));
}

// fmaxf over non-negative values (|x|): the same bits in any order.
__device__ inline float wave_max_abs(float v) {
  return __uint_as_float(wave_butterfly(__float_as_uint(v), [](uint32_t x, uint32_t y) {
    return __float_as_uint(fmaxf(__uint_as_float(x), __uint_as_float(y)));
  }));
}

__device__ inline uint32_t wave_max_u32(uint32_t v) {
  return wave_butterfly(v, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
}

// ------------------------------------------------- residual-add epilogue
// The residual add of a decoder layer in the activation dtype (hidden +
// attn_out, hidden + mlp_out: lightweight_runner.py:247-257, 552): the
// linear's output already rounded to T plus the residual, rounded to T once
// (binary32 holds the sum of two binary16 / bfloat16 values closely enough
// that its rounding to T is the correct rounding of the exact sum).
template <typename T>
__device__ inline T add_rounded(T y, T r) {
  return from_f32<T>(__fadd_rn(to_f32(y), to_f32(r)));
}

// RMSNorm sums of squares per 8-column chunk, in the order of the norm
// kernels (per chunk in element order from +0, each square rounded to
// binary32 and added with one rounding): lanes 8j .. 8j+7 hold elements 0..7
// of one chunk (0 for an element past the row) and every lane of the group
// returns the chunk's sum.  Every lane of the wavefront must be active.
__device__ inline float chunk_sumsq8(float v) {
  const float sq = __fmul_rn(v, v);
  const int base = static_cast<int>(__lane_id()) & ~7;
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) s = __fadd_rn(s, __shfl(sq, base + j));
  return s;
}

// The RMSNorm sum of squares of a row of K <= 4096 elements, in the order
// every route takes (activation prologue, fused decode kernels, the chunk
// sums of the residual-add epilogue): s_c per 8-column chunk (chunk_sumsq8),
// then T_L = ((s_8L + s_8L+1) + (s_8L+2 + s_8L+3)) + ((s_8L+4 + s_8L+5) +
// (s_8L+6 + s_8L+7)) for L < 64 (chunks past the row count 0), then the xor
// butterfly of wave_sum_xor over T_0 .. T_63.
//
// tree8_sum: lanes 8j .. 8j+7 holding s_8L .. s_8L+7 all return T_L (quad
// permutations for the first two levels, the half-row mirror for the third:
// after two levels lanes 0-3 of a group hold the first half's sum and lanes
// 4-7 the second's, and the mirror pairs each lane with the other half).
// Every lane of the wavefront must be active.
__device__ inline float tree8_sum(float v) {
  constexpr int kQuadXor1 = 0xb1, kQuadXor2 = 0x4e, kRowHalfMirror = 0x141;
  uint32_t u = __float_as_uint(v);
  v = __fadd_rn(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, u, kQuadXor1, 0xf, 0xf, false)));
  u = __float_as_uint(v);
  v = __fadd_rn(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, u, kQuadXor2, 0xf, 0xf, false)));
  u = __float_as_uint(v);
  return __fadd_rn(v, __uint_as_float(__builtin_amdgcn_update_dpp(0u, u, kRowHalfMirror, 0xf,
                                                                  0xf, false)));
}

// T_L of eight consecutive chunk sums held by one lane, the same tree.
__device__ inline float tree8_sum_lane(const float (&s)[8]) {
  return __fadd_rn(__fadd_rn(__fadd_rn(s[0], s[1]), __fadd_rn(s[2], s[3])),
                   __fadd_rn(__fadd_rn(s[4], s[5]), __fadd_rn(s[6], s[7])));
}

// Packed-tile byte offset of element (r, k) of a [rows, K] operand.
__host__ __device__ inline int64_t packed_offset(int64_t r, int64_t k, int64_t KB) {
  int64_t tile = (r >> 4) * KB + (k >> 6);
  int64_t lane = (r & 15) + 16 * ((k & 63) >> 4);
  return tile * kTileBytes + lane * 16 + (k & 15);
}

}  // namespace w8a8
