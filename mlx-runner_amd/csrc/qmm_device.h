// Device helpers for the gfx950 quantized-linear kernels: format decoders,
// bf16 rounding, cross-lane reductions.
//
// Formats (the two microscaling modes mlx-runner serves, src/weights.zig:37-55):
//   mxfp8: 32 OCP E4M3 elements per group, one E8M0 scale byte (2^(X-127), 0xFF = NaN).
//   nvfp4: 16 OCP E2M1 elements per group, one E4M3 scale byte.
// Packing: element k of a row is byte k%4 of uint32 word k/4 (mxfp8) or
// nibble k%8 of word k/8 (nvfp4), least significant first.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmm {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load (non-temporal: weights are read once per call).
__device__ __forceinline__ uint4 load_stream16(const void *p) {
  u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}


// 8 nvfp4 elements (one dword, lowest nibble first) times the E4M3 scale byte, as 8 bf16:
// E2M1 -> f32, times the scale, -> bf16.  E2M1 x E4M3 has at most 6 significant bits, so
// the product and its bf16 are exact (the bf16 MFMA then multiplies it with x exactly).
__device__ __forceinline__ bf16x8_t deq8_nvfp4(uint32_t word, uint32_t scale_byte) {
  const float sc = __builtin_amdgcn_cvt_f32_fp8((int)scale_byte, 0);
  bf16x8_t r;
  const f32x2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 0);
  const f32x2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 1);
  const f32x2_t p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 2);
  const f32x2_t p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 3);
  r[0] = (__bf16)(p0.x * sc);
  r[1] = (__bf16)(p0.y * sc);
  r[2] = (__bf16)(p1.x * sc);
  r[3] = (__bf16)(p1.y * sc);
  r[4] = (__bf16)(p2.x * sc);
  r[5] = (__bf16)(p2.y * sc);
  r[6] = (__bf16)(p3.x * sc);
  r[7] = (__bf16)(p3.y * sc);
  return r;
}

// E8M0 scale byte -> f32: 2^(X-127); X = 0 is the subnormal 2^-127; 0xFF -> NaN.
__device__ __forceinline__ float e8m0_to_f32(uint32_t b) {
  uint32_t u = b << 23;
  u = (b == 0u) ? 0x00400000u : u;
  u = (b == 0xFFu) ? 0x7FC00000u : u;
  return __uint_as_float(u);
}

// E4M3 (OCP "fn") byte -> f32 by integer construction (exact; NaN for S.1111.111).
__device__ __forceinline__ float e4m3_to_f32_int(uint32_t b) {
  uint32_t s = (b & 0x80u) << 24;
  uint32_t e = (b >> 3) & 0xFu;
  uint32_t m = b & 7u;
  float sub = (float)m * 0x1p-9f;                       // e == 0: m/8 * 2^-6
  float nor = __uint_as_float(((e + 120u) << 23) | (m << 20));
  float v = (e == 0u) ? sub : nor;
  v = __uint_as_float(__float_as_uint(v) | s);
  return ((b & 0x7Fu) == 0x7Fu) ? __uint_as_float(0x7FC00000u) : v;
}

// E4M3 byte `sel` (0..3) of a word -> f32 with the gfx950 converter (OCP E4M3).
__device__ __forceinline__ float e4m3_to_f32_hw(uint32_t word, int sel) {
  switch (sel) {
    case 0: return __builtin_amdgcn_cvt_f32_fp8((int)word, 0);
    case 1: return __builtin_amdgcn_cvt_f32_fp8((int)word, 1);
    case 2: return __builtin_amdgcn_cvt_f32_fp8((int)word, 2);
    default: return __builtin_amdgcn_cvt_f32_fp8((int)word, 3);
  }
}

// E2M1 nibble -> f32 by table-free integer construction (exact).
__device__ __forceinline__ float e2m1_to_f32_int(uint32_t nib) {
  uint32_t s = (nib & 8u) << 28;
  uint32_t e = (nib >> 1) & 3u;
  uint32_t m = nib & 1u;
  float sub = m ? 0.5f : 0.0f;
  float nor = __uint_as_float(((e + 126u) << 23) | (m << 22));
  float v = (e == 0u) ? sub : nor;
  return __uint_as_float(__float_as_uint(v) | s);
}

// Two E2M1 nibbles (byte `sel` of a word) -> packed bf16 pair, unscaled.
template <int SEL>
__device__ __forceinline__ bf16x2_t fp4x2_to_bf16x2(uint32_t word) {
  return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, 1.0f, SEL);
}
// Two E4M3 bytes (half-word `HI` of a word) -> packed bf16 pair, unscaled.
template <bool HI>
__device__ __forceinline__ bf16x2_t fp8x2_to_bf16x2(uint32_t word) {
  return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, 1.0f, HI);
}
template <int SEL>
__device__ __forceinline__ f32x2_t fp4x2_to_f32x2(uint32_t word) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, SEL);
}
template <bool HI>
__device__ __forceinline__ f32x2_t fp8x2_to_f32x2(uint32_t word) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word, 1.0f, HI);
}

// Scale operand 2^t (t in [-127, 127]) for the v_cvt_scalef32_* conversions, which read
// only the f32's exponent field as an E8M0 code (field 0, here t = -127, is 2^-127).
// Measured on gfx950 for every bf16 input at t from -127 to 127:
//   cvt_scalef32_pk_fp8_f32 / _fp8_bf16 (a, b, 2^t) == cvt_pk_fp8_f32(a * 2^-t, b * 2^-t)
//   cvt_scalef32_pk_f32_fp8 (w, 2^t)              == cvt_pk_f32_fp8(w) * 2^t
__device__ __forceinline__ float e8m0_scale_operand(int t) { return __uint_as_float((uint32_t)(t + 127) << 23); }

typedef short i16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(bf16x2_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(a, __builtin_bit_cast(bf16x2_t, b), c, false);
}

// f32 -> bf16 bits, round to nearest even; NaN -> 0x7FC0 (quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  return (f != f) ? (uint16_t)0x7FC0u : (uint16_t)r;
}
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16_rne(f)); }

// mlx-runner's MLP activation on bf16 arrays (src/model.zig:405-415 silu, :451-456
// mul, used by mlpForwardQ :905-915), every op rounding its result to bf16:
//   g, u = the two projections (bf16), sg = sigmoid(g), sl = g * sg, h = sl * u.
// sigmoid is 1 / (1 + exp(-g)) in f32.  Returns h in f32, already a bf16 value.
__device__ __forceinline__ float silu_mul_bf16(float g, float u) {
  const float gb = bf16_round(g), ub = bf16_round(u);
  const float sg = bf16_round(1.f / (1.f + expf(-gb)));
  const float sl = bf16_round(gb * sg);
  return bf16_round(sl * ub);
}

// Smallest t with 448 * 2^t >= amax (amax > 0, finite), clamped to the E8M0 range.
__device__ __forceinline__ int ceil_scale_exp(float amax) {
  uint32_t u = __float_as_uint(amax);
  int e = (int)((u >> 23) & 0xFF);
  int fl = e - 127;
  uint32_t mant = u & 0x7FFFFFu;
  if (e == 0) {  // f32 subnormal
    fl = 31 - __builtin_clz(mant) - 149;
    mant = (mant << (__builtin_clz(mant) - 8)) & 0x7FFFFFu;
  }
  int t = fl - 8;
  if (mant > 0x600000u) t += 1;  // significand > 1.75: 448 * 2^(fl-8) < amax
  if (t < -127) t = -127;
  if (t > 127) t = 127;
  return t;
}

// Sum over the 64 lanes of a wave; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <typename T>
struct OutStore;
template <>
struct OutStore<uint16_t> {
  __device__ static void put(uint16_t *p, float v) { *p = f32_to_bf16_rne(v); }
};
template <>
struct OutStore<float> {
  __device__ static void put(float *p, float v) { *p = v; }
};

}  // namespace qmm
