// Rounding points shared by every kernel of the forward path.
//
// The reference's WGSL fixes most of its arithmetic by writing it out: an
// explicit fma where it fuses, a separate multiply and add everywhere else.
// Kernels here are compiled with -ffp-contract=off and use __builtin_fmaf
// exactly where the reference calls fma, so each operation rounds where the
// reference's does.
//
// The reference leaves a few rounding points to WGSL built-ins whose results
// are implementation-defined. Each gets one definition here, built from
// correctly rounded f32 operations only, so a kernel's bits do not depend on
// the GPU's transcendental units:
//   dot4          ((a0*b0 + a1*b1) + a2*b2) + a3*b3, each op rounded
//   inverse_sqrt  1 / sqrt(x): IEEE division and square root
//   exp2f_fixed   2^x: k = rint(x), 2^(x-k) by its Taylor series to r^7
//                 (truncation under 2^-27), times 2^k from exponent bits;
//                 0 below -125.5
//   cos/sin       quarter-turn split (pi/2 in three parts), Taylor series to
//                 r^12 and r^11 on [-pi/4, pi/4]
//   exp, x <= 0   the reference's own explicit form (matmul.wgsl:122-135)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define FRZ_HD __host__ __device__ __forceinline__

namespace frz {

FRZ_HD float bits_to_float(uint32_t u) { return __builtin_bit_cast(float, u); }
FRZ_HD uint32_t float_to_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

FRZ_HD float fmaf_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

// Round to nearest integer, ties to even (WGSL round; v_rndne_f32).
FRZ_HD float rint_(float x) { return __builtin_rintf(x); }

FRZ_HD float dot4(float a0, float a1, float a2, float a3, float b0, float b1,
                  float b2, float b3) {
  return ((a0 * b0 + a1 * b1) + a2 * b2) + a3 * b3;
}

FRZ_HD float inverse_sqrt(float x) { return 1.0f / __builtin_sqrtf(x); }

// e^x for x <= 0 (matmul.wgsl:122-135).
FRZ_HD float exp_nonpositive(float x) {
  const float xc = __builtin_fmaxf(x, -100.0f);
  const float k = __builtin_floorf(fmaf_(xc, 1.4426950408889634f, 0.5f));
  float r = fmaf_(k, -0.693145751953125f, xc);
  r = fmaf_(k, -1.4286068203094172e-06f, r);
  float p = (float)(1.0 / 720.0);
  p = fmaf_(p, r, (float)(1.0 / 120.0));
  p = fmaf_(p, r, (float)(1.0 / 24.0));
  p = fmaf_(p, r, (float)(1.0 / 6.0));
  p = fmaf_(p, r, 0.5f);
  p = fmaf_(p, r, 1.0f);
  p = fmaf_(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)k);
}

// GELU, tanh form (matmul.wgsl:141-147).
FRZ_HD float gelu_tanh(float g) {
  const float z = 0.7978845608028654f * fmaf_(0.044715f * g * g, g, g);
  const float e = exp_nonpositive(-2.0f * __builtin_fabsf(z));
  const float sign = z > 0.0f ? 1.0f : (z < 0.0f ? -1.0f : 0.0f);
  const float t = sign * ((1.0f - e) * (1.0f / (1.0f + e)));
  const float half_g = 0.5f * g;
  return fmaf_(half_g, t, half_g);
}

FRZ_HD float exp2f_fixed(float x) {
  if (x < -125.5f) return 0.0f;
  if (x > 127.0f) x = 127.0f;
  const float k = rint_(x);
  const float r = x - k;
  float p = 1.525273380405984e-05f;
  p = fmaf_(p, r, 1.5403530393381608e-04f);
  p = fmaf_(p, r, 1.3333558146428443e-03f);
  p = fmaf_(p, r, 9.618129107628477e-03f);
  p = fmaf_(p, r, 5.550410866482158e-02f);
  p = fmaf_(p, r, 2.402265069591007e-01f);
  p = fmaf_(p, r, 6.931471805599453e-01f);
  p = fmaf_(p, r, 1.0f);
  return p * bits_to_float((uint32_t)((int)k + 127) << 23);
}

FRZ_HD float sin_poly(float r) {
  const float z = r * r;
  float p = (float)(-1.0 / 39916800.0);
  p = fmaf_(p, z, (float)(1.0 / 362880.0));
  p = fmaf_(p, z, (float)(-1.0 / 5040.0));
  p = fmaf_(p, z, (float)(1.0 / 120.0));
  p = fmaf_(p, z, (float)(-1.0 / 6.0));
  return fmaf_(r * z, p, r);
}

FRZ_HD float cos_poly(float r) {
  const float z = r * r;
  float p = (float)(1.0 / 479001600.0);
  p = fmaf_(p, z, (float)(-1.0 / 3628800.0));
  p = fmaf_(p, z, (float)(1.0 / 40320.0));
  p = fmaf_(p, z, (float)(-1.0 / 720.0));
  p = fmaf_(p, z, (float)(1.0 / 24.0));
  p = fmaf_(p, z, -0.5f);
  return fmaf_(z, p, 1.0f);
}

// cos and sin of an angle in [-pi, pi], together.
FRZ_HD void sincos_fixed(float angle, float* s, float* c) {
  const float k = rint_(angle * 0.63661977236758134f);
  float r = fmaf_(-k, 1.5707963705062866f, angle);
  r = fmaf_(-k, -4.3711388286737929e-08f, r);
  r = fmaf_(-k, -1.7151245100059026e-15f, r);
  const int q = (int)k & 3;
  const float sp = sin_poly(r), cp = cos_poly(r);
  switch (q) {
    case 0: *s = sp; *c = cp; break;
    case 1: *s = cp; *c = -sp; break;
    case 2: *s = -sp; *c = -cp; break;
    default: *s = -cp; *c = sp; break;
  }
}

// F16 pack (f16_pack.wgsl:16-20): saturate to +-65504, round to nearest even.
FRZ_HD uint16_t f16_pack(float x) {
  if (x != x) return 0x7E00;
  x = __builtin_fminf(__builtin_fmaxf(x, -65504.0f), 65504.0f);
  const uint32_t bits = float_to_bits(x);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t mag = bits & 0x7FFFFFFFu;
  const uint32_t e = mag >> 23;
  uint32_t h;
  if (e >= 113) {
    const uint32_t mant = mag & 0x7FFFFFu;
    h = ((e - 112) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  } else if (e >= 102) {
    const uint32_t mant = (mag & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126 - e;
    h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;
  } else {
    h = 0;
  }
  return (uint16_t)(sign | h);
}

// f16_pack on the device: the same saturation, then the hardware's f32 to
// f16 conversion, which rounds to nearest even and keeps f16 subnormals (the
// kernels run with f16 denormals on); a NaN packs as 0x7E00.
__device__ __forceinline__ uint16_t f16_pack_device(float x) {
  if (x != x) return 0x7E00;
  x = __builtin_fminf(__builtin_fmaxf(x, -65504.0f), 65504.0f);
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}

// Lane l + N of the calling lane l's 16-lane row, as a VALU operation (DPP
// row_shl; lanes past the row get 0).
template <int N>
__device__ __forceinline__ float row_shl(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x100 + N, 0xF, 0xF, true));
}

// v_permlane32_swap a, b exchanges rows 2-3 of a with rows 0-1 of b, and
// v_permlane16_swap a, b the odd rows of a with the even rows of b (a row is
// 16 lanes), both VALU operations. Written as asm with their operands named,
// so each result is the register the instruction defines; the wait states
// before them cover a VALU write of their inputs just before.
__device__ __forceinline__ float lane_plus32(float v) {
  float a = v, b = v;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return b;  // lanes 0-31: lane l + 32; lanes 32-63: their own
}

__device__ __forceinline__ float lane_plus16(float v) {
  float a = v, b = v;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return b;  // rows 0 and 2: lane l + 16; rows 1 and 3: their own
}

// The last six levels of a halving tree over a wave's 64 sums (norm.wgsl:
// 75-85): lane l adds lane l + stride for strides 32 .. 1 (32 and 16 by lane
// swaps, 8 .. 1 by DPP); lane 0's total, broadcast.
__device__ __forceinline__ float wave_tree(float s) {
  s = s + lane_plus32(s);
  s = s + lane_plus16(s);
  s = s + row_shl<8>(s);
  s = s + row_shl<4>(s);
  s = s + row_shl<2>(s);
  s = s + row_shl<1>(s);
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, s)));
}

// F16 to f32, exact, subnormals kept.
FRZ_HD float f16_unpack(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  const uint32_t mant = h & 0x3FFu;
  if (e == 0) {
    const float v = (float)mant * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (e == 31) return bits_to_float(sign | 0x7F800000u | (mant << 13));
  return bits_to_float(sign | ((e + 112) << 23) | (mant << 13));
}

// Top-k's order-preserving key of a logit's bits (topk.wgsl:32-55).
FRZ_HD uint32_t topk_key(uint32_t b) {
  if (b == 0x80000000u) b = 0;
  if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu) != 0) return 0xFFFFFFFFu;
  if (b & 0x80000000u) return ~b;
  return b | 0x80000000u;
}
FRZ_HD uint32_t topk_bits(uint32_t key) {
  if (key == 0xFFFFFFFFu) return 0x7FC00000u;
  if (key & 0x80000000u) return key & 0x7FFFFFFFu;
  return ~key;
}

}  // namespace frz
