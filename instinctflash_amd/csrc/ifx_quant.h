// Element arithmetic of the per-token / per-tensor E4M3 quantization recipe:
//   scale = max(amax, 1e-12) * fl32(1/448)   (NaN amax -> NaN scale)
//   q     = E4M3_RNE(clamp(x / scale, -448, 448))   with IEEE division
// (reference: runtime/fp8_pack.py:48-83, kernels/norm.py:150-176).
#pragma once

#include "ifx_device.h"

namespace ifx {

__device__ __forceinline__ void unpack_bf16x8(const uint4 r, float* v) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

__device__ __forceinline__ uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7FFFFFFFu; }

// scale from the max |x| bit pattern; NaN patterns (> +inf) give a NaN scale.
__device__ __forceinline__ float scale_from_amax_bits(uint32_t amax_bits) {
#pragma clang fp contract(off)
  if (amax_bits > 0x7F800000u) return __uint_as_float(0x7FC00000u);
  return fmaxf(__uint_as_float(amax_bits), kAmaxFloor) * kInvFp8Max;
}

// Reference-exact element path: IEEE division, NaN-propagating clamp, RNE.
__device__ __forceinline__ uint32_t q1(float v, float s) {
#pragma clang fp contract(off)
  return f32_to_e4m3(clamp_fp8(v / s));
}

// Fast path for a row whose scale s is finite (then no element is NaN or inf,
// and |x| <= amax). The correctly rounded quotient x/s comes from the row's
// correctly rounded reciprocal r = 1/s and one FMA correction (Markstein):
//   q = RN(x*r), e = RN(x - q*s) (exact), RN(q + e*r) = RN(x/s).
// Quotients small enough to be subnormal in FP32 quantize to +-0 either way.
// The correction computes (+0) + (-0) = +0 for x = -0, so the sign of x (s > 0)
// is put back. The result is clamped to +-448 and packed by the hardware E4M3
// (OCP) converter, round-to-nearest-even; tests compare every byte with the
// oracle.
__device__ __forceinline__ float div_rn(float x, float s, float r) {
#pragma clang fp contract(off)
  const float q = x * r;
  const float e = __builtin_fmaf(-q, s, x);
  return __builtin_copysignf(__builtin_fmaf(e, r, q), x);
}

__device__ __forceinline__ float clamp_finite(float v) { return fminf(fmaxf(v, -kFp8Max), kFp8Max); }

// Eight values -> eight E4M3 codes (little-endian in a uint2).
__device__ __forceinline__ uint2 pack8_fast(const float* v, float s, float r) {
  float c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = clamp_finite(div_rn(v[i], s, r));
  uint2 o;
  o.x = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false);
  o.x = __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], o.x, true);
  o.y = __builtin_amdgcn_cvt_pk_fp8_f32(c[4], c[5], 0, false);
  o.y = __builtin_amdgcn_cvt_pk_fp8_f32(c[6], c[7], o.y, true);
  return o;
}

__device__ __forceinline__ uint2 pack8_exact(const float* v, float s) {
  uint2 o;
  o.x = q1(v[0], s) | (q1(v[1], s) << 8) | (q1(v[2], s) << 16) | (q1(v[3], s) << 24);
  o.y = q1(v[4], s) | (q1(v[5], s) << 8) | (q1(v[6], s) << 16) | (q1(v[7], s) << 24);
  return o;
}

// Byte offset of element (m, k) (k % 8 == 0) in the skinny tile layout with ks
// K steps per 16-row block: tile (m/16, k/128) of 2 KB, lane l = 16*((k%128)/32)
// + m%16 holds K bytes [32*(l/16), +16) at 16l and the next 16 at 1024 + 16l.
__device__ __forceinline__ int64_t tile_offset(int64_t m, int64_t k, int64_t ks) {
  return ((m >> 4) * ks + (k >> 7)) * 2048 + ((k >> 4) & 1) * 1024 + ((((k >> 5) & 3) << 4) + (m & 15)) * 16 +
         (k & 15);
}

__device__ __forceinline__ bool finite_scale(float s) { return (__float_as_uint(s) & 0x7F800000u) != 0x7F800000u; }

}  // namespace ifx
