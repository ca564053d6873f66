// Device-side helpers shared by the FP8 projection kernels (gfx950 only).
//
// * OCP E4M3FN encoding (bias 7, no infinities, 0x7F/0xFF = NaN, max finite 448)
//   written from the OCP 8-bit floating point specification: round to nearest,
//   ties to even, on the FP32 bit pattern.
// * BF16 <-> FP32 bit helpers.
// * MFMA fragment types for v_mfma_f32_{16x16x128,32x32x64}_f8f6f4.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ifx {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Largest finite E4M3FN magnitude.
constexpr float kFp8Max = 448.0f;
// The activation/weight scale is amax * fl32(1/448): this is how a device
// division by a host scalar is evaluated (multiply by the FP32 reciprocal),
// which the reference recipe relies on (instinctflash/runtime/fp8_pack.py:88-89,
// tests/test_sm89_fp8.py:48-56). The constant is the correctly rounded FP32
// reciprocal of 448.
constexpr float kInvFp8Max = 1.0f / 448.0f;
// Scale floor of the recipe (instinctflash/kernels/fp8.py:33 clamp_min(1e-12)).
constexpr float kAmaxFloor = 1e-12f;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// FP32 -> BF16 bits, round to nearest even; NaN stays NaN (quiet bit forced).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two FP32 -> packed BF16 (lo in bits 0..15), round to nearest even: one
// v_cvt_pk_bf16_f32 on gfx950 (NaN stays NaN).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// FP32 -> E4M3FN byte, round-to-nearest-even.
//  * |f| >= 2^-6 (normal range): keep 3 mantissa bits of the FP32 pattern with
//    RNE, then rebias the exponent from 127 to 7 (127-7 = 120 -> 120<<3 = 960
//    in the >>20 domain).
//  * |f| <  2^-6: the E4M3 subnormal step is 2^-9, so the code is the integer
//    RNE(|f| * 2^9); code 8 coincides with the smallest normal (exp 1, mant 0).
//  * Magnitudes whose rounding leaves the finite range (above 464, the tie
//    that rounds to even 448), infinities and NaN encode as NaN (0x7F) with the
//    input's sign. Callers clamp finite inputs to +-448 first, so only NaN
//    reaches that case.
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  uint32_t code;
  if (a >= 0x43F00000u) {            // >= 480.0 (incl. inf/NaN); (464,480) -> 0x7F below
    code = 0x7Fu;
  } else if (a >= 0x3C800000u) {     // >= 2^-6
    code = ((a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20) - 960u;
  } else {
    const uint32_t e = a >> 23;      // 0 .. 120
    // value = m * 2^(e-150) for normal FP32 (m with implicit bit); we need
    // RNE(value * 2^9) = RNE(m * 2^-(141-e)). FP32 subnormals and anything
    // below 2^-11 round to zero.
    if (e < 115u) {
      code = 0u;
    } else {
      const uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
      const uint32_t sh = 141u - e;  // 21 .. 26
      code = (m + (1u << (sh - 1u)) - 1u + ((m >> sh) & 1u)) >> sh;
    }
  }
  return code | sign;
}

// NaN-propagating clamp to [-448, 448] (a NaN input stays NaN).
__device__ __forceinline__ float clamp_fp8(float v) {
  return v != v ? v : fminf(fmaxf(v, -kFp8Max), kFp8Max);
}

// Wave-wide (64 lanes) reductions through DPP lane moves within each 16-lane
// row (quad swaps, then the half-row and row mirrors), then the four row
// results read as scalars: no LDS round trips, and every lane returns the same
// value in a fixed combination order. All 64 lanes must be active.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), CTRL, 0xF,
                                                           0xF, false));
}

constexpr int kDppQuadSwap1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror
constexpr int kDppRowMirror = 0x140;  // row_mirror

__device__ __forceinline__ uint32_t row_lane(uint32_t v, int lane) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  auto mx = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  v = mx(v, dpp_u32<kDppQuadSwap1>(v));
  v = mx(v, dpp_u32<kDppQuadSwap2>(v));
  v = mx(v, dpp_u32<kDppHalfMirror>(v));
  v = mx(v, dpp_u32<kDppRowMirror>(v));
  return mx(mx(row_lane(v, 0), row_lane(v, 16)), mx(row_lane(v, 32), row_lane(v, 48)));
}

__device__ __forceinline__ float wave_sum_f32(float v) {
  v = v + __uint_as_float(dpp_u32<kDppQuadSwap1>(__float_as_uint(v)));
  v = v + __uint_as_float(dpp_u32<kDppQuadSwap2>(__float_as_uint(v)));
  v = v + __uint_as_float(dpp_u32<kDppHalfMirror>(__float_as_uint(v)));
  v = v + __uint_as_float(dpp_u32<kDppRowMirror>(__float_as_uint(v)));
  const uint32_t b = __float_as_uint(v);
  return (__uint_as_float(row_lane(b, 0)) + __uint_as_float(row_lane(b, 16))) +
         (__uint_as_float(row_lane(b, 32)) + __uint_as_float(row_lane(b, 48)));
}

typedef __attribute__((address_space(3))) void* lds_void_ptr;

// LDS byte offset of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_ptr)(p)));
}

// One global_load_lds_dwordx4: 64 lanes x 16 bytes from `src` (per lane) into
// the 1 KB LDS block at byte offset `lds` (wave-uniform, via M0). Written as
// inline asm on purpose: the compiler does not know this instruction writes
// LDS, so it does not put an s_waitcnt vmcnt(0) in front of every later LDS
// read "in case they alias" -- that wait would also drain the loads of the
// stages that are meant to stay in flight. The caller orders the DMA and the
// LDS reads itself (s_waitcnt vmcnt(N) + s_barrier before each stage is read;
// vector-memory loads complete in issue order, so the compiler's own vmcnt
// counts for other loads stay conservative).
__device__ __forceinline__ void dma16(const uint8_t* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(src) : "memory", "m0");
}

// dma16 with the address split into a wave-uniform base (SGPR pair) and a
// per-lane 32-bit byte offset: one VGPR per source instead of two.
__device__ __forceinline__ void dma16s(const uint8_t* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(off), "s"(base) : "memory", "m0");
}

// s_waitcnt vmcnt(N) for a compile-time N (0..63).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Rotary pair: (lo, hi) -> (lo*c - hi*s, hi*c + lo*s), each product rounded
// on its own (no fused multiply-add), so every kernel that rotates a pair
// produces the same bits.
__device__ __forceinline__ void rotate_pair(float& lo, float& hi, float c, float s) {
#pragma clang fp contract(off)
  const float l = lo * c - hi * s;
  const float h = hi * c + lo * s;
  lo = l;
  hi = h;
}

// GELU, tanh form: 0.5*x*(1+tanh(u)), u = sqrt(2/pi)*(x + 0.044715 x^3).
// Since 0.5*(1+tanh(u)) = 1/(1+e^{-2u}), this is x / (1 + 2^z) with
// z = -2u*log2(e) = x*(a + b*x^2): one FMA-based polynomial, one exp2 and one
// reciprocal (hardware approximations, ~1 ulp each).
__device__ __forceinline__ float gelu_tanh(float x) {
  constexpr float a = -2.0 * 0.7978845608028654 * 1.4426950408889634;
  constexpr float b = a * 0.044715;
  const float z = x * __builtin_fmaf(b, x * x, a);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z));
}

__device__ __forceinline__ float silu(float x) {
  const float e = __builtin_amdgcn_exp2f(-x * 1.4426950408889634f);  // e^{-x}
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

}  // namespace ifx
