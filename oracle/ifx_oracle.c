/*
 * CPU oracle of the FP8 quantization recipe -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this code, and only as the checker. The product path (instinctflash_amd/)
 * never links or calls it.
 *
 * Restates, in plain C with IEEE single precision (compile without fast-math
 * and with -ffp-contract=off), the reference recipe:
 *   instinctflash/kernels/fp8.py:30-37        quantize_weight (per row)
 *   instinctflash/runtime/fp8_pack.py:26-45   pack: IEEE x/scale, NaN-propagating
 *                                             clamp to +-448, RNE to E4M3
 *   instinctflash/runtime/fp8_pack.py:63-91   per-tensor amax (NaN => NaN scale),
 *                                             floor 1e-12, scale = amax * fl32(1/448)
 *   instinctflash/runtime/torch_fp8_linear.py:39-48 (the reciprocal-multiply scale)
 *
 * The E4M3 rounding here is derived from the value (frexp + nearbyint under the
 * default round-to-nearest-even mode), independently of the bit manipulation the
 * HIP kernel uses, so a mistake in one does not repeat in the other.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* OCP E4M3FN: value = (-1)^s * 2^(E-7) * (1 + m/8) for E in 1..15 (E=15,m=7 is
 * NaN), 2^-6 * m/8 for E = 0. Round to nearest, ties to even. Results above the
 * largest finite value (448) and NaN encode as NaN (0x7F | sign). */
uint8_t oracle_e4m3(float f) {
  const uint8_t s = signbit(f) ? 0x80 : 0x00;
  if (isnan(f)) return s | 0x7F;
  const double a = fabs((double)f);
  if (a < 0.015625) { /* 2^-6: subnormal step 2^-9 */
    const double n = nearbyint(a * 512.0); /* 0..8; 8 is the smallest normal */
    return s | (uint8_t)n;
  }
  int e;
  const double fr = frexp(a, &e); /* a = fr * 2^e, fr in [0.5, 1) */
  int E = e - 1;                  /* a = sig * 2^E, sig in [1, 2) */
  double steps = nearbyint((2.0 * fr - 1.0) * 8.0);
  if (steps == 8.0) {
    steps = 0.0;
    E += 1;
  }
  if (E > 8 || (E == 8 && steps > 6.0)) return s | 0x7F; /* beyond 448 */
  return s | (uint8_t)(((E + 7) << 3) | (int)steps);
}

static float scale_from_amax(float amax, int nan) {
  if (nan) return NAN;
  const float inv = 1.0f / 448.0f;
  return fmaxf(amax, 1e-12f) * inv;
}

static uint8_t pack1(float x, float scale) {
  float v = x / scale;
  if (!isnan(v)) v = fminf(fmaxf(v, -448.0f), 448.0f);
  return oracle_e4m3(v);
}

/* Per-row quantization of an f32 matrix (row stride ldx). */
void oracle_quant_rows_f32(const float* x, int64_t ldx, int64_t M, int64_t K, uint8_t* q,
                           int64_t ldq, float* scale) {
  for (int64_t m = 0; m < M; ++m) {
    const float* r = x + m * ldx;
    float amax = 0.0f;
    int nan = 0;
    for (int64_t k = 0; k < K; ++k) {
      if (isnan(r[k])) nan = 1;
      else amax = fmaxf(amax, fabsf(r[k]));
    }
    const float s = scale_from_amax(amax, nan);
    scale[m] = s;
    for (int64_t k = 0; k < K; ++k) q[m * ldq + k] = pack1(r[k], s);
  }
}

/* Per-row quantization of a bf16 matrix. */
void oracle_quant_rows_bf16(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, uint8_t* q,
                            int64_t ldq, float* scale) {
  for (int64_t m = 0; m < M; ++m) {
    const uint16_t* r = x + m * ldx;
    float amax = 0.0f;
    int nan = 0;
    for (int64_t k = 0; k < K; ++k) {
      const float v = bf16_to_f32(r[k]);
      if (isnan(v)) nan = 1;
      else amax = fmaxf(amax, fabsf(v));
    }
    const float s = scale_from_amax(amax, nan);
    scale[m] = s;
    for (int64_t k = 0; k < K; ++k) q[m * ldq + k] = pack1(bf16_to_f32(r[k]), s);
  }
}

/* Pack with a fixed scale (reference fp8_pack.py:48-60 pack_bf16_e4m3). */
void oracle_pack_bf16(const uint16_t* x, int64_t count, float scale, uint8_t* q) {
  for (int64_t i = 0; i < count; ++i) q[i] = pack1(bf16_to_f32(x[i]), scale);
}

/* Per-tensor dynamic quantization: one row holding every element. */
void oracle_quant_tensor_bf16(const uint16_t* x, int64_t count, uint8_t* q, float* scale) {
  oracle_quant_rows_bf16(x, count, 1, count, q, count, scale);
}
