// Pre-norm producer for gfx950: residual update, RMS / LayerNorm, affine and
// adaptive (adaLN) modulation, and per-row FP8 E4M3 quantization, in one pass
// over each row:
//
//   if delta:  res[m] += (delta[m] * delta_row[m] * delta_col + bias) * gate
//   y[m] = norm(res[m])                          RMS, or mean-centred LayerNorm
//   y[m] = y[m] * weight + beta                  optional learned affine
//   y[m] = y[m] * (1 + mod_scale) + mod_shift    optional adaptive modulation
//   q[m], q_scale[m] = E4M3 recipe of y[m]       optional; y[m] optionally stored
//
// Reference: instinctflash/kernels/norm.py:25-94 (`residual_norm_quant`). The
// residual sum is formed in FP32 and the value stored in res's dtype (FP32, or
// BF16 for the LingBot-VA engine) is the one normalized (norm.py:55-57); gate,
// mod_scale and mod_shift may be per-row tables selected by mod_index
// (norm.py:38-42). Quantization follows this package's recipe
// (scale = max(amax, 1e-12) * fl32(1/448), IEEE division, RNE) like every other
// quantizer here, instead of the Triton kernel's 1e-8 floor and 448/amax
// multiply (norm.py:80-83).
//
// Design (HBM-bound: res read + written, delta read, q written): a 256-lane
// workgroup owns one row, the row stays in registers (VPT groups of 8 elements
// per lane, 16/32-byte loads), and the two LayerNorm reductions run on the
// registers. The element arithmetic of the residual update is evaluated in the
// reference's order with no contraction, so res is reproducible bit for bit.

#include "ifx_abi.h"
#include "ifx_device.h"
#include "ifx_quant.h"

#pragma clang fp contract(off)

namespace ifx {
namespace {

constexpr int kRnqThreads = 256;

struct RnqArgs {
  void* res;
  int64_t ldres;
  const void* delta;
  int64_t lddelta;
  const float* drow;
  const float* dcol;
  const float* bias;
  const float* gate;
  const float* weight;
  const float* beta;
  const float* mscale;
  const float* mshift;
  const int32_t* mod_index;
  void* y;
  int64_t ldy;
  uint8_t* q;
  int64_t ldq;
  float* qs;
  int64_t D;
  float eps;
  int flags;
  int y_f32;
};

__device__ __forceinline__ void load8_bf16(const void* p, float* v) {
  unpack_bf16x8(*reinterpret_cast<const uint4*>(p), v);
}

__device__ __forceinline__ void load8_f32(const void* p, float* v) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ void store8_f32(void* p, const float* v) {
  reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

__device__ __forceinline__ void store8_bf16(void* p, const float* v) {
  *reinterpret_cast<uint4*>(p) =
      make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
}

// Workgroup-wide FP32 sum in a fixed order (per-lane, then wave butterfly,
// then the 4 wave totals in wave order): deterministic.
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  __syncthreads();  // red may still be read by a previous reduction
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = red[0];
#pragma unroll
  for (int w = 1; w < kRnqThreads / 64; ++w) s += red[w];
  return s;
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
  v = wave_max_u32(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t m = red[0];
#pragma unroll
  for (int w = 1; w < kRnqThreads / 64; ++w) m = m > red[w] ? m : red[w];
  return m;
}

template <int VPT, bool RES_BF16, bool DELTA_BF16>
__global__ __launch_bounds__(kRnqThreads) void residual_norm_quant_kernel(RnqArgs a) {
  __shared__ float red[kRnqThreads / 64];
  const int64_t row = blockIdx.x;
  const int64_t D = a.D;
  const int64_t mofs = a.mod_index ? static_cast<int64_t>(a.mod_index[row]) * D : 0;
  const bool has_delta = a.delta != nullptr;
  const bool layernorm = (a.flags & IFX_RNQ_LAYERNORM) != 0;

  float x[VPT][8];
  bool on[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t c = (static_cast<int64_t>(j) * kRnqThreads + threadIdx.x) * 8;
    on[j] = c < D;
    if (!on[j]) {
#pragma unroll
      for (int t = 0; t < 8; ++t) x[j][t] = 0.0f;
      continue;
    }
    if constexpr (RES_BF16) load8_bf16(static_cast<const uint16_t*>(a.res) + row * a.ldres + c, x[j]);
    else load8_f32(static_cast<const float*>(a.res) + row * a.ldres + c, x[j]);
    if (has_delta) {
      float d[8];
      if constexpr (DELTA_BF16) load8_bf16(static_cast<const uint16_t*>(a.delta) + row * a.lddelta + c, d);
      else load8_f32(static_cast<const float*>(a.delta) + row * a.lddelta + c, d);
      if (a.drow) {
        const float r = a.drow[row];
#pragma unroll
        for (int t = 0; t < 8; ++t) d[t] = d[t] * r;
      }
      float v[8];
      if (a.dcol) {
        load8_f32(a.dcol + c, v);
#pragma unroll
        for (int t = 0; t < 8; ++t) d[t] = d[t] * v[t];
      }
      if (a.bias) {
        load8_f32(a.bias + c, v);
#pragma unroll
        for (int t = 0; t < 8; ++t) d[t] = d[t] + v[t];
      }
      if (a.gate) {
        load8_f32(a.gate + mofs + c, v);
#pragma unroll
        for (int t = 0; t < 8; ++t) d[t] = d[t] * v[t];
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) x[j][t] = x[j][t] + d[t];
      if (a.flags & IFX_RNQ_WRITE_RES) {
        if constexpr (RES_BF16) {
          void* p = static_cast<uint16_t*>(a.res) + row * a.ldres + c;
          store8_bf16(p, x[j]);
          load8_bf16(p, x[j]);  // normalize the stored (rounded) value
        } else {
          store8_f32(static_cast<float*>(a.res) + row * a.ldres + c, x[j]);
        }
      }  // without the write the FP32 sum is normalized (norm.py:55-57 rounds only what it stores)
    }
  }

  // Normalization statistics over the row (masked lanes hold 0).
  float part = 0.0f;
#pragma unroll
  for (int j = 0; j < VPT; ++j)
#pragma unroll
    for (int t = 0; t < 8; ++t) part = part + x[j][t];
  float rstd;
  if (layernorm) {
    const float mean = block_sum(part, red) / static_cast<float>(D);
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      if (!on[j]) continue;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        x[j][t] = x[j][t] - mean;
        sq = sq + x[j][t] * x[j][t];
      }
    }
    const float var = block_sum(sq, red) / static_cast<float>(D);
    rstd = 1.0f / __builtin_sqrtf(var + a.eps);
  } else {
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j)
#pragma unroll
      for (int t = 0; t < 8; ++t) sq = sq + x[j][t] * x[j][t];
    const float var = block_sum(sq, red) / static_cast<float>(D);
    rstd = 1.0f / __builtin_sqrtf(var + a.eps);
  }

  uint32_t amax = 0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    if (!on[j]) continue;
    const int64_t c = (static_cast<int64_t>(j) * kRnqThreads + threadIdx.x) * 8;
    float v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) x[j][t] = x[j][t] * rstd;
    if (a.weight) {
      load8_f32(a.weight + c, v);
#pragma unroll
      for (int t = 0; t < 8; ++t) x[j][t] = x[j][t] * v[t];
    }
    if (a.beta) {
      load8_f32(a.beta + c, v);
#pragma unroll
      for (int t = 0; t < 8; ++t) x[j][t] = x[j][t] + v[t];
    }
    if (a.mscale) {
      float h[8];
      load8_f32(a.mscale + mofs + c, v);
      load8_f32(a.mshift + mofs + c, h);
#pragma unroll
      for (int t = 0; t < 8; ++t) x[j][t] = x[j][t] * (1.0f + v[t]) + h[t];
    }
    if (a.y) {
      if (a.y_f32) store8_f32(static_cast<float*>(a.y) + row * a.ldy + c, x[j]);
      else store8_bf16(static_cast<uint16_t*>(a.y) + row * a.ldy + c, x[j]);
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint32_t b = abs_bits(x[j][t]);
      amax = amax > b ? amax : b;
    }
  }
  if (!a.q) return;

  amax = block_max_u32(amax, reinterpret_cast<uint32_t*>(red));
  const float s = scale_from_amax_bits(amax);
  if (threadIdx.x == 0) a.qs[row] = s;
  const bool fast = finite_scale(s);
  const float r = 1.0f / s;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    if (!on[j]) continue;
    const int64_t c = (static_cast<int64_t>(j) * kRnqThreads + threadIdx.x) * 8;
    *reinterpret_cast<uint2*>(a.q + row * a.ldq + c) = fast ? pack8_fast(x[j], s, r) : pack8_exact(x[j], s);
  }
}

template <int VPT>
void launch_rnq(const RnqArgs& a, int64_t M, bool res_bf16, bool delta_bf16, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(M)), block(kRnqThreads);
  if (res_bf16) {
    if (delta_bf16) hipLaunchKernelGGL((residual_norm_quant_kernel<VPT, true, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((residual_norm_quant_kernel<VPT, true, false>), grid, block, 0, st, a);
  } else {
    if (delta_bf16) hipLaunchKernelGGL((residual_norm_quant_kernel<VPT, false, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((residual_norm_quant_kernel<VPT, false, false>), grid, block, 0, st, a);
  }
}

bool aligned_vec(const void* p) { return p == nullptr || aligned16(p); }

}  // namespace
}  // namespace ifx

using namespace ifx;

extern "C" {

int ifx_residual_norm_quant(void* res, int res_dtype, int64_t ldres, const void* delta, int delta_dtype,
                            int64_t lddelta, const float* delta_row, const float* delta_col, const float* bias,
                            const float* gate, const float* weight, const float* beta, const float* mod_scale,
                            const float* mod_shift, const int32_t* mod_index, int flags, float eps, void* q,
                            int64_t ldq, float* q_scale, void* y, int y_dtype, int64_t ldy, int64_t M, int64_t D,
                            void* stream) {
  constexpr int kKnown = IFX_RNQ_WRITE_RES | IFX_RNQ_LAYERNORM;
  if (flags & ~kKnown) return IFX_ERR_INVALID;
  auto dtype_ok = [](int d) { return d == IFX_DTYPE_BF16 || d == IFX_DTYPE_F32; };
  if (!dtype_ok(res_dtype) || (delta && !dtype_ok(delta_dtype)) || (y && !dtype_ok(y_dtype))) return IFX_ERR_INVALID;
  if (M < 0 || D <= 0 || D % 8 != 0) return IFX_ERR_INVALID;
  if (D > static_cast<int64_t>(kRnqThreads) * 8 * 8) return IFX_ERR_UNSUPPORTED;
  if (ldres < D || (delta && lddelta < D) || (q && ldq < D) || (y && ldy < D)) return IFX_ERR_INVALID;
  if ((mod_scale == nullptr) != (mod_shift == nullptr)) return IFX_ERR_INVALID;
  if (q && !q_scale) return IFX_ERR_INVALID;
  if (!(eps >= 0.0f)) return IFX_ERR_INVALID;
  if (M == 0) return IFX_OK;
  if (!res) return IFX_ERR_INVALID;
  if (!aligned16(res) || ldres % 8 != 0 || !aligned_vec(delta) || (delta && lddelta % 8 != 0) ||
      !aligned_vec(y) || (y && ldy % 8 != 0) || (q && ((reinterpret_cast<uintptr_t>(q) & 7u) || ldq % 8 != 0)))
    return IFX_ERR_ALIGN;
  for (const float* v : {delta_col, bias, gate, weight, beta, mod_scale, mod_shift})
    if (!aligned_vec(v)) return IFX_ERR_ALIGN;

  RnqArgs a{res, ldres, delta, lddelta, delta_row, delta_col, bias, gate, weight, beta, mod_scale, mod_shift,
            mod_index, y, ldy, static_cast<uint8_t*>(q), ldq, q_scale, D, eps, delta ? flags : (flags & ~IFX_RNQ_WRITE_RES),
            y_dtype == IFX_DTYPE_F32 ? 1 : 0};
  const bool rb = res_dtype == IFX_DTYPE_BF16, db = delta_dtype == IFX_DTYPE_BF16;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t groups = (D / 8 + kRnqThreads - 1) / kRnqThreads;  // 8-element groups per lane
  if (groups <= 1) launch_rnq<1>(a, M, rb, db, st);
  else if (groups <= 2) launch_rnq<2>(a, M, rb, db, st);
  else if (groups <= 4) launch_rnq<4>(a, M, rb, db, st);
  else launch_rnq<8>(a, M, rb, db, st);
  return launch_status();
}

}  // extern "C"
