// QKV split consumer for gfx950: a fused QKV projection's raw accumulator
// [T, (HQ + 2*HKV) * HD] is rescaled (row / column dequantization scales, bias),
// query and key heads optionally RMS-normalized per head (q_norm / k_norm
// weights), rotated (rotary embedding, split-half pairing: element i pairs with
// i + HD/2), and stored: Q to q_out[t, h], K and V to KV-cache rows
// k_out / v_out[kv_base + t, h].
//
// Reference: instinctflash/kernels/rope.py:21-80 (`_qkv_split_kernel`) and
// :89-116 (`qkv_split`). Rotary angles are FP32 products pos[t, section[i]] *
// inv_freq[i] as there (rope.py:60-64); cos/sin are the accurate library
// functions, not the hardware approximations, since angles reach thousands of
// radians. kv_base may be a device int32 (graph-captured decode steps).
//
// Layout: one 4-wave workgroup per token, waves looping over its heads; lane l
// holds the pairs (i, i + HD/2) for i = l, l + 64 (HD <= 256), and the rotary
// cos/sin of its i are computed once per wave. Row loads/stores are
// lane-consecutive elements.

#include "ifx_abi.h"
#include "ifx_device.h"

#pragma clang fp contract(off)

namespace ifx {
namespace {

constexpr int kWavesPerBlock = 4;

struct QkvArgs {
  const void* qkv;
  int64_t ldqkv;
  const float* row;
  const float* col;
  const float* bias;
  const float* qnw;
  const float* knw;
  float eps;
  const float* inv_freq;
  const float* pos;
  int64_t ldpos;
  const int32_t* sections;
  void* q;
  int64_t sq_t, sq_h;
  void* k;
  int64_t sk_t, sk_h;
  void* v;
  int64_t sv_t, sv_h;
  int64_t kv_base;
  const int32_t* kv_base_dev;
  int64_t T, HQ, HKV, HD;
  int in_f32;
  int out_dtype;
};

__device__ __forceinline__ float load_in(const QkvArgs& a, int64_t idx) {
  if (a.in_f32) return static_cast<const float*>(a.qkv)[idx];
  return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(a.qkv)[idx]) << 16);
}

__device__ __forceinline__ void store_out(const QkvArgs& a, void* base, int64_t idx, float v) {
  if (a.out_dtype == IFX_DTYPE_F32) {
    static_cast<float*>(base)[idx] = v;
  } else if (a.out_dtype == IFX_DTYPE_F16) {
    static_cast<_Float16*>(base)[idx] = static_cast<_Float16>(v);
  } else {
    static_cast<__bf16*>(base)[idx] = static_cast<__bf16>(v);
  }
}

// One workgroup per token; wave w handles heads w, w + 4, ... Each lane holds
// the pairs (i, i + HD/2) for i = lane + 64 j; the rotary cos/sin of its i are
// computed once per wave and reused for every head of the token.
template <int NJ>
__global__ __launch_bounds__(64 * kWavesPerBlock) void qkv_split_kernel(QkvArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t t = blockIdx.x;
  const int64_t H = a.HQ + 2 * a.HKV;
  const int64_t half = a.HD / 2;
  const float r = a.row ? a.row[t] : 1.0f;
  const int64_t krow = (a.kv_base_dev ? static_cast<int64_t>(*a.kv_base_dev) : a.kv_base) + t;

  bool on[NJ];
  float cs[NJ], sn[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t i = lane + 64 * j;
    on[j] = i < half;
    cs[j] = 1.0f;
    sn[j] = 0.0f;
    if (on[j] && a.inv_freq) {
      const int64_t sec = a.sections ? a.sections[i] : 0;
      const float ang = a.pos[t * a.ldpos + sec] * a.inv_freq[i];
      sincosf(ang, &sn[j], &cs[j]);
    }
  }

  for (int64_t h = wave; h < H; h += kWavesPerBlock) {
    float lo[NJ], hi[NJ];
    const int64_t base = t * a.ldqkv + h * a.HD;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int64_t i = lane + 64 * j;
      lo[j] = hi[j] = 0.0f;
      if (!on[j]) continue;
      lo[j] = load_in(a, base + i);
      hi[j] = load_in(a, base + half + i);
      if (a.row) {
        lo[j] = lo[j] * r;
        hi[j] = hi[j] * r;
      }
      if (a.col) {
        lo[j] = lo[j] * a.col[h * a.HD + i];
        hi[j] = hi[j] * a.col[h * a.HD + half + i];
      }
      if (a.bias) {
        lo[j] = lo[j] + a.bias[h * a.HD + i];
        hi[j] = hi[j] + a.bias[h * a.HD + half + i];
      }
    }
    if (h < a.HQ + a.HKV) {  // wave-uniform
      if (a.qnw) {  // q_norm and k_norm come together
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < NJ; ++j) ss = ss + (lo[j] * lo[j] + hi[j] * hi[j]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ss = ss + __shfl_xor(ss, off, 64);
        const float rs = 1.0f / __builtin_sqrtf(ss / static_cast<float>(a.HD) + a.eps);
        const float* w = h < a.HQ ? a.qnw : a.knw;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          if (!on[j]) continue;
          const int64_t i = lane + 64 * j;
          lo[j] = lo[j] * rs * w[i];
          hi[j] = hi[j] * rs * w[half + i];
        }
      }
      if (a.inv_freq) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const float rlo = lo[j] * cs[j] - hi[j] * sn[j];
          hi[j] = hi[j] * cs[j] + lo[j] * sn[j];
          lo[j] = rlo;
        }
      }
    }
    void* dst;
    int64_t off;
    if (h < a.HQ) {
      dst = a.q;
      off = t * a.sq_t + h * a.sq_h;
    } else if (h < a.HQ + a.HKV) {
      dst = a.k;
      off = krow * a.sk_t + (h - a.HQ) * a.sk_h;
    } else {
      dst = a.v;
      off = krow * a.sv_t + (h - a.HQ - a.HKV) * a.sv_h;
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (!on[j]) continue;
      const int64_t i = lane + 64 * j;
      store_out(a, dst, off + i, lo[j]);
      store_out(a, dst, off + half + i, hi[j]);
    }
  }
}

}  // namespace
}  // namespace ifx

using namespace ifx;

extern "C" {

int ifx_qkv_split(const void* qkv, int qkv_dtype, int64_t ldqkv, const float* row, const float* col,
                  const float* bias, const float* q_norm, const float* k_norm, float eps, const float* inv_freq,
                  const float* pos, int64_t ldpos, const int32_t* sections, void* q_out, int64_t sq_t,
                  int64_t sq_h, void* k_out, int64_t sk_t, int64_t sk_h, void* v_out, int64_t sv_t, int64_t sv_h,
                  int out_dtype, int64_t kv_base, const int32_t* kv_base_dev, int64_t T, int64_t HQ, int64_t HKV,
                  int64_t HD, void* stream) {
  if (qkv_dtype != IFX_DTYPE_BF16 && qkv_dtype != IFX_DTYPE_F32) return IFX_ERR_INVALID;
  if (out_dtype != IFX_DTYPE_BF16 && out_dtype != IFX_DTYPE_F32 && out_dtype != IFX_DTYPE_F16) return IFX_ERR_INVALID;
  if (T < 0 || HQ <= 0 || HKV <= 0 || HD <= 0 || HD % 2 != 0) return IFX_ERR_INVALID;
  if (HD > 256) return IFX_ERR_UNSUPPORTED;
  if (ldqkv < (HQ + 2 * HKV) * HD) return IFX_ERR_INVALID;
  if ((q_norm == nullptr) != (k_norm == nullptr)) return IFX_ERR_INVALID;
  if (inv_freq && (!pos || ldpos < 1)) return IFX_ERR_INVALID;
  if (!(eps >= 0.0f) || kv_base < 0) return IFX_ERR_INVALID;
  if (T == 0) return IFX_OK;
  if (!qkv || !q_out || !k_out || !v_out) return IFX_ERR_INVALID;
  QkvArgs a{qkv,  ldqkv, row, col,  bias, q_norm, k_norm, eps,  inv_freq,    pos, ldpos, sections,
            q_out, sq_t, sq_h, k_out, sk_t, sk_h,   v_out,  sv_t, sv_h,        kv_base, kv_base_dev,
            T,    HQ,    HKV, HD,   qkv_dtype == IFX_DTYPE_F32 ? 1 : 0,         out_dtype};
  const int64_t blocks = T;  // one workgroup per token
  if (blocks > 0x7FFFFFFFLL) return IFX_ERR_UNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (HD / 2 <= 64)
    hipLaunchKernelGGL(qkv_split_kernel<1>, dim3(static_cast<unsigned>(blocks)), dim3(64 * kWavesPerBlock), 0, st, a);
  else
    hipLaunchKernelGGL(qkv_split_kernel<2>, dim3(static_cast<unsigned>(blocks)), dim3(64 * kWavesPerBlock), 0, st, a);
  return launch_status();
}

}  // extern "C"
