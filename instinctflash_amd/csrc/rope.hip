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
// Layout: one 4-wave workgroup per (token, group of 4 heads), one head per
// wave; lane l holds the pairs (i, i + HD/2) for i = l, l + 64 (HD <= 256).
// A wave issues all loads of its head before the arithmetic. Row loads/stores
// are lane-consecutive elements.

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

__device__ __forceinline__ void store_out(int out_dtype, void* base, int64_t idx, float v) {
  if (out_dtype == IFX_DTYPE_F32) {
    static_cast<float*>(base)[idx] = v;
  } else if (out_dtype == IFX_DTYPE_F16) {
    static_cast<_Float16*>(base)[idx] = static_cast<_Float16>(v);
  } else {
    static_cast<__bf16*>(base)[idx] = static_cast<__bf16>(v);
  }
}

// Eight consecutive values at a 16-byte aligned element index.
__device__ __forceinline__ void load8(const void* base, bool f32, int64_t idx, float* v) {
  if (f32) {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 r = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + idx);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
}

__device__ __forceinline__ void load8_f32(const float* p, float* v) { load8(p, true, 0, v); }

__device__ __forceinline__ void store8(int out_dtype, void* base, int64_t idx, const float* v) {
  if (out_dtype == IFX_DTYPE_F32) {
    float* p = static_cast<float*>(base) + idx;
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else if (out_dtype == IFX_DTYPE_F16) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = static_cast<_Float16>(v[i]);
    *reinterpret_cast<h8*>(static_cast<_Float16*>(base) + idx) = h;
  } else {
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + idx) =
        make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
  }
}

// Workgroup (t, g) handles token t; its wave w handles head 4g + w. Each lane
// holds the pairs (i, i + HD/2) for i = lane + 64 j and computes the rotary
// cos/sin of its i.
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

  {
    // one head per wave: head blockIdx.y * waves + wave
    const int64_t h = static_cast<int64_t>(blockIdx.y) * kWavesPerBlock + wave;
    if (h >= H) return;  // wave-uniform; no workgroup barrier follows
    float lo[NJ], hi[NJ], cl[NJ], ch[NJ], bl[NJ], bh[NJ];
    const int64_t base = t * a.ldqkv + h * a.HD;
    // all loads of the head first (clamped in-row indices, no per-element branch)
    if (a.in_f32) {
      const float* x = static_cast<const float*>(a.qkv) + base;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int64_t i = on[j] ? lane + 64 * j : 0;
        lo[j] = x[i];
        hi[j] = x[half + i];
      }
    } else {
      const uint16_t* x = static_cast<const uint16_t*>(a.qkv) + base;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int64_t i = on[j] ? lane + 64 * j : 0;
        lo[j] = __uint_as_float(static_cast<uint32_t>(x[i]) << 16);
        hi[j] = __uint_as_float(static_cast<uint32_t>(x[half + i]) << 16);
      }
    }
    if (a.col)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int64_t i = on[j] ? lane + 64 * j : 0;
        cl[j] = a.col[h * a.HD + i];
        ch[j] = a.col[h * a.HD + half + i];
      }
    if (a.bias)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int64_t i = on[j] ? lane + 64 * j : 0;
        bl[j] = a.bias[h * a.HD + i];
        bh[j] = a.bias[h * a.HD + half + i];
      }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (a.row) {
        lo[j] = lo[j] * r;
        hi[j] = hi[j] * r;
      }
      if (a.col) {
        lo[j] = lo[j] * cl[j];
        hi[j] = hi[j] * ch[j];
      }
      if (a.bias) {
        lo[j] = lo[j] + bl[j];
        hi[j] = hi[j] + bh[j];
      }
      if (!on[j]) lo[j] = hi[j] = 0.0f;
    }
    if (h < a.HQ + a.HKV) {  // wave-uniform
      if (a.qnw) {  // q_norm and k_norm come together
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < NJ; ++j) ss = ss + (lo[j] * lo[j] + hi[j] * hi[j]);
        ss = wave_sum_f32(ss);
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
        for (int j = 0; j < NJ; ++j) rotate_pair(lo[j], hi[j], cs[j], sn[j]);
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
      store_out(a.out_dtype, dst, off + i, lo[j]);
      store_out(a.out_dtype, dst, off + half + i, hi[j]);
    }
  }
}

// ---------------------------------------------------------------------------
// Wan DiT QKV consumer (reference instinctflash/kernels/wan.py:19-116): parts
// Q | K | V of a raw accumulator row, each H*HD wide. Q and K are RMS-normalized
// over their full width (before the head split) and rotated on adjacent channel
// pairs (2j, 2j+1) of every head by pos[t, section[j]] * inv_freq[j]; Q is stored
// densely, K / V into per-batch pools at row slots[t] (t = row % tokens).
// One 256-lane workgroup per (row, part); 8-element groups per lane (4 pairs);
// the row's HD/2 cos/sin values are computed once into LDS.
// ---------------------------------------------------------------------------

struct WanArgs {
  const void* raw;
  int64_t ldraw;
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
  int64_t sq;
  void* kp;
  int64_t sk_b, sk_s;
  void* vp;
  int64_t sv_b, sv_s;
  const int32_t* slots;
  int64_t tokens, D, HD;
  int has_k, has_v;
  int in_f32;
  int out_dtype;
};

template <int VPT>
__global__ __launch_bounds__(256) void wan_qkv_kernel(WanArgs a) {
  __shared__ float red[4];
  __shared__ float cs[128], sn[128];
  const int64_t row = blockIdx.x;
  const int part = blockIdx.y;  // 0 = Q, 1 = K, 2 = V
  if ((part == 1 && !a.has_k) || (part == 2 && !a.has_v)) return;  // block-uniform
  const int64_t b = row / a.tokens, t = row - b * a.tokens;
  const int64_t D = a.D, half = a.HD / 2;
  const bool rope = a.inv_freq != nullptr && part < 2;
  const float* nw = part == 0 ? a.qnw : (part == 1 ? a.knw : nullptr);
  if (rope) {
    for (int64_t j = threadIdx.x; j < half; j += 256) {
      const int64_t sec = a.sections ? a.sections[j] : 0;
      sincosf(a.pos[t * a.ldpos + sec] * a.inv_freq[j], &sn[j], &cs[j]);
    }
  }
  const int64_t col0 = part * D;
  const float r = a.row ? a.row[row] : 1.0f;
  float x[VPT][8];
  bool on[VPT];
  float ss = 0.0f;
#pragma unroll
  for (int jv = 0; jv < VPT; ++jv) {
    const int64_t c = (static_cast<int64_t>(jv) * 256 + threadIdx.x) * 8;
    on[jv] = c < D;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[jv][e] = 0.0f;
    if (!on[jv]) continue;
    load8(a.raw, a.in_f32 != 0, row * a.ldraw + col0 + c, x[jv]);
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[jv][e] = x[jv][e] * r;
    if (a.col) {
      load8_f32(a.col + col0 + c, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[jv][e] = x[jv][e] * v[e];
    }
    if (a.bias) {
      load8_f32(a.bias + col0 + c, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[jv][e] = x[jv][e] + v[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = ss + x[jv][e] * x[jv][e];
  }
  if (nw) {  // block-uniform
    ss = wave_sum_f32(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = red[0] + red[1] + red[2] + red[3];
    const float rs = 1.0f / __builtin_sqrtf(tot / static_cast<float>(D) + a.eps);
#pragma unroll
    for (int jv = 0; jv < VPT; ++jv) {
      if (!on[jv]) continue;
      const int64_t c = (static_cast<int64_t>(jv) * 256 + threadIdx.x) * 8;
      float w[8];
      load8_f32(nw + c, w);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[jv][e] = x[jv][e] * rs * w[e];
    }
  }
  if (rope) __syncthreads();  // the cos/sin table is complete
  void* dst;
  int64_t base;
  if (part == 0) {
    dst = a.q;
    base = row * a.sq;
  } else {
    const int64_t slot = a.slots ? static_cast<int64_t>(a.slots[t]) : t;
    dst = part == 1 ? a.kp : a.vp;
    base = part == 1 ? b * a.sk_b + slot * a.sk_s : b * a.sv_b + slot * a.sv_s;
  }
#pragma unroll
  for (int jv = 0; jv < VPT; ++jv) {
    if (!on[jv]) continue;
    const int64_t c = (static_cast<int64_t>(jv) * 256 + threadIdx.x) * 8;
    if (rope) {
      const int64_t j0 = (c % a.HD) / 2;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const float ev = x[jv][2 * p], od = x[jv][2 * p + 1];
        const float cc = cs[j0 + p], s = sn[j0 + p];
        x[jv][2 * p] = ev * cc - od * s;
        x[jv][2 * p + 1] = ev * s + od * cc;
      }
    }
    store8(a.out_dtype, dst, base + c, x[jv]);
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
  // one workgroup per (token, group of kWavesPerBlock heads), one head per wave
  const int64_t hb = (HQ + 2 * HKV + kWavesPerBlock - 1) / kWavesPerBlock;
  if (T > 0x7FFFFFFFLL || hb > 65535) return IFX_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>(T), static_cast<unsigned>(hb));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (HD / 2 <= 64)
    hipLaunchKernelGGL(qkv_split_kernel<1>, grid, dim3(64 * kWavesPerBlock), 0, st, a);
  else
    hipLaunchKernelGGL(qkv_split_kernel<2>, grid, dim3(64 * kWavesPerBlock), 0, st, a);
  return launch_status();
}

}  // extern "C"

extern "C" int ifx_wan_qkv(const void* raw, int raw_dtype, int64_t ldraw, const float* row, const float* col,
                           const float* bias, const float* q_norm, const float* k_norm, float eps,
                           const float* inv_freq, const float* pos, int64_t ldpos, const int32_t* sections,
                           void* q_out, int64_t sq, void* k_pool, int64_t sk_b, int64_t sk_s, void* v_pool,
                           int64_t sv_b, int64_t sv_s, const int32_t* slots, int out_dtype, int64_t rows,
                           int64_t tokens, int64_t heads, int64_t head_dim, void* stream) {
  if (raw_dtype != IFX_DTYPE_BF16 && raw_dtype != IFX_DTYPE_F32) return IFX_ERR_INVALID;
  if (out_dtype != IFX_DTYPE_BF16 && out_dtype != IFX_DTYPE_F32 && out_dtype != IFX_DTYPE_F16) return IFX_ERR_INVALID;
  if (rows < 0 || tokens <= 0 || heads <= 0 || head_dim <= 0 || head_dim % 8 != 0) return IFX_ERR_INVALID;
  if (head_dim > 256) return IFX_ERR_UNSUPPORTED;
  const int64_t D = heads * head_dim;
  if (D > 256 * 8 * 8) return IFX_ERR_UNSUPPORTED;
  const int parts = 1 + (k_pool != nullptr) + (v_pool != nullptr);
  if (ldraw < parts * D || sq < D) return IFX_ERR_INVALID;
  if (inv_freq && (!pos || ldpos < 1)) return IFX_ERR_INVALID;
  if (!(eps >= 0.0f)) return IFX_ERR_INVALID;
  if (rows == 0) return IFX_OK;
  if (!raw || !q_out) return IFX_ERR_INVALID;
  // 16-byte groups of 8 elements: aligned bases, strides in multiples of 8
  auto al = [](const void* p) { return p == nullptr || aligned16(p); };
  if (!aligned16(raw) || !aligned16(q_out) || !al(k_pool) || !al(v_pool) || !al(col) || !al(bias) || !al(q_norm) ||
      !al(k_norm) || ldraw % 8 || sq % 8 || (k_pool && (sk_b % 8 || sk_s % 8)) || (v_pool && (sv_b % 8 || sv_s % 8)))
    return IFX_ERR_ALIGN;
  // grid.y = parts as in the reference launch (wan.py:97): part 1 is always K
  WanArgs a{raw,    ldraw, row,  col,   bias,   q_norm, k_norm, eps,   inv_freq, pos, ldpos, sections, q_out, sq,
            k_pool, sk_b,  sk_s, v_pool, sv_b,  sv_s,   slots,  tokens, D,       head_dim, k_pool != nullptr,
            v_pool != nullptr, raw_dtype == IFX_DTYPE_F32 ? 1 : 0, out_dtype};
  if (rows > 0x7FFFFFFFLL) return IFX_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>(rows), static_cast<unsigned>(parts));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t groups = (D / 8 + 255) / 256;
  if (groups <= 1) hipLaunchKernelGGL(wan_qkv_kernel<1>, grid, dim3(256), 0, st, a);
  else if (groups <= 2) hipLaunchKernelGGL(wan_qkv_kernel<2>, grid, dim3(256), 0, st, a);
  else if (groups <= 4) hipLaunchKernelGGL(wan_qkv_kernel<4>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(wan_qkv_kernel<8>, grid, dim3(256), 0, st, a);
  return launch_status();
}
