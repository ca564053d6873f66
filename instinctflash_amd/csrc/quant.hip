// Per-row (per-token / per-output-channel) and per-tensor dynamic FP8 E4M3
// quantizers for gfx950, plus the consumer-side producers `row_quant`,
// `gated_act_quant` and `dequant_rows`.
//
// Reference recipe: instinctflash/kernels/fp8.py:30-37 (quantize_weight), with
// the device scale arithmetic of instinctflash/runtime/fp8_pack.py:83-91:
//   scale = max(amax, 1e-12) * fl32(1/448),  q = e4m3_rne(clamp(x / scale, +-448))
// The division is IEEE round-to-nearest (fp8_pack.py:32-34): this file must be
// compiled with correctly rounded FP32 division (-fhip-fp32-correctly-rounded-
// divide-sqrt, hipcc's default).
//
// Design (HBM-bound: 2-4 B read + 1 B written per element):
//  * A "team" of T = 64/128/256 lanes owns one row; the row stays in registers
//    (VPT 16-byte vectors per lane), so it is read from HBM exactly once.
//  * The absmax reduction runs on |x| bit patterns as unsigned integers: for
//    non-NaN floats that order equals the numeric order, and every NaN pattern
//    compares above +inf (0x7F800000), so one integer max both finds amax and
//    propagates NaN exactly as torch's amax does.
//  * 128-bit loads, 64-bit stores of 8 packed E4M3 codes, scale written once.

#include <type_traits>

#include "ifx_abi.h"
#include "ifx_device.h"
#include "ifx_quant.h"

// No multiply-add contraction in this file: the producers' FP32 arithmetic
// (x*row*col + bias) must round after every operation, like the reference's
// element-wise torch/numpy formulation, so the quantized bytes are reproducible.
#pragma clang fp contract(off)

namespace ifx {
namespace {

constexpr int kBlock = 256;

// ---- row sources -----------------------------------------------------------
// Each source produces FP32 values of row m in two forms:
//  * fetch(m, k, raw) issues every load of the 8 elements k..k+7 with no
//    branch (m and k must be in range), finish(raw, m, k, v) turns them into
//    values: the register-resident kernel issues the fetches of all its groups
//    before the first finish, so a row's loads are in flight together instead
//    of one memory latency per group;
//  * load1(m, k): one element, for the two-pass kernel.
// Optional column vectors are template flags so that fetch stays branch-free;
// the per-row scale is read once per row by begin(m).

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// 16-byte nontemporal load of a source row: every row source is read once
// (8192 x 14336 bf16 rows: 63.0 -> 55.5 us per launch against plain loads).
__device__ __forceinline__ uint4 ld_nt(const void* p) {
  const v4u t = __builtin_nontemporal_load(static_cast<const v4u*>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}

struct SrcBf16 {
  const uint16_t* x;
  int64_t ldx;
  struct Raw { uint4 a; };
  __device__ __forceinline__ float begin(int64_t) const { return 1.0f; }
  __device__ __forceinline__ void fetch(int64_t m, int64_t k, Raw& r) const {
    r.a = ld_nt(x + m * ldx + k);
  }
  __device__ __forceinline__ void finish(const Raw& r, float, int64_t, int64_t, float* v) const {
    unpack_bf16x8(r.a, v);
  }
  __device__ __forceinline__ float load1(int64_t m, int64_t k) const {
    return bf16_bits_to_f32(x[m * ldx + k]);
  }
};

struct SrcF32 {
  const float* x;
  int64_t ldx;
  struct Raw { float4 a, b; };
  __device__ __forceinline__ float begin(int64_t) const { return 1.0f; }
  __device__ __forceinline__ void fetch(int64_t m, int64_t k, Raw& r) const {
    r.a = *reinterpret_cast<const float4*>(x + m * ldx + k);
    r.b = *reinterpret_cast<const float4*>(x + m * ldx + k + 4);
  }
  __device__ __forceinline__ void finish(const Raw& r, float, int64_t, int64_t, float* v) const {
    v[0] = r.a.x; v[1] = r.a.y; v[2] = r.a.z; v[3] = r.a.w;
    v[4] = r.b.x; v[5] = r.b.y; v[6] = r.b.z; v[7] = r.b.w;
  }
  __device__ __forceinline__ float load1(int64_t m, int64_t k) const { return x[m * ldx + k]; }
};

struct Vec8 {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = reinterpret_cast<const float4*>(p)[0];
    b = reinterpret_cast<const float4*>(p)[1];
  }
  __device__ __forceinline__ float operator[](int i) const {
    const float t[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    return t[i];
  }
};

// v = x*row[m]*col[k] + bias[k] (-> gelu_tanh); reference kernels/norm.py:135-144.
// HC / HB: col / bias present (vector fetch only; load1 tests the pointers).
template <bool HC = true, bool HB = true>
struct SrcAffine {
  const uint16_t* x;
  int64_t ldx;
  const float* row;
  const float* col;
  const float* bias;
  int gelu;
  int f16;  // x holds fp16 (else bf16)
  int f32;  // x holds float32 (element path only)
  struct Raw { uint4 a; Vec8 c, b; };
  __device__ __forceinline__ void unpack(const uint4& r, float* v) const {
    if (!f16) {
      unpack_bf16x8(r, v);
      return;
    }
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[i] & 0xFFFFu)));
      v[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[i] >> 16)));
    }
  }
  __device__ __forceinline__ float elem(int64_t m, int64_t k) const {
    if (f32) return reinterpret_cast<const float*>(x)[m * ldx + k];
    const uint16_t h = x[m * ldx + k];
    return f16 ? static_cast<float>(__builtin_bit_cast(_Float16, h)) : bf16_bits_to_f32(h);
  }
  __device__ __forceinline__ float op(float v, float r, float c, float b) const {
    if (row) v = v * r;
    if (col) v = v * c;
    if (bias) v = v + b;
    if (gelu) v = gelu_tanh(v);
    return v;
  }
  __device__ __forceinline__ float begin(int64_t m) const { return row ? row[m] : 1.0f; }
  __device__ __forceinline__ void fetch(int64_t m, int64_t k, Raw& r) const {
    r.a = ld_nt(x + m * ldx + k);
    if constexpr (HC) r.c.load(col + k);
    if constexpr (HB) r.b.load(bias + k);
  }
  __device__ __forceinline__ void finish(const Raw& r, float rs, int64_t, int64_t, float* v) const {
    unpack(r.a, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = op(v[i], rs, HC ? r.c[i] : 1.0f, HB ? r.b[i] : 0.0f);
  }
  __device__ __forceinline__ float load1(int64_t m, int64_t k) const {
    return op(elem(m, k), row ? row[m] : 1.0f, col ? col[k] : 1.0f, bias ? bias[k] : 0.0f);
  }
};

// h = act(g)*u from a gate|up accumulator; reference kernels/activation.py:26-40.
template <bool HC = true>
struct SrcGated {
  const uint16_t* gu;
  int64_t ldgu;
  int64_t F;
  const float* row;
  const float* col;
  int act;
  struct Raw { uint4 g, u; Vec8 cg, cu; };
  __device__ __forceinline__ float op(float g, float u, float r, float cg, float cu) const {
    if (row) {
      g = g * r;
      u = u * r;
    }
    if (col) {
      g = g * cg;
      u = u * cu;
    }
    const float a = act == IFX_ACT_SILU ? silu(g) : gelu_tanh(g);
    return a * u;
  }
  __device__ __forceinline__ float begin(int64_t m) const { return row ? row[m] : 1.0f; }
  __device__ __forceinline__ void fetch(int64_t m, int64_t k, Raw& r) const {
    r.g = ld_nt(gu + m * ldgu + k);
    r.u = ld_nt(gu + m * ldgu + F + k);
    if constexpr (HC) {
      r.cg.load(col + k);
      r.cu.load(col + F + k);
    }
  }
  __device__ __forceinline__ void finish(const Raw& r, float rs, int64_t, int64_t, float* v) const {
    float g[8], u[8];
    unpack_bf16x8(r.g, g);
    unpack_bf16x8(r.u, u);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = op(g[i], u[i], rs, HC ? r.cg[i] : 1.0f, HC ? r.cu[i] : 1.0f);
  }
  __device__ __forceinline__ float load1(int64_t m, int64_t k) const {
    return op(bf16_bits_to_f32(gu[m * ldgu + k]), bf16_bits_to_f32(gu[m * ldgu + F + k]), row ? row[m] : 1.0f,
              col ? col[k] : 1.0f, col ? col[F + k] : 1.0f);
  }
};

// h = silu(g)*u*wr with the routing weight wr = route_w[m, min(k/group, E-1)] for
// routed columns k < n_routed and 1 for the shared expert's columns; reference
// kernels/activation.py:103-128. The vector fetch needs group % 8 == 0 and
// n_routed % 8 == 0 (one weight per 8-column group) and route_w != NULL.
template <bool HC = true>
struct SrcMoe {
  SrcGated<HC> base;  // act is always SiLU
  const float* rw;
  int64_t E;
  int64_t group;
  int64_t n_routed;
  struct Raw { typename SrcGated<HC>::Raw b; float w; };
  __device__ __forceinline__ int64_t expert(int64_t k) const {
    const int64_t e = k / group;
    return e < E - 1 ? e : E - 1;
  }
  __device__ __forceinline__ float begin(int64_t m) const { return base.begin(m); }
  __device__ __forceinline__ void fetch(int64_t m, int64_t k, Raw& r) const {
    base.fetch(m, k, r.b);
    r.w = rw[m * E + expert(k)];
  }
  __device__ __forceinline__ void finish(const Raw& r, float rs, int64_t m, int64_t k, float* v) const {
    base.finish(r.b, rs, m, k, v);
    const float w = k < n_routed ? r.w : 1.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] * w;
  }
  __device__ __forceinline__ float load1(int64_t m, int64_t k) const {
    return base.load1(m, k) * (k < n_routed ? rw[m * E + expert(k)] : 1.0f);
  }
};

// Team-wide max: lanes [team*T, team*T+T) of the block.
template <int T>
__device__ __forceinline__ uint32_t team_max(uint32_t v, uint32_t* red) {
  v = wave_max_u32(v);
  if constexpr (T > 64) {
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    const int first = (threadIdx.x / T) * (T / 64);
    v = red[first];
#pragma unroll
    for (int i = 1; i < T / 64; ++i) v = v > red[first + i] ? v : red[first + i];
  }
  return v;
}

// Register-resident row quantizer: K % 8 == 0, 16-byte aligned rows,
// ceil(K/8) <= T*VPT.
// ks == 0: q is row-major with stride ldq. ks > 0: q is the skinny tile layout
// (rows M..16*ceil(M/16)-1 and K bytes K..128*ks-1 are written as zeros, by the
// launch covering m_rows = 16*ceil(M/16) rows).
// BLK lanes per workgroup: R = BLK / T rows per workgroup.
template <int T, int VPT, class Src, int BLK = kBlock>
__global__ __launch_bounds__(BLK) void quant_rows_vec(Src src, int64_t M, int64_t K, uint8_t* q,
                                                     int64_t ldq, float* scale, int64_t ks, int64_t m_rows) {
  __shared__ uint32_t red[BLK / 64];
  constexpr int R = BLK / T;
  const int lt = threadIdx.x % T;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * R + threadIdx.x / T;
  const bool row_ok = m < M;
  const int64_t nvec = K >> 3;
  // the loads of up to 8 groups first (clamped into range, so no branch), then
  // their math: one memory latency per batch of 8 groups
  constexpr int kMaxBatch = BLK >= 1024 ? 2 : 8;  // 128 VGPRs per lane at 1024 lanes
  constexpr int kBatch = VPT < kMaxBatch ? VPT : kMaxBatch;
  const int64_t mc = row_ok ? m : M - 1;
  const float rs = src.begin(mc);
  float v[VPT][8];
  uint32_t amax = 0;
#pragma unroll
  for (int j0 = 0; j0 < VPT; j0 += kBatch) {
    typename Src::Raw raw[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int64_t idx = lt + static_cast<int64_t>(j0 + j) * T;
      src.fetch(mc, (idx < nvec ? idx : nvec - 1) * 8, raw[j]);
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int64_t idx = lt + static_cast<int64_t>(j0 + j) * T;
      src.finish(raw[j], rs, mc, (idx < nvec ? idx : nvec - 1) * 8, v[j0 + j]);
      const bool on = row_ok && idx < nvec;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t b = on ? abs_bits(v[j0 + j][i]) : 0u;
        amax = amax > b ? amax : b;
      }
    }
  }
  amax = team_max<T>(amax, red);
  if (ks > 0 && m < m_rows) {  // zero padding of the tile layout
    for (int64_t idx = row_ok ? nvec + lt : lt; idx < ks * 16; idx += T)
      *reinterpret_cast<uint2*>(q + tile_offset(m, idx * 8, ks)) = make_uint2(0u, 0u);
  }
  if (!row_ok) return;
  const float s = scale_from_amax_bits(amax);
  if (lt == 0) scale[m] = s;
  auto dst = [&](int64_t idx) -> uint2* {
    return reinterpret_cast<uint2*>(q + (ks > 0 ? tile_offset(m, idx * 8, ks) : m * ldq + idx * 8));
  };
  if (finite_scale(s)) {  // row-uniform branch
    const float r = 1.0f / s;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int64_t idx = lt + static_cast<int64_t>(j) * T;
      if (idx < nvec) *dst(idx) = pack8_fast(v[j], s, r);
    }
  } else {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int64_t idx = lt + static_cast<int64_t>(j) * T;
      if (idx < nvec) *dst(idx) = pack8_exact(v[j], s);
    }
  }
}

// Any K / alignment: one 256-lane block per row, two passes over the row.
template <class Src>
__global__ __launch_bounds__(kBlock) void quant_rows_generic(Src src, int64_t M, int64_t K,
                                                            uint8_t* q, int64_t ldq, float* scale) {
  __shared__ uint32_t red[kBlock / 64];
  const int64_t m = blockIdx.x;
  uint32_t amax = 0;
  for (int64_t k = threadIdx.x; k < K; k += kBlock) {
    const uint32_t b = abs_bits(src.load1(m, k));
    amax = amax > b ? amax : b;
  }
  amax = team_max<kBlock>(amax, red);
  const float s = scale_from_amax_bits(amax);
  if (threadIdx.x == 0) scale[m] = s;
  for (int64_t k = threadIdx.x; k < K; k += kBlock)
    q[m * ldq + k] = static_cast<uint8_t>(q1(src.load1(m, k), s));
}

template <int T, int VPT, class Src, int BLK = kBlock>
void launch_vec(const Src& src, int64_t M, int64_t K, uint8_t* q, int64_t ldq, float* scale,
                hipStream_t st, int64_t ks = 0) {
  constexpr int R = BLK / T;
  const int64_t m_rows = ks > 0 ? (M + 15) / 16 * 16 : M;
  const int64_t grid = (m_rows + R - 1) / R;
  hipLaunchKernelGGL((quant_rows_vec<T, VPT, Src, BLK>), dim3(static_cast<unsigned>(grid)), dim3(BLK),
                     0, st, src, M, K, q, ldq, scale, ks, m_rows);
}

// Picks the register-resident variant (team size, vectors per lane) or falls
// back to the two-pass kernel.
// ldq == IFX_LD_TILED: q is the skinny tile layout of ifx_quant_rows_tiled
// (M <= 64, K % 16 == 0, 16-byte aligned rows).
template <class Src>
int dispatch_rows(const Src& src, bool vec_ok, int64_t M, int64_t K, uint8_t* q, int64_t ldq,
                  float* scale, hipStream_t st) {
  if (M == 0 || K == 0) {
    if (M > 0 && K == 0) return IFX_ERR_INVALID;  // amax of an empty row is undefined
    return IFX_OK;
  }
  if (M > 0x7FFFFFFFLL) return IFX_ERR_INVALID;
  const int64_t nvec = K / 8;
  if (ldq == IFX_LD_TILED) {
    if (!vec_ok || K % 16 != 0 || M > 64 || nvec > 2048 || !aligned16(q)) return IFX_ERR_UNSUPPORTED;
    const int64_t ks = (K + 127) / 128;
    if (nvec <= 256) launch_vec<256, 1>(src, M, K, q, 0, scale, st, ks);
    else if (nvec <= 512) launch_vec<512, 1, Src, 512>(src, M, K, q, 0, scale, st, ks);
    else if (nvec <= 1024) launch_vec<1024, 1, Src, 1024>(src, M, K, q, 0, scale, st, ks);
    else launch_vec<1024, 2, Src, 1024>(src, M, K, q, 0, scale, st, ks);
    return launch_status();
  }
  if (vec_ok && K % 8 == 0 && nvec <= 4096 && M < 256) {
    // Few rows: latency-bound, so give every row a whole 256-lane block
    // instead of packing rows per block; wide rows get up to 1024 lanes, so
    // that each SIMD interleaves several waves of the row's arithmetic.
    if (nvec <= 256) launch_vec<256, 1>(src, M, K, q, ldq, scale, st);
    else if (nvec <= 512) launch_vec<512, 1, Src, 512>(src, M, K, q, ldq, scale, st);
    else if (nvec <= 1024) launch_vec<1024, 1, Src, 1024>(src, M, K, q, ldq, scale, st);
    else if (nvec <= 2048) launch_vec<1024, 2, Src, 1024>(src, M, K, q, ldq, scale, st);
    else launch_vec<1024, 4, Src, 1024>(src, M, K, q, ldq, scale, st);
  } else if (vec_ok && K % 8 == 0 && nvec <= 2048) {
    if (nvec <= 64) launch_vec<64, 1>(src, M, K, q, ldq, scale, st);
    else if (nvec <= 128) launch_vec<64, 2>(src, M, K, q, ldq, scale, st);
    else if (nvec <= 256) launch_vec<64, 4>(src, M, K, q, ldq, scale, st);
    // 6 groups per lane for K <= 3072 (none clamped at K = 3072:
    // 8192 x 3072 14.6 -> 14.0 us against 8 groups)
    else if (nvec <= 384) launch_vec<64, 6>(src, M, K, q, ldq, scale, st);
    else if (nvec <= 512) launch_vec<64, 8>(src, M, K, q, ldq, scale, st);
    else if (nvec <= 1024) launch_vec<128, 8>(src, M, K, q, ldq, scale, st);
    else launch_vec<256, 8>(src, M, K, q, ldq, scale, st);
  } else if (vec_ok && K % 8 == 0 && nvec <= 4096) {
    launch_vec<256, 16>(src, M, K, q, ldq, scale, st);
  } else {
    hipLaunchKernelGGL((quant_rows_generic<Src>), dim3(static_cast<unsigned>(M)), dim3(kBlock), 0, st,
                       src, M, K, q, ldq, scale);
  }
  return launch_status();
}

// ---- per-tensor quantizer (two launches, no host sync) --------------------

constexpr int64_t kTensorChunk = 8192;  // elements per partial (one block)

__global__ __launch_bounds__(kBlock) void tensor_amax_partial(const uint16_t* x, int64_t count,
                                                             uint32_t* partial) {
  __shared__ uint32_t red[kBlock / 64];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTensorChunk;
  uint32_t amax = 0;
  for (int64_t i = base + threadIdx.x; i < base + kTensorChunk && i < count; i += kBlock) {
    const uint32_t b = x[i] & 0x7FFFu;
    amax = amax > b ? amax : b;
  }
  amax = team_max<kBlock>(amax, red);
  if (threadIdx.x == 0) partial[blockIdx.x] = amax;
}

// Dynamic mode (partial != null): every block reduces the partials itself, so
// no third launch is needed; block 0 writes the scale. Fixed mode: *scale is
// read, not written (reference fp8_pack.py:48-60 pack_bf16_e4m3).
__global__ __launch_bounds__(kBlock) void tensor_pack(const uint16_t* x, int64_t count,
                                                     const uint32_t* partial, int64_t nparts,
                                                     uint8_t* q, float* scale) {
  __shared__ uint32_t red[kBlock / 64];
  float s;
  if (partial) {
    uint32_t amax = 0;
    for (int64_t i = threadIdx.x; i < nparts; i += kBlock) amax = amax > partial[i] ? amax : partial[i];
    amax = team_max<kBlock>(amax, red);
    // bf16 |x| bits -> f32 bits; NaN stays above +inf.
    s = scale_from_amax_bits(amax << 16);
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale = s;
  } else {
    s = *scale;
  }
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTensorChunk;
  for (int64_t i = base + threadIdx.x; i < base + kTensorChunk && i < count; i += kBlock)
    q[i] = static_cast<uint8_t>(q1(bf16_bits_to_f32(x[i]), s));
}

// Vector forms (count % 8 == 0, 16-byte aligned x, 8-byte aligned q): each lane
// handles 16-byte groups of 8 elements, kTensorChunk / 8 groups per block.
__global__ __launch_bounds__(kBlock) void tensor_amax_partial_vec(const uint16_t* x, int64_t count,
                                                                 uint32_t* partial) {
  __shared__ uint32_t red[kBlock / 64];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTensorChunk;
  uint32_t amax = 0;
#pragma unroll
  for (int j = 0; j < kTensorChunk / 8 / kBlock; ++j) {
    const int64_t i = base + (static_cast<int64_t>(j) * kBlock + threadIdx.x) * 8;
    if (i < count) {
      const uint4 r = *reinterpret_cast<const uint4*>(x + i);
      const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t lo = w[t] & 0x7FFFu, hi = (w[t] >> 16) & 0x7FFFu;
        amax = amax > lo ? amax : lo;
        amax = amax > hi ? amax : hi;
      }
    }
  }
  amax = team_max<kBlock>(amax, red);
  if (threadIdx.x == 0) partial[blockIdx.x] = amax;
}

__global__ __launch_bounds__(kBlock) void tensor_pack_vec(const uint16_t* x, int64_t count,
                                                         const uint32_t* partial, int64_t nparts, uint8_t* q,
                                                         float* scale) {
  __shared__ uint32_t red[kBlock / 64];
  float s;
  if (partial) {
    uint32_t amax = 0;
    for (int64_t i = threadIdx.x; i < nparts; i += kBlock) amax = amax > partial[i] ? amax : partial[i];
    amax = team_max<kBlock>(amax, red);
    s = scale_from_amax_bits(amax << 16);
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale = s;
  } else {
    s = *scale;
  }
  // The reciprocal form needs |x| / s <= 448 (true when s comes from this tensor's
  // amax); a caller-fixed scale can overflow x * (1/s), so it keeps the division.
  const bool fast = partial != nullptr && finite_scale(s);
  const float r = 1.0f / s;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTensorChunk;
#pragma unroll
  for (int j = 0; j < kTensorChunk / 8 / kBlock; ++j) {
    const int64_t i = base + (static_cast<int64_t>(j) * kBlock + threadIdx.x) * 8;
    if (i < count) {
      float v[8];
      unpack_bf16x8(*reinterpret_cast<const uint4*>(x + i), v);
      *reinterpret_cast<uint2*>(q + i) = fast ? pack8_fast(v, s, r) : pack8_exact(v, s);
    }
  }
}

// ---- dequant_rows / GLU weight repack --------------------------------------

__device__ __forceinline__ float load_any(const void* base, int dtype, int64_t i) {
  if (dtype == IFX_DTYPE_F32) return static_cast<const float*>(base)[i];
  if (dtype == IFX_DTYPE_F16) return static_cast<float>(static_cast<const _Float16*>(base)[i]);
  return bf16_bits_to_f32(static_cast<const uint16_t*>(base)[i]);
}

__global__ __launch_bounds__(kBlock) void dequant_rows_kernel(const void* x, int x_dtype, int64_t ldx,
                                                             int64_t M, int64_t D, const float* row,
                                                             const float* col, const float* bias,
                                                             void* y, int y_dtype, int64_t ldy) {
  const int64_t m = blockIdx.y;
  const int64_t d = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (d >= D) return;
  float v = load_any(x, x_dtype, m * ldx + d);
  if (row) v = v * row[m];
  if (col) v = v * col[d];
  if (bias) v = v + bias[d];
  const int64_t o = m * ldy + d;
  if (y_dtype == IFX_DTYPE_F32) static_cast<float*>(y)[o] = v;
  else if (y_dtype == IFX_DTYPE_F16) static_cast<_Float16*>(y)[o] = static_cast<_Float16>(v);
  else static_cast<uint16_t*>(y)[o] = static_cast<uint16_t>(f32_to_bf16_bits(v));
}

// One block per packed row p: source row = gate or up row per the 16-row interleave.
__global__ __launch_bounds__(kBlock) void pack_glu_kernel(const uint8_t* w, const float* scale,
                                                         const float* bias, int64_t F, int64_t K,
                                                         uint8_t* wo, float* so, float* bo) {
  const int64_t p = blockIdx.x;
  const int64_t j = (p >> 5) * 16 + (p & 15);
  const int64_t src = (p & 16) ? F + j : j;
  const uint8_t* s = w + src * K;
  uint8_t* d = wo + p * K;
  for (int64_t k = threadIdx.x; k < K; k += kBlock) d[k] = s[k];
  if (threadIdx.x == 0) {
    so[p] = scale[src];
    if (bias && bo) bo[p] = bias[src];
  }
}

}  // namespace
}  // namespace ifx

using namespace ifx;

extern "C" {

int ifx_abi_version(void) { return IFX_ABI_VERSION; }

const char* ifx_status_string(int status) {
  switch (status) {
    case IFX_OK: return "ok";
    case IFX_ERR_INVALID: return "invalid size, stride or flag";
    case IFX_ERR_ALIGN: return "pointer or stride breaks 16-byte alignment";
    case IFX_ERR_WORKSPACE: return "workspace missing or too small";
    case IFX_ERR_UNSUPPORTED: return "shape not supported by any kernel variant";
    case IFX_ERR_SCRATCH: return "call needs more than the library's fixed scratch buffer";
    default: return status > 0 ? hipGetErrorString(static_cast<hipError_t>(status)) : "unknown";
  }
}

size_t ifx_quant_rows_tiled_bytes(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0 || M > 64 || K % 16 != 0) return 0;
  return static_cast<size_t>((M + 15) / 16) * ((K + 127) / 128) * 2048;
}

int ifx_quant_rows_tiled(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, void* q, float* scale,
                         void* stream) {
  if (x_dtype != IFX_DTYPE_BF16 && x_dtype != IFX_DTYPE_F32) return IFX_ERR_INVALID;
  if (M < 0 || M > 64 || K <= 0 || K % 16 != 0 || ldx < K) return IFX_ERR_INVALID;
  if (M == 0) return IFX_OK;
  if (!x || !q || !scale) return IFX_ERR_INVALID;
  const bool f32 = x_dtype == IFX_DTYPE_F32;
  if (!aligned16(x) || !aligned16(q) || ldx % (f32 ? 4 : 8) != 0) return IFX_ERR_ALIGN;
  const int64_t nvec = K / 8, ks = (K + 127) / 128;
  if (nvec > 2048) return IFX_ERR_UNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t* qb = static_cast<uint8_t*>(q);
  auto go = [&](const auto& src) {
    using S = std::decay_t<decltype(src)>;
    if (nvec <= 256) launch_vec<256, 1, S>(src, M, K, qb, 0, scale, st, ks);
    else if (nvec <= 512) launch_vec<512, 1, S, 512>(src, M, K, qb, 0, scale, st, ks);
    else if (nvec <= 1024) launch_vec<1024, 1, S, 1024>(src, M, K, qb, 0, scale, st, ks);
    else launch_vec<1024, 2, S, 1024>(src, M, K, qb, 0, scale, st, ks);
  };
  if (f32) go(SrcF32{static_cast<const float*>(x), ldx});
  else go(SrcBf16{static_cast<const uint16_t*>(x), ldx});
  return launch_status();
}

int ifx_quant_rows(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, void* q,
                   int64_t ldq, float* scale, void* stream) {
  if (M < 0 || K < 0 || ldx < K || ldq < K) return IFX_ERR_INVALID;
  if (M > 0 && (!x || !q || !scale)) return IFX_ERR_INVALID;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool vec_ok = aligned16(x) && (reinterpret_cast<uintptr_t>(q) & 7u) == 0 && ldq % 8 == 0;
  if (x_dtype == IFX_DTYPE_BF16) {
    SrcBf16 s{static_cast<const uint16_t*>(x), ldx};
    return dispatch_rows(s, vec_ok && ldx % 8 == 0, M, K, static_cast<uint8_t*>(q), ldq, scale, st);
  }
  if (x_dtype == IFX_DTYPE_F32) {
    SrcF32 s{static_cast<const float*>(x), ldx};
    return dispatch_rows(s, vec_ok && ldx % 4 == 0, M, K, static_cast<uint8_t*>(q), ldq, scale, st);
  }
  return IFX_ERR_INVALID;
}

size_t ifx_quant_tensor_workspace_size(int64_t count) {
  if (count <= 0) return 0;
  return static_cast<size_t>((count + kTensorChunk - 1) / kTensorChunk) * sizeof(uint32_t);
}

int ifx_quant_tensor_bf16(const void* x, int64_t count, void* q, float* scale, void* partial,
                          size_t partial_bytes, void* stream) {
  if (count <= 0 || !x || !q || !scale) return IFX_ERR_INVALID;
  const int64_t nparts = (count + kTensorChunk - 1) / kTensorChunk;
  if (nparts > 0x7FFFFFFFLL) return IFX_ERR_INVALID;
  if (!partial || partial_bytes < ifx_quant_tensor_workspace_size(count)) return IFX_ERR_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* xs = static_cast<const uint16_t*>(x);
  if (count % 8 == 0 && aligned16(x) && (reinterpret_cast<uintptr_t>(q) & 7u) == 0) {
    hipLaunchKernelGGL(tensor_amax_partial_vec, dim3(static_cast<unsigned>(nparts)), dim3(kBlock), 0, st, xs, count,
                       static_cast<uint32_t*>(partial));
    hipLaunchKernelGGL(tensor_pack_vec, dim3(static_cast<unsigned>(nparts)), dim3(kBlock), 0, st, xs, count,
                       static_cast<const uint32_t*>(partial), nparts, static_cast<uint8_t*>(q), scale);
  } else {
    hipLaunchKernelGGL(tensor_amax_partial, dim3(static_cast<unsigned>(nparts)), dim3(kBlock), 0, st, xs, count,
                       static_cast<uint32_t*>(partial));
    hipLaunchKernelGGL(tensor_pack, dim3(static_cast<unsigned>(nparts)), dim3(kBlock), 0, st, xs, count,
                       static_cast<const uint32_t*>(partial), nparts, static_cast<uint8_t*>(q), scale);
  }
  return launch_status();
}

int ifx_pack_tensor_bf16(const void* x, int64_t count, const float* scale, void* q, void* stream) {
  if (count < 0 || (count > 0 && (!x || !q || !scale))) return IFX_ERR_INVALID;
  if (count == 0) return IFX_OK;
  const int64_t nparts = (count + kTensorChunk - 1) / kTensorChunk;
  if (nparts > 0x7FFFFFFFLL) return IFX_ERR_INVALID;
  const uint16_t* xs = static_cast<const uint16_t*>(x);
  if (count % 8 == 0 && aligned16(x) && (reinterpret_cast<uintptr_t>(q) & 7u) == 0)
    hipLaunchKernelGGL(tensor_pack_vec, dim3(static_cast<unsigned>(nparts)), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), xs, count, static_cast<const uint32_t*>(nullptr), nparts,
                       static_cast<uint8_t*>(q), const_cast<float*>(scale));
  else
    hipLaunchKernelGGL(tensor_pack, dim3(static_cast<unsigned>(nparts)), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), xs, count, static_cast<const uint32_t*>(nullptr), nparts,
                       static_cast<uint8_t*>(q), const_cast<float*>(scale));
  return launch_status();
}

int ifx_row_quant(const void* x, int64_t ldx, int64_t M, int64_t K, const float* row,
                  const float* col, const float* bias, int flags, void* q, int64_t ldq,
                  float* scale, void* stream) {
  if (M < 0 || K < 0 || ldx < K || (ldq != IFX_LD_TILED && ldq < K)) return IFX_ERR_INVALID;
  if (flags & ~(IFX_RQ_GELU | IFX_RQ_F16 | IFX_RQ_F32) || (flags & IFX_RQ_F16 && flags & IFX_RQ_F32))
    return IFX_ERR_INVALID;
  if (M > 0 && (!x || !q || !scale)) return IFX_ERR_INVALID;
  const bool f32 = (flags & IFX_RQ_F32) != 0;
  const bool vec_ok = !f32 && aligned16(x) && ldx % 8 == 0 && (reinterpret_cast<uintptr_t>(q) & 7u) == 0 &&
                      ldq % 8 == 0 && aligned16(col) && aligned16(bias);
  auto go = [&](auto s) {
    s.x = static_cast<const uint16_t*>(x);
    s.ldx = ldx;
    s.row = row;
    s.col = col;
    s.bias = bias;
    s.gelu = (flags & IFX_RQ_GELU) ? 1 : 0;
    s.f16 = (flags & IFX_RQ_F16) ? 1 : 0;
    s.f32 = f32 ? 1 : 0;
    return dispatch_rows(s, vec_ok, M, K, static_cast<uint8_t*>(q), ldq, scale, static_cast<hipStream_t>(stream));
  };
  if (col) return bias ? go(SrcAffine<true, true>{}) : go(SrcAffine<true, false>{});
  return bias ? go(SrcAffine<false, true>{}) : go(SrcAffine<false, false>{});
}

int ifx_gated_act_quant(const void* gu, int64_t ldgu, int64_t M, int64_t F, const float* row,
                        const float* col, int act, void* q, int64_t ldq, float* scale, void* stream) {
  if (M < 0 || F < 0 || ldgu < 2 * F || (ldq != IFX_LD_TILED && ldq < F)) return IFX_ERR_INVALID;
  if (act != IFX_ACT_GELU_TANH && act != IFX_ACT_SILU) return IFX_ERR_INVALID;
  if (M > 0 && (!gu || !q || !scale)) return IFX_ERR_INVALID;
  const bool vec_ok = aligned16(gu) && ldgu % 8 == 0 && F % 8 == 0 &&
                      (reinterpret_cast<uintptr_t>(q) & 7u) == 0 && ldq % 8 == 0 && aligned16(col);
  const uint16_t* g = static_cast<const uint16_t*>(gu);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (col) return dispatch_rows(SrcGated<true>{g, ldgu, F, row, col, act}, vec_ok, M, F, static_cast<uint8_t*>(q),
                                ldq, scale, st);
  return dispatch_rows(SrcGated<false>{g, ldgu, F, row, col, act}, vec_ok, M, F, static_cast<uint8_t*>(q), ldq,
                       scale, st);
}

int ifx_moe_act_quant(const void* gu, int64_t ldgu, int64_t M, int64_t F, const float* row, const float* col,
                      const float* route_w, int64_t E, int64_t group, int64_t n_routed, void* q, int64_t ldq,
                      float* scale, void* stream) {
  if (M < 0 || F < 0 || ldgu < 2 * F || (ldq != IFX_LD_TILED && ldq < F) || E <= 0 || group <= 0 || n_routed < 0)
    return IFX_ERR_INVALID;
  if (M > 0 && (!gu || !q || !scale || (n_routed > 0 && !route_w))) return IFX_ERR_INVALID;
  if (n_routed == 0)  // no routed columns: the plain SwiGLU
    return ifx_gated_act_quant(gu, ldgu, M, F, row, col, IFX_ACT_SILU, q, ldq, scale, stream);
  const bool vec_ok = aligned16(gu) && ldgu % 8 == 0 && F % 8 == 0 &&
                      (reinterpret_cast<uintptr_t>(q) & 7u) == 0 && ldq % 8 == 0 && aligned16(col) &&
                      group % 8 == 0 && n_routed % 8 == 0;
  const uint16_t* g = static_cast<const uint16_t*>(gu);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (col)
    return dispatch_rows(SrcMoe<true>{{g, ldgu, F, row, col, IFX_ACT_SILU}, route_w, E, group, n_routed}, vec_ok, M,
                         F, static_cast<uint8_t*>(q), ldq, scale, st);
  return dispatch_rows(SrcMoe<false>{{g, ldgu, F, row, col, IFX_ACT_SILU}, route_w, E, group, n_routed}, vec_ok, M,
                       F, static_cast<uint8_t*>(q), ldq, scale, st);
}

int ifx_dequant_rows(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t D, const float* row,
                     const float* col, const float* bias, void* y, int y_dtype, int64_t ldy,
                     void* stream) {
  if (M < 0 || D < 0 || ldx < D || ldy < D || M > 65535) return IFX_ERR_INVALID;
  for (int dt : {x_dtype, y_dtype})
    if (dt != IFX_DTYPE_BF16 && dt != IFX_DTYPE_F32 && dt != IFX_DTYPE_F16) return IFX_ERR_INVALID;
  if (M == 0 || D == 0) return IFX_OK;
  if (!x || !y) return IFX_ERR_INVALID;
  const dim3 grid(static_cast<unsigned>((D + kBlock - 1) / kBlock), static_cast<unsigned>(M));
  hipLaunchKernelGGL(dequant_rows_kernel, grid, dim3(kBlock), 0, static_cast<hipStream_t>(stream), x, x_dtype, ldx,
                     M, D, row, col, bias, y, y_dtype, ldy);
  return launch_status();
}

int ifx_fp8_pack_glu(const void* w, const float* scale, const float* bias, int64_t F, int64_t K,
                     void* w_out, float* scale_out, float* bias_out, void* stream) {
  if (F <= 0 || K <= 0 || F % 16 != 0 || !w || !scale || !w_out || !scale_out) return IFX_ERR_INVALID;
  if (2 * F > 0x7FFFFFFFLL) return IFX_ERR_INVALID;
  hipLaunchKernelGGL(pack_glu_kernel, dim3(static_cast<unsigned>(2 * F)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(w), scale, bias, F,
                     K, static_cast<uint8_t*>(w_out), scale_out, bias_out);
  return launch_status();
}

}  // extern "C"
