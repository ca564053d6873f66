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

constexpr int kRouterMaxD = 16384;
constexpr int kRouterMaxE = 256;

struct RouterArgs {
  const float* w;   // [E, D]
  const float* eb;  // [E]
  float* out;       // [M, E]
  int E;
  int topk;
  float scale;
};

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
  RouterArgs router;
  int64_t M;
  int64_t ks;  // > 0: q in the skinny tile layout with ks K steps (grid covers 16*ceil(M/16) rows)
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
  v = wave_sum_f32(v);
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

// ---------------------------------------------------------------------------
// MoE router (reference instinctflash/kernels/activation.py:71-100, and the
// router option of norm.py:84-94): per token, logits[e] = w[e] . x, s =
// sigmoid(logits); the top_k experts by s + e_bias (ties: lowest index) keep
// their weight s, renormalized to sum to `scale`; the others get 0.
// One 256-lane workgroup per token with the row in LDS: each wave computes the
// dot products of blocks of 8 experts (lane-strided float4 over D, then a
// fixed-order wave butterfly), then wave 0 selects, holding up to 4 experts per
// lane.
// ---------------------------------------------------------------------------

// Prefetch path (E <= 32, D % 4 == 0, D <= 1024, 16-byte aligned weights):
// wave w's 8 experts 8w..8w+7 are read into registers up front (before the
// row is known, so the loads overlap the row's own work), 4 float4 per lane
// per expert.
constexpr int kPfIt = 4;

struct RouterPf {
  float4 w[kPfIt][8];
};

bool router_prefetch_ok(int64_t E, int64_t D, const float* w) {
  return E <= 32 && D % 4 == 0 && D <= 4 * 64 * kPfIt && (reinterpret_cast<uintptr_t>(w) & 15u) == 0;
}

__device__ __forceinline__ void router_prefetch(const RouterArgs& r, int64_t D, RouterPf& p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t D4 = D / 4;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int e = 8 * wave + u < r.E ? 8 * wave + u : r.E - 1;
    const float4* wr = reinterpret_cast<const float4*>(r.w + e * D);
#pragma unroll
    for (int it = 0; it < kPfIt; ++it) {
      const int64_t d = lane + 64 * it;
      p.w[it][u] = wr[d < D4 ? d : D4 - 1];
    }
  }
}

// logits of the prefetched experts against the row xs (LDS); then a barrier.
__device__ __forceinline__ void router_logits_pf(const float* xs, int64_t D, const RouterArgs& r, const RouterPf& p,
                                                 float* logit) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t D4 = D / 4;
  const float4* x4 = reinterpret_cast<const float4*>(xs);
  float acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = 0.0f;
#pragma unroll
  for (int it = 0; it < kPfIt; ++it) {
    const int64_t d = lane + 64 * it;
    if (d < D4) {
      const float4 xv = x4[d];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        acc[u] = acc[u] + p.w[it][u].x * xv.x + p.w[it][u].y * xv.y + p.w[it][u].z * xv.z + p.w[it][u].w * xv.w;
    }
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    acc[u] = wave_sum_f32(acc[u]);
    if (lane == 0 && 8 * wave + u < r.E) logit[8 * wave + u] = acc[u];
  }
  __syncthreads();
}

// Generic path: logits from the row xs (LDS) and the weights in memory; then a
// barrier.
__device__ void router_logits(const float* xs, int64_t D, const RouterArgs& r, float* logit) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (D % 4 == 0 && (reinterpret_cast<uintptr_t>(r.w) & 15u) == 0) {
    // wave w owns experts w*8.. in blocks of 8 (block b: experts 32b + 8w ..
    // +7): each step loads 8 independent float4 of the weight rows against one
    // float4 of the row, so a step costs one memory latency for 8 experts
    const int64_t D4 = D / 4;
    const float4* x4 = reinterpret_cast<const float4*>(xs);
    for (int e0 = 8 * wave; e0 < r.E; e0 += 32) {
      float acc[8];
      const float4* wr[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        acc[u] = 0.0f;
        const int e = e0 + u < r.E ? e0 + u : r.E - 1;
        wr[u] = reinterpret_cast<const float4*>(r.w + e * D);
      }
#pragma unroll 4
      for (int64_t d = lane; d < D4; d += 64) {
        float4 w4[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) w4[u] = wr[u][d];
        const float4 xv = x4[d];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          acc[u] = acc[u] + w4[u].x * xv.x + w4[u].y * xv.y + w4[u].z * xv.z + w4[u].w * xv.w;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        acc[u] = wave_sum_f32(acc[u]);
        if (lane == 0 && e0 + u < r.E) logit[e0 + u] = acc[u];
      }
    }
  } else {
    for (int e = wave; e < r.E; e += 4) {
      float acc = 0.0f;
      for (int64_t d = lane; d < D; d += 64) acc = acc + r.w[e * D + d] * xs[d];
      acc = wave_sum_f32(acc);
      if (lane == 0) logit[e] = acc;
    }
  }
  __syncthreads();
}

// Selection and weights from logit (LDS [E], all written; overwritten here)
// with wsl (LDS [E]) as scratch: thread e owns expert e (E <= 256, all threads
// of the workgroup take part). Expert e is chosen when fewer than top_k experts
// rank before it, ranking by selection score, then lower index -- the order of
// a repeated argmax. The chosen weights are summed in expert order, the same
// order in every thread.
__device__ void router_select(const RouterArgs& r, int64_t t, float* logit, float* wsl) {
  const int e = threadIdx.x;
  const bool mine = e < r.E;
  float sg = 0.0f, sel = 0.0f;
  if (mine) {
    sg = 1.0f / (1.0f + expf(-logit[e]));
    sel = sg + r.eb[e];
  }
  __syncthreads();  // every logit read
  if (mine) logit[e] = sel;
  __syncthreads();
  int rank = 0;
  if (mine) {
#pragma unroll 8
    for (int j = 0; j < r.E; ++j) {
      const float o = logit[j];
      rank += (o > sel || (o == sel && j < e)) ? 1 : 0;
    }
  }
  const float w = mine && rank < r.topk ? sg : 0.0f;
  if (mine) wsl[e] = w;
  __syncthreads();
  float sum = 0.0f;
#pragma unroll 8
  for (int j = 0; j < r.E; ++j) sum = sum + wsl[j];
  if (mine) r.out[t * r.E + e] = w / (sum + 1e-20f) * r.scale;
}

template <bool PF>
__global__ __launch_bounds__(256) void moe_router_kernel(const void* x, int x_f32, int64_t ldx, int64_t D,
                                                         RouterArgs r) {
  __shared__ float xs[kRouterMaxD];
  __shared__ float logit[kRouterMaxE];
  __shared__ float wsl[kRouterMaxE];
  const int64_t t = blockIdx.x;
  RouterPf pf;
  if constexpr (PF) router_prefetch(r, D, pf);
#pragma unroll 4
  for (int64_t d = threadIdx.x; d < D; d += 256)
    xs[d] = x_f32 ? static_cast<const float*>(x)[t * ldx + d]
                  : __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(x)[t * ldx + d]) << 16);
  __syncthreads();
  if constexpr (PF) router_logits_pf(xs, D, r, pf, logit);
  else router_logits(xs, D, r, logit);
  router_select(r, t, logit, wsl);
}

// KB: groups per load batch (2 for latency-bound launches of few rows, 1 when
// many rows keep the CUs busy and occupancy matters more than per-row latency).
// ROUTER: 0 none, 1 router (generic path), 2 router with prefetched weights.
template <int VPT, bool RES_BF16, bool DELTA_BF16, int ROUTER, int KB>
__global__ __launch_bounds__(kRnqThreads) void residual_norm_quant_kernel(RnqArgs a) {
  __shared__ float red[kRnqThreads / 64];
  // the normalized row for the router (instances without it keep no LDS)
  __shared__ float ys[ROUTER ? kRouterMaxD : 1];
  __shared__ float logit[ROUTER ? kRouterMaxE : 1];
  __shared__ float wsl[ROUTER ? kRouterMaxE : 1];
  const int64_t row = blockIdx.x;
  if (row >= a.M) {  // tile-layout padding row (workgroup-uniform): zeros only
    for (int64_t idx = threadIdx.x; idx < a.ks * 16; idx += kRnqThreads)
      *reinterpret_cast<uint2*>(a.q + tile_offset(row, idx * 8, a.ks)) = make_uint2(0u, 0u);
    return;
  }
  const int64_t D = a.D;
  const int64_t mofs = a.mod_index ? static_cast<int64_t>(a.mod_index[row]) * D : 0;
  const bool has_delta = a.delta != nullptr;
  const bool layernorm = (a.flags & IFX_RNQ_LAYERNORM) != 0;
  RouterPf pf;
  if constexpr (ROUTER == 2) router_prefetch(a.router, D, pf);

  // Loads are grouped so that a row's reads are in flight together: every res
  // group first, then the delta operands in batches of kB groups (one memory
  // latency per batch); out-of-row groups read the row's last group (clamped
  // addresses, no branch) and are masked afterwards.
  constexpr int kB = VPT < KB ? VPT : KB;
  float x[VPT][8];
  bool on[VPT];
  int64_t cs[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t c = (static_cast<int64_t>(j) * kRnqThreads + threadIdx.x) * 8;
    on[j] = c < D;
    cs[j] = on[j] ? c : D - 8;
    if constexpr (RES_BF16) load8_bf16(static_cast<const uint16_t*>(a.res) + row * a.ldres + cs[j], x[j]);
    else load8_f32(static_cast<const float*>(a.res) + row * a.ldres + cs[j], x[j]);
  }
  if (has_delta) {
    const float r = a.drow ? a.drow[row] : 1.0f;
#pragma unroll
    for (int j0 = 0; j0 < VPT; j0 += kB) {
      float d[kB][8], vc[kB][8], vb[kB][8], vg[kB][8];
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        const int64_t c = cs[j0 + j];
        if constexpr (DELTA_BF16) load8_bf16(static_cast<const uint16_t*>(a.delta) + row * a.lddelta + c, d[j]);
        else load8_f32(static_cast<const float*>(a.delta) + row * a.lddelta + c, d[j]);
      }
      if (a.dcol)
#pragma unroll
        for (int j = 0; j < kB; ++j) load8_f32(a.dcol + cs[j0 + j], vc[j]);
      if (a.bias)
#pragma unroll
        for (int j = 0; j < kB; ++j) load8_f32(a.bias + cs[j0 + j], vb[j]);
      if (a.gate)
#pragma unroll
        for (int j = 0; j < kB; ++j) load8_f32(a.gate + mofs + cs[j0 + j], vg[j]);
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        float* xj = x[j0 + j];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          float dt = d[j][t];
          if (a.drow) dt = dt * r;
          if (a.dcol) dt = dt * vc[j][t];
          if (a.bias) dt = dt + vb[j][t];
          if (a.gate) dt = dt * vg[j][t];
          xj[t] = xj[t] + dt;
        }
        if ((a.flags & IFX_RNQ_WRITE_RES) && on[j0 + j]) {
          if constexpr (RES_BF16) {
            void* p = static_cast<uint16_t*>(a.res) + row * a.ldres + cs[j0 + j];
            store8_bf16(p, xj);
            // normalize the stored (rounded) value
            const uint4 h = make_uint4(pack_bf16x2(xj[0], xj[1]), pack_bf16x2(xj[2], xj[3]),
                                       pack_bf16x2(xj[4], xj[5]), pack_bf16x2(xj[6], xj[7]));
            unpack_bf16x8(h, xj);
          } else {
            store8_f32(static_cast<float*>(a.res) + row * a.ldres + cs[j0 + j], xj);
          }
        }  // without the write the FP32 sum is normalized (norm.py:55-57 rounds only what it stores)
      }
    }
  }
#pragma unroll
  for (int j = 0; j < VPT; ++j)
    if (!on[j])
#pragma unroll
      for (int t = 0; t < 8; ++t) x[j][t] = 0.0f;

  // The affine / adaptive vectors: when the whole row is one batch their loads
  // are issued here, so that they are in flight during the reductions.
  float vw[kB][8], vb[kB][8], vs[kB][8], vh[kB][8];
  auto load_post = [&](int j0) {
    if (a.weight)
#pragma unroll
      for (int j = 0; j < kB; ++j) load8_f32(a.weight + cs[j0 + j], vw[j]);
    if (a.beta)
#pragma unroll
      for (int j = 0; j < kB; ++j) load8_f32(a.beta + cs[j0 + j], vb[j]);
    if (a.mscale)
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        load8_f32(a.mscale + mofs + cs[j0 + j], vs[j]);
        load8_f32(a.mshift + mofs + cs[j0 + j], vh[j]);
      }
  };
  if constexpr (VPT == kB) load_post(0);

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

  // affine and adaptive terms, their vector loads batched like the inputs
  uint32_t amax = 0;
#pragma unroll
  for (int j0 = 0; j0 < VPT; j0 += kB) {
    if constexpr (VPT != kB) load_post(j0);
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      if (!on[j0 + j]) continue;
      const int64_t c = cs[j0 + j];
      float* xj = x[j0 + j];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        float v = xj[t] * rstd;
        if (a.weight) v = v * vw[j][t];
        if (a.beta) v = v + vb[j][t];
        if (a.mscale) v = v * (1.0f + vs[j][t]) + vh[j][t];
        xj[t] = v;
      }
      if constexpr (ROUTER) {
#pragma unroll
        for (int t = 0; t < 8; ++t) ys[c + t] = xj[t];
      }
      if (a.y) {
        if (a.y_f32) store8_f32(static_cast<float*>(a.y) + row * a.ldy + c, xj);
        else store8_bf16(static_cast<uint16_t*>(a.y) + row * a.ldy + c, xj);
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t b = abs_bits(xj[t]);
        amax = amax > b ? amax : b;
      }
    }
  }
  if (a.q) {  // uniform per workgroup
    amax = block_max_u32(amax, reinterpret_cast<uint32_t*>(red));
    const float s = scale_from_amax_bits(amax);
    if (threadIdx.x == 0) a.qs[row] = s;
    const bool fast = finite_scale(s);
    const float r = 1.0f / s;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      if (!on[j]) continue;
      const int64_t c = (static_cast<int64_t>(j) * kRnqThreads + threadIdx.x) * 8;
      uint8_t* dst = a.ks > 0 ? a.q + tile_offset(row, c, a.ks) : a.q + row * a.ldq + c;
      *reinterpret_cast<uint2*>(dst) = fast ? pack8_fast(x[j], s, r) : pack8_exact(x[j], s);
    }
    if (a.ks > 0)  // K padding of the tile layout
      for (int64_t idx = D / 8 + threadIdx.x; idx < a.ks * 16; idx += kRnqThreads)
        *reinterpret_cast<uint2*>(a.q + tile_offset(row, idx * 8, a.ks)) = make_uint2(0u, 0u);
  }
  if constexpr (ROUTER != 0) {
    __syncthreads();
    if constexpr (ROUTER == 2) router_logits_pf(ys, D, a.router, pf, logit);
    else router_logits(ys, D, a.router, logit);
    router_select(a.router, row, logit, wsl);
  }
}

template <int VPT>
void launch_rnq(const RnqArgs& a, int64_t M, bool res_bf16, bool delta_bf16, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(a.ks > 0 ? (M + 15) / 16 * 16 : M)), block(kRnqThreads);
  const bool router = a.router.w != nullptr;
  const bool pf = router && VPT == 1 && router_prefetch_ok(a.router.E, a.D, a.router.w);
  const bool many = M >= 1024;
#define IFX_RNQ(RB, DB)                                                                                            \
  if (pf) hipLaunchKernelGGL((residual_norm_quant_kernel<1, RB, DB, 2, 1>), grid, block, 0, st, a);             \
  else if (router) hipLaunchKernelGGL((residual_norm_quant_kernel<VPT, RB, DB, 1, 2>), grid, block, 0, st, a);  \
  else if (many) hipLaunchKernelGGL((residual_norm_quant_kernel<VPT, RB, DB, 0, 1>), grid, block, 0, st, a);    \
  else hipLaunchKernelGGL((residual_norm_quant_kernel<VPT, RB, DB, 0, 2>), grid, block, 0, st, a)
  if (res_bf16) {
    if (delta_bf16) { IFX_RNQ(true, true); }
    else { IFX_RNQ(true, false); }
  } else {
    if (delta_bf16) { IFX_RNQ(false, true); }
    else { IFX_RNQ(false, false); }
  }
#undef IFX_RNQ
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
                            int64_t ldq, float* q_scale, void* y, int y_dtype, int64_t ldy, const float* router_w,
                            const float* router_bias, float* route_w, int64_t router_E, int router_top_k,
                            float router_scale, int64_t M, int64_t D, void* stream) {
  constexpr int kKnown = IFX_RNQ_WRITE_RES | IFX_RNQ_LAYERNORM;
  if (flags & ~kKnown) return IFX_ERR_INVALID;
  auto dtype_ok = [](int d) { return d == IFX_DTYPE_BF16 || d == IFX_DTYPE_F32; };
  if (!dtype_ok(res_dtype) || (delta && !dtype_ok(delta_dtype)) || (y && !dtype_ok(y_dtype))) return IFX_ERR_INVALID;
  if (M < 0 || D <= 0 || D % 8 != 0) return IFX_ERR_INVALID;
  if (D > static_cast<int64_t>(kRnqThreads) * 8 * 8) return IFX_ERR_UNSUPPORTED;
  if (ldres < D || (delta && lddelta < D) || (q && ldq != IFX_LD_TILED && ldq < D) || (y && ldy < D)) return IFX_ERR_INVALID;
  if ((mod_scale == nullptr) != (mod_shift == nullptr)) return IFX_ERR_INVALID;
  if (q && !q_scale) return IFX_ERR_INVALID;
  if (!(eps >= 0.0f)) return IFX_ERR_INVALID;
  if (router_w) {
    if (!router_bias || !route_w || router_E <= 0 || router_top_k < 0 || router_top_k > router_E)
      return IFX_ERR_INVALID;
    if (router_E > kRouterMaxE) return IFX_ERR_UNSUPPORTED;
  }
  if (M == 0) return IFX_OK;
  if (!res) return IFX_ERR_INVALID;
  if (!aligned16(res) || ldres % 8 != 0 || !aligned_vec(delta) || (delta && lddelta % 8 != 0) ||
      !aligned_vec(y) || (y && ldy % 8 != 0) || (q && ((reinterpret_cast<uintptr_t>(q) & 7u) || ldq % 8 != 0)))
    return IFX_ERR_ALIGN;
  for (const float* v : {delta_col, bias, gate, weight, beta, mod_scale, mod_shift})
    if (!aligned_vec(v)) return IFX_ERR_ALIGN;

  RnqArgs a{res, ldres, delta, lddelta, delta_row, delta_col, bias, gate, weight, beta, mod_scale, mod_shift,
            mod_index, y, ldy, static_cast<uint8_t*>(q), ldq, q_scale, D, eps, delta ? flags : (flags & ~IFX_RNQ_WRITE_RES),
            y_dtype == IFX_DTYPE_F32 ? 1 : 0,
            RouterArgs{router_w, router_bias, route_w, static_cast<int>(router_E), router_top_k, router_scale}, M,
            q && ldq == IFX_LD_TILED ? (D + 127) / 128 : 0};
  if (a.ks > 0 && (M > 64 || D % 16 != 0 || !aligned16(q))) return IFX_ERR_UNSUPPORTED;
  const bool rb = res_dtype == IFX_DTYPE_BF16, db = delta_dtype == IFX_DTYPE_BF16;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t groups = (D / 8 + kRnqThreads - 1) / kRnqThreads;  // 8-element groups per lane
  if (groups <= 1) launch_rnq<1>(a, M, rb, db, st);
  else if (groups <= 2) launch_rnq<2>(a, M, rb, db, st);
  else if (groups <= 4) launch_rnq<4>(a, M, rb, db, st);
  else launch_rnq<8>(a, M, rb, db, st);
  return launch_status();
}

int ifx_moe_router(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t D, const float* gate_w,
                   const float* e_bias, float* route_w, int64_t E, int top_k, float scale, void* stream) {
  if (x_dtype != IFX_DTYPE_BF16 && x_dtype != IFX_DTYPE_F32) return IFX_ERR_INVALID;
  if (M < 0 || D <= 0 || E <= 0 || ldx < D || top_k < 0 || top_k > E) return IFX_ERR_INVALID;
  if (D > kRouterMaxD || E > kRouterMaxE) return IFX_ERR_UNSUPPORTED;
  if (M == 0) return IFX_OK;
  if (!x || !gate_w || !e_bias || !route_w) return IFX_ERR_INVALID;
  const RouterArgs r{gate_w, e_bias, route_w, static_cast<int>(E), top_k, scale};
  const int x_f32 = x_dtype == IFX_DTYPE_F32 ? 1 : 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (router_prefetch_ok(E, D, gate_w))
    hipLaunchKernelGGL(moe_router_kernel<true>, dim3(static_cast<unsigned>(M)), dim3(256), 0, st, x, x_f32, ldx, D, r);
  else
    hipLaunchKernelGGL(moe_router_kernel<false>, dim3(static_cast<unsigned>(M)), dim3(256), 0, st, x, x_f32, ldx, D, r);
  return launch_status();
}

}  // extern "C"
