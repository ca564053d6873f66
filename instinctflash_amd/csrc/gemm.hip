// FP8 (OCP E4M3FN) x FP8 GEMM with fp32 accumulation and a fused epilogue, for
// gfx950 (MI355X) matrix cores.
//
//   acc[m,n] = sum_k a[m,k] * w[n,k]         (a: activations [M,K], w: weights [N,K])
//   out[m,n] = epilogue(acc[m,n] * sa[m] * sw[n])
//
// Reference: instinctflash/kernels/fp8.py:50-53 (`gemm`: torch._scaled_mm with
// unit scales, raw accumulator to bf16) plus the consumer kernels whose per-
// element work this epilogue absorbs: kernels/norm.py:161-175 (dequant_rows),
// kernels/norm.py:45-58 (residual / gated residual), kernels/norm.py:135-144
// (GELU-tanh), kernels/activation.py:26-40 (GeGLU / SwiGLU),
// kernels/rope.py:36-45 and kernels/wan.py:27-31 (rescale + bias).
//
// Matrix-core mapping. Both kernels issue v_mfma_f32_16x16x128_f8f6f4 with the
// WEIGHT fragment as source 0 (the MFMA "row" operand) and the ACTIVATION
// fragment as source 1 (the "column" operand). A lane then holds D[n0+4g+r][m]
// for r = 0..3 (g = lane/16, m = lane%16): four consecutive output columns of one
// token, so the epilogue reads sw/bias/gate and writes out in 8-16 byte pieces.
// Within one MFMA, lane l supplies row l%16 and the 32 K-bytes
// [32*(l/16), 32*(l/16)+32) of the 128-byte K slice, for both operands; any
// K permutation applied identically to both operands leaves the dot products
// unchanged.
//
// Kernels (dispatch in ifx_fp8_linear)
//  * gemm_big (M > 64, K % 128 == 0): 256 weight rows x 256 (or fewer) tokens
//    per workgroup, 32x32x64 MFMAs, operands copied global -> LDS by
//    direct-to-LDS DMA through a multi-stage ring, LDS-staged epilogue; split K
//    (+ splitk_reduce) when the output has too few tiles to fill the GPU.
//  * gemm_lds (M > 64 with K % 128 != 0): BN x BM tile, 16x16x128 MFMAs,
//    register-staged double-buffered LDS tiles (16-byte chunks XOR-swizzled by
//    row), epilogue from registers.
//  * gemm_skinny (M <= 64): bound by the weight stream. A workgroup owns 16 (32
//    for GLU) weight rows and the whole of K; its waves split the K steps,
//    stream weight fragments straight from HBM into MFMA registers, and add
//    their partial sums in LDS in a fixed order (deterministic).

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "ifx_abi.h"
#include "ifx_device.h"

namespace ifx {
namespace {

// ---------------------------------------------------------------------------
// Epilogue
// ---------------------------------------------------------------------------

struct Epi {
  const float* sa;       // [M] or null
  const float* sw;       // [N] or null (packed order for GLU)
  const float* bias;     // [N] or null (packed order for GLU)
  const void* res;       // [M, ldr] bf16 / f32 or null
  int64_t ldr;
  const uint16_t* gate;  // [N_out] bf16 or null
  void* out;             // [M, ldo] bf16 / f32
  int64_t ldo;
  int flags;
  int64_t M, N;
  int nt_out = 0;        // 1: large-M bf16 output rows stored nontemporally
};

// 8-byte nontemporal load / store (residual rows are read once; large
// outputs are written once and read back only after the next kernels'
// traffic has passed through the caches).
typedef unsigned v2u __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 ld8_nt(const void* p) {
  const v2u t = __builtin_nontemporal_load(static_cast<const v2u*>(p));
  return make_uint2(t.x, t.y);
}
__device__ __forceinline__ void st8_nt(void* p, uint2 v) {
  v2u t;
  t.x = v.x;
  t.y = v.y;
  __builtin_nontemporal_store(t, static_cast<v2u*>(p));
}

__device__ __forceinline__ float4 load_f4_or(const float* p, int64_t i, float dflt) {
  if (!p) return make_float4(dflt, dflt, dflt, dflt);
  return *reinterpret_cast<const float4*>(p + i);
}

// Token scale sa[m] (one shared value with IFX_EPI_SCALAR_SA; 1 if absent).
__device__ __forceinline__ float epi_sa(const Epi& e, int64_t m) {
  return e.sa ? e.sa[(e.flags & IFX_EPI_SCALAR_SA) ? 0 : m] : 1.0f;
}

// Weight scales sw[n..n+3] (one shared value with IFX_EPI_SCALAR_SW; 1 if absent).
__device__ __forceinline__ float4 epi_sw4(const Epi& e, int64_t n) {
  if (e.sw && (e.flags & IFX_EPI_SCALAR_SW)) {
    const float v = e.sw[0];
    return make_float4(v, v, v, v);
  }
  return load_f4_or(e.sw, n, 1.0f);
}

// y * g rounded on its own: the residual add that follows must not fuse with
// it, so every epilogue rounds the adaLN-gated value identically.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}

__device__ __forceinline__ void epi_store4(const Epi& e, int64_t m, int64_t c, const float* y);

// y (four consecutive output columns c..c+3 of row m, after activation) ->
// gate, residual, store.
__device__ __forceinline__ void epi_finish4(const Epi& e, int64_t m, int64_t c, float* y) {
  if (e.flags & IFX_EPI_GATE) {
    const uint2 g = *reinterpret_cast<const uint2*>(e.gate + c);
    y[0] = mul_rn(y[0], __uint_as_float(g.x << 16));
    y[1] = mul_rn(y[1], __uint_as_float(g.x & 0xFFFF0000u));
    y[2] = mul_rn(y[2], __uint_as_float(g.y << 16));
    y[3] = mul_rn(y[3], __uint_as_float(g.y & 0xFFFF0000u));
  }
  if (e.flags & IFX_EPI_RESIDUAL) {
    if (e.flags & IFX_EPI_RES_F32) {
      const float4 r = *reinterpret_cast<const float4*>(static_cast<const float*>(e.res) + m * e.ldr + c);
      y[0] += r.x; y[1] += r.y; y[2] += r.z; y[3] += r.w;
    } else {
      const uint2 r = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(e.res) + m * e.ldr + c);
      y[0] += __uint_as_float(r.x << 16);
      y[1] += __uint_as_float(r.x & 0xFFFF0000u);
      y[2] += __uint_as_float(r.y << 16);
      y[3] += __uint_as_float(r.y & 0xFFFF0000u);
    }
  }
  epi_store4(e, m, c, y);
}

// First half of the epilogue for one lane's D fragment (weight rows n..n+3,
// token m): dequantization scales, bias, GELU. Caller guarantees m < M, n < N.
__device__ __forceinline__ void epi_pre(const Epi& e, const v4f acc, int64_t n, int64_t m, float* y) {
  const float sa = epi_sa(e, m);
  const float4 sw = epi_sw4(e, n);
  const float4 b = load_f4_or((e.flags & IFX_EPI_BIAS) ? e.bias : nullptr, n, 0.0f);
  y[0] = acc[0] * sa * sw.x + b.x;
  y[1] = acc[1] * sa * sw.y + b.y;
  y[2] = acc[2] * sa * sw.z + b.z;
  y[3] = acc[3] * sa * sw.w + b.w;
  if (e.flags & IFX_EPI_GELU_TANH) {
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = gelu_tanh(y[r]);
  }
}

// Store four finished values at out[m, c..c+3] (bf16; f32 with IFX_EPI_OUT_F32,
// fp16 with IFX_EPI_OUT_F16).
__device__ __forceinline__ void epi_store4(const Epi& e, int64_t m, int64_t c, const float* y) {
  if (e.flags & IFX_EPI_OUT_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(e.out) + m * e.ldo + c) = make_float4(y[0], y[1], y[2], y[3]);
  } else if (e.flags & IFX_EPI_OUT_F16) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 h = {static_cast<_Float16>(y[0]), static_cast<_Float16>(y[1]), static_cast<_Float16>(y[2]),
                  static_cast<_Float16>(y[3])};
    *reinterpret_cast<h4*>(static_cast<_Float16*>(e.out) + m * e.ldo + c) = h;
  } else {
    uint2 o;
    o.x = pack_bf16x2(y[0], y[1]);
    o.y = pack_bf16x2(y[2], y[3]);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(e.out) + m * e.ldo + c) = o;
  }
}

// residual[m, c..c+3] widened to fp32 (bf16 or f32 residual).
__device__ __forceinline__ float4 load_res4(const Epi& e, int64_t m, int64_t c) {
  if (e.flags & IFX_EPI_RES_F32)
    return *reinterpret_cast<const float4*>(static_cast<const float*>(e.res) + m * e.ldr + c);
  const uint2 r = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(e.res) + m * e.ldr + c);
  return make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xFFFF0000u), __uint_as_float(r.y << 16),
                     __uint_as_float(r.y & 0xFFFF0000u));
}

// Plain epilogue for one lane's D fragment: rows n..n+3 of W, token m.
__device__ __forceinline__ void epi_store(const Epi& e, const v4f acc, int64_t n, int64_t m) {
  if (m >= e.M || n >= e.N) return;
  float y[4];
  epi_pre(e, acc, n, m, y);
  epi_finish4(e, m, n, y);
}

// GLU first half: `ng` is the packed row of the gate fragment, the up fragment
// is 16 packed rows later. Caller guarantees m < M, ng < N.
__device__ __forceinline__ void epi_pre_glu(const Epi& e, const v4f accg, const v4f accu, int64_t ng,
                                            int64_t m, float* y) {
  const float sa = epi_sa(e, m);
  const float4 swg = epi_sw4(e, ng);
  const float4 swu = epi_sw4(e, ng + 16);
  const float* bp = (e.flags & IFX_EPI_BIAS) ? e.bias : nullptr;
  const float4 bg = load_f4_or(bp, ng, 0.0f);
  const float4 bu = load_f4_or(bp, ng + 16, 0.0f);
  const float g[4] = {accg[0] * sa * swg.x + bg.x, accg[1] * sa * swg.y + bg.y,
                      accg[2] * sa * swg.z + bg.z, accg[3] * sa * swg.w + bg.w};
  const float u[4] = {accu[0] * sa * swu.x + bu.x, accu[1] * sa * swu.y + bu.y,
                      accu[2] * sa * swu.z + bu.z, accu[3] * sa * swu.w + bu.w};
  const bool swiglu = (e.flags & IFX_EPI_SWIGLU) != 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) y[r] = (swiglu ? silu(g[r]) : gelu_tanh(g[r])) * u[r];
}

// GLU epilogue; output column = (ng / 32) * 16 + (ng % 16).
__device__ __forceinline__ void epi_store_glu(const Epi& e, const v4f accg, const v4f accu, int64_t ng,
                                              int64_t m) {
  if (m >= e.M || ng >= e.N) return;
  float y[4];
  epi_pre_glu(e, accg, accu, ng, m, y);
  epi_finish4(e, m, (ng >> 5) * 16 + (ng & 15), y);
}

__device__ __forceinline__ v4f mfma16(const v8i& w, const v8i& a, const v4f& c) {
  // cbsz = blgp = 0: both operands are FP8 E4M3 (OCP); no block scales.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w, a, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ v8i cat8(const v4i lo, const v4i hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ v4i ld16(const uint8_t* p) { return *reinterpret_cast<const v4i*>(p); }
// Streaming load: the weight stream of a skinny GEMM is read once per call.
__device__ __forceinline__ v4i ld16_nt(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
}

// ---------------------------------------------------------------------------
// Large-M kernel: LDS double-buffered tiles
// ---------------------------------------------------------------------------

constexpr int kBK = 128;  // K bytes per stage (one MFMA K step)

template <int BN, int BM, int WGN, int WGM, bool GLU>
struct TileCfg {
  static constexpr int kThreads = WGN * WGM * 64;
  static constexpr int kTN = BN / WGN;  // wave tile (weight rows)
  static constexpr int kTM = BM / WGM;  // wave tile (tokens)
  static constexpr int kFN = kTN / 16;
  static constexpr int kFM = kTM / 16;
  static constexpr int kCW = BN * 8 / kThreads;  // 16-byte chunks per thread per stage
  static constexpr int kCA = BM * 8 / kThreads;
  static constexpr int kStageBytes = (BN + BM) * kBK;
  static_assert(kTN % 16 == 0 && kTM % 16 == 0, "wave tile");
  static_assert(!GLU || kFN % 2 == 0, "GLU needs gate/up fragment pairs");
  static_assert(BN * 8 % kThreads == 0 && BM * 8 % kThreads == 0, "load split");
  static_assert(2 * kStageBytes <= 160 * 1024, "LDS");
};

// Byte offset of 16-byte chunk `ch` of tile row `row` (rows are 128 bytes).
// gfx950's LDS serves a ds_read_b128 16 lanes at a time from 64 banks (a
// 256-byte window = two tile rows). A fragment read has 16 lanes on 16
// consecutive rows with the same logical chunk, so the physical chunk
// ch ^ f(row), f(row) = (row % 8) ^ ((row / 8) % 2), must put every
// (row parity, chunk) pair in a different place: f is a bijection on the even
// and on the odd rows of any 16-row block (and on any 8 consecutive rows,
// which also keeps a 32-bank, 8-lanes-per-cycle LDS conflict free).
__device__ __forceinline__ int swz_f(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int swz(int row, int ch) { return row * kBK + ((ch ^ swz_f(row)) << 4); }

template <int BN, int BM, int WGN, int WGM, bool GLU>
__global__ __launch_bounds__(WGN* WGM * 64, 1) void gemm_lds(const uint8_t* __restrict__ A, int64_t lda,
                                                             const uint8_t* __restrict__ W, int64_t ldw,
                                                             int64_t K, int tiles_m, Epi e) {
  using C = TileCfg<BN, BM, WGN, WGM, GLU>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * C::kStageBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wn = wave / WGM;
  const int wm = wave % WGM;

  // Tile order: consecutive workgroups walk M first, sharing one weight tile.
  const int tm = blockIdx.x % tiles_m;
  const int tn = blockIdx.x / tiles_m;
  const int64_t n0 = static_cast<int64_t>(tn) * BN;
  const int64_t m0 = static_cast<int64_t>(tm) * BM;
  const int nk = static_cast<int>((K + kBK - 1) / kBK);

  // Per-thread global chunk coordinates (fixed across stages).
  const uint8_t* wsrc[C::kCW];
  int wdst[C::kCW];
#pragma unroll
  for (int i = 0; i < C::kCW; ++i) {
    const int c = tid + i * C::kThreads;
    const int row = c >> 3, ch = c & 7;
    int64_t n = n0 + row;
    n = n < e.N ? n : e.N - 1;  // clamp: rows past N are computed but never stored
    wsrc[i] = W + n * ldw + ch * 16;
    wdst[i] = swz(row, ch);
  }
  const uint8_t* asrc[C::kCA];
  int adst[C::kCA];
#pragma unroll
  for (int i = 0; i < C::kCA; ++i) {
    const int c = tid + i * C::kThreads;
    const int row = c >> 3, ch = c & 7;
    int64_t m = m0 + row;
    m = m < e.M ? m : e.M - 1;
    asrc[i] = A + m * lda + ch * 16;
    adst[i] = BN * kBK + swz(row, ch);
  }

  uint4 pw[C::kCW], pa[C::kCA];
  auto gload = [&](int kt) {
    const int64_t k0 = static_cast<int64_t>(kt) * kBK;
#pragma unroll
    for (int i = 0; i < C::kCW; ++i) {
      const int ch = (tid + i * C::kThreads) & 7;
      pw[i] = (k0 + ch * 16 < K) ? *reinterpret_cast<const uint4*>(wsrc[i] + k0) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < C::kCA; ++i) {
      const int ch = (tid + i * C::kThreads) & 7;
      pa[i] = (k0 + ch * 16 < K) ? *reinterpret_cast<const uint4*>(asrc[i] + k0) : make_uint4(0, 0, 0, 0);
    }
  };
  auto sstore = [&](int buf) {
    uint8_t* base = smem + buf * C::kStageBytes;
#pragma unroll
    for (int i = 0; i < C::kCW; ++i) *reinterpret_cast<uint4*>(base + wdst[i]) = pw[i];
#pragma unroll
    for (int i = 0; i < C::kCA; ++i) *reinterpret_cast<uint4*>(base + adst[i]) = pa[i];
  };

  v4f acc[C::kFN][C::kFM];
#pragma unroll
  for (int i = 0; i < C::kFN; ++i)
#pragma unroll
    for (int j = 0; j < C::kFM; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // Fragment read offsets: lane supplies row lane%16, chunks 2g and 2g+1.
  const int frow = lane & 15;
  const int g = lane >> 4;

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
    const uint8_t* base = smem + buf * C::kStageBytes;
    v8i af[C::kFM];
#pragma unroll
    for (int j = 0; j < C::kFM; ++j) {
      const int row = wm * C::kTM + j * 16 + frow;
      const uint8_t* p = base + BN * kBK;
      af[j] = cat8(ld16(p + swz(row, 2 * g)), ld16(p + swz(row, 2 * g + 1)));
    }
#pragma unroll
    for (int i = 0; i < C::kFN; ++i) {
      const int row = wn * C::kTN + i * 16 + frow;
      const v8i wf = cat8(ld16(base + swz(row, 2 * g)), ld16(base + swz(row, 2 * g + 1)));
#pragma unroll
      for (int j = 0; j < C::kFM; ++j) acc[i][j] = mfma16(wf, af[j], acc[i][j]);
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

  // Epilogue straight from the accumulators.
  const int64_t nb = n0 + wn * C::kTN + 4 * g;
  const int64_t mb = m0 + wm * C::kTM + frow;
  if constexpr (GLU) {
#pragma unroll
    for (int i = 0; i < C::kFN; i += 2)
#pragma unroll
      for (int j = 0; j < C::kFM; ++j) epi_store_glu(e, acc[i][j], acc[i + 1][j], nb + i * 16, mb + j * 16);
  } else {
#pragma unroll
    for (int i = 0; i < C::kFN; ++i)
#pragma unroll
      for (int j = 0; j < C::kFM; ++j) epi_store(e, acc[i][j], nb + i * 16, mb + j * 16);
  }
}

// ---------------------------------------------------------------------------
// Large-M kernel: direct-to-LDS multi-stage ring, 32x32x64 matrix cores
// ---------------------------------------------------------------------------
//
// Workgroup tile: BN weight rows x BM tokens, 2 x BM/(32 FM) waves (2 along
// weight rows), wave tile BN/2 x 32 FM: 128 x 64 with 8 waves (FM = 2), or
// 128 x 128 with 4 waves (FM = 4: accumulators in AccVGPRs, a third less LDS
// read traffic per MFMA, and a register-pipelined K loop, described at the
// loop), built from v_mfma_f32_32x32x64_f8f6f4 (the 32x32 form keeps
// the matrix pipe ~97% busy from a single wave per SIMD on gfx950; the 16x16x128
// form reaches ~75% there). Operand roles as in the other kernels: weights are
// source 0, so a lane of a 32x32 fragment holds, for q = 0..3, the four
// consecutive weight rows 8q + 4*(lane/32) + 0..3 of token lane%32.
//
// Stage = (256 + BM) rows x KB K-bytes (KB = 64 or 128), STAGES stages in a
// ring. Global -> LDS copies use gfx950's global_load_lds_dwordx4: one
// instruction moves 64 lanes x 16 B into a contiguous 1 KB LDS block, lane l
// landing at byte 16*l; the row swizzle (`Swz`) is therefore applied on the
// global side, each lane fetching the logical chunk that belongs at its LDS
// position. K must be a multiple of KB (whole stages, no zero fill).
//
// OCC workgroups share a CU (OCC = 2 with 64-byte stages: 3 x 24 KB of LDS and
// <= 128 VGPRs per wave), so one workgroup's barrier waits, epilogue and store
// drain overlap the other's matrix-core work.
//
// Pipeline: loads run STAGES-1 stages ahead; one barrier per K step.
//   wait until this wave's loads of stage k landed (vmcnt <= loads still
//   allowed in flight); s_barrier (stage k visible to all; all waves finished
//   stage k-1, whose slot is reused next); issue stage k+STAGES-1; MFMAs on k.
// The barrier is the bare s_barrier: a __syncthreads() fence would also wait
// for the loads that are meant to stay in flight.

// LDS layout of a tile with KB-byte rows: 16-byte chunk `ch` of row `row` is
// stored at chunk position ch ^ f(row). gfx950's LDS serves a ds_read_b128 16
// lanes at a time from 64 banks (a 256-byte window); a fragment read puts 16
// lanes on 16 consecutive rows with the same logical chunk, so f must send
// those 16 reads to 16 different 16-byte bank groups:
//   KB = 128 (two rows per window): f(r) = (r % 8) ^ ((r / 8) % 2)
//   KB = 64  (four rows per window): f(r) = (r / 4) % 4
template <int KB>
struct Swz {
  static constexpr int kChunks = KB / 16;
  static __device__ __forceinline__ int f(int row) {
    if constexpr (KB == 128) return (row & 7) ^ ((row >> 3) & 1);
    else return (row >> 2) & 3;
  }
  static __device__ __forceinline__ int off(int row, int ch) { return row * KB + ((ch ^ f(row)) << 4); }
};

// Tile order. The hardware hands workgroup b to XCD b % 8, and each XCD has its
// own L2. Workgroup b is given logical tile xcd * per_xcd + b / 8, so every XCD
// walks one contiguous range of logical tiles; logical tiles are ordered in
// groups of `group_m` token-tile rows, walking the weight tiles inside a group
// (tile (tm, tn) with tm fastest), so the ~32 tiles an XCD runs at once form a
// compact block that shares weight and token panels in that XCD's L2.
// With split-K the logical index also carries the K slice (slowest), so the
// slices of one tile are spread over all XCDs.
struct TileMap {
  int tiles_m, tiles_n, group_m, per_xcd, ksplit;
};

__device__ __forceinline__ bool map_tile(const TileMap& t, int& tm, int& tn, int& split) {
  const int b = blockIdx.x;
  int logical = (b & 7) * t.per_xcd + (b >> 3);
  const int tiles = t.tiles_m * t.tiles_n;
  if (logical >= tiles * t.ksplit) return false;
  split = logical / tiles;
  logical -= split * tiles;
  const int per_group = t.group_m * t.tiles_n;
  const int grp = logical / per_group;
  const int first_m = grp * t.group_m;
  const int gsize = min(t.tiles_m - first_m, t.group_m);
  const int r = logical - grp * per_group;
  tm = first_m + r % gsize;
  tn = r / gsize;
  // Groups run on different XCDs (one group of 4 token tiles per XCD at C5's
  // shapes), and every group sweeps all weight tiles: start each group's sweep
  // at a different eighth of them (a bijection within the group), so the XCDs
  // do not fetch the same weight panel from HBM at the same time when the
  // weights are not yet in the memory-side cache (C5 step 1189 -> 1094 us;
  // C5 up with weights not cached 366 -> 337 us).
  tn += (grp & 7) * t.tiles_n / 8;
  if (tn >= t.tiles_n) tn -= t.tiles_n;
  return true;
}

__host__ inline TileMap make_tile_map(int64_t tiles_m, int64_t tiles_n, int ksplit = 1) {
  TileMap t;
  t.tiles_m = static_cast<int>(tiles_m);
  t.tiles_n = static_cast<int>(tiles_n);
  t.group_m = static_cast<int>(tiles_m < 4 ? tiles_m : 4);
  t.ksplit = ksplit;
  t.per_xcd = static_cast<int>((tiles_m * tiles_n * ksplit + 7) / 8);
  return t;
}

// Split-K partial sums: raw fp32 accumulators of K slice s at
// base + (s * M + m) * ld + n (n = packed weight row), written by gemm_big and
// summed in slice order by splitk_reduce.
struct Partials {
  float* base;
  int64_t ld;
  int64_t kstages;  // K stages per slice
};

__device__ __forceinline__ v16f mfma32(const v8i& w, const v8i& a, const v16f& c) {
  // cbsz = blgp = 0: both operands FP8 E4M3 (OCP); no block scales.
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, a, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ v4f quad(const v16f& v, int q) {
  return v4f{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
}

template <int BM, int BN, int KB, int STAGES, int OCC, bool GLU, int FM>
__global__ __launch_bounds__(4 * BM / FM, OCC) void gemm_big(const uint8_t* __restrict__ A, int64_t lda,
                                                     const uint8_t* __restrict__ W, int64_t ldw, int64_t K,
                                                     TileMap tmap, Epi e, Partials part) {
  using S = Swz<KB>;
  constexpr int kRows = BN + BM;
  constexpr int kStage = kRows * KB;
  constexpr int kRowsPerDma = 1024 / KB;           // rows one DMA instruction fills
  constexpr int kWT = 32 * FM;                     // tokens per wave tile
  constexpr int kWM = BM / kWT;                    // waves along tokens (2 along weight rows)
  constexpr int kWaves = 2 * kWM;
  constexpr int kLoads = kRows / kRowsPerDma / kWaves;  // DMA instructions per wave per stage
  constexpr int kFN = BN / 64;                     // 32-row weight fragments per wave (2 waves along BN)
  static_assert(BN % 64 == 0 && BN >= 128 && BN <= 256, "weight tile");
  constexpr int kFM = FM;                          // 32-token fragments per wave
  constexpr int kHalves = KB / 64;                 // 32x32x64 K steps per stage
  static_assert(BM % kWT == 0 && kRows % (kWaves * kRowsPerDma) == 0, "tile");
  static_assert(KB == 64 || KB == 128, "stage depth");
  constexpr int kPitch = 128 + 4;                  // floats per epilogue tile row
  constexpr int kEpiBytes = kWaves * 32 * kPitch * 4;
  // The 4-wave wide tiles keep the weight rows of three stages and the token
  // rows of two (a weight-row ring one stage deeper than the token-row ring):
  // 3 x BN x 128 + 2 x 256 x 128 bytes (160 KB at BN = 256). In an engine the
  // weights arrive from HBM while the token rows were just written by their
  // producer (C5 step 1004 -> 996 us against the token rows three deep). The
  // token scales of the epilogue then live in the ring's space after the K loop.
  constexpr bool kW3 = FM == 4 && KB == 128 && STAGES == 2;
  constexpr int kWSlot = BN * KB, kASlot = BM * KB;  // bytes of one stage's weight / token rows
  constexpr int kRing = kW3 ? 3 * kWSlot + 2 * kASlot : STAGES * kStage;
  constexpr int kSmem = kRing > kEpiBytes + BM * 4 ? kRing : kEpiBytes + BM * 4;
  // the token scales (s_sa): after the ring, or (kW3) inside it after the K loop
  constexpr int kLds = kW3 ? kSmem : kSmem + BM * 4;
  static_assert(OCC * kLds <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kLds];
  float* const s_sa = reinterpret_cast<float*>(smem + (kW3 ? kEpiBytes : kSmem));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  const int wn = wave / kWM;  // weight-row half
  const int wm = wave % kWM;  // token slice of kWT tokens

  int tm, tn, split;
  if (!map_tile(tmap, tm, tn, split)) return;
  const int64_t n0 = static_cast<int64_t>(tn) * BN;
  const int64_t m0 = static_cast<int64_t>(tm) * BM;
  // this workgroup's K stages: [kt0, kt0 + nk)
  const int kt0 = static_cast<int>(split * part.kstages);
  const int nk = static_cast<int>(min(static_cast<int64_t>(K / KB) - kt0, part.kstages));

  // Epilogue operands of this lane (column scales, bias, adaLN gate) and this
  // thread's token scale, loaded before the K loop so their latency hides
  // under it (after the loop they were a serialized round trip per tile).
  constexpr int kCols = GLU ? 16 * kFN : 32 * kFN;  // output columns of a wave tile
  constexpr int kLanesPerRow = kCols / 4;
  // whole rows per 64-lane pass, a power of two (12 lanes per row for 192-row
  // GLU tiles: 4 rows, 16 lanes idle)
  constexpr int kRowsPerPass = 64 / kLanesPerRow >= 8 ? 8 : 64 / kLanesPerRow >= 4 ? 4 : 64 / kLanesPerRow >= 2 ? 2 : 1;
  constexpr int kRowIters = 32 / kRowsPerPass;
  static_assert(32 % kRowsPerPass == 0, "epilogue row passes");
  const int64_t nw = n0 + wn * (32 * kFN);                // first (packed) weight row of the wave tile
  const int64_t mw = m0 + wm * kWT;                 // first token of the wave tile
  const int oc = (lane % kLanesPerRow) * 4;        // this lane's first output column in the tile
  const int pc = GLU ? (oc / 16) * 32 + (oc % 16) : oc;  // its (gate) packed column
  const int64_t c_out = (GLU ? nw / 2 : nw) + oc;
  // lanes past kRowsPerPass whole rows (96-column tiles) have no column of their own
  const bool col_ok = lane < kRowsPerPass * kLanesPerRow && c_out < (GLU ? e.N / 2 : e.N);
  const int64_t np = col_ok ? nw + pc : 0;         // packed weight row (any valid row if unused)
  const float* bp = (e.flags & IFX_EPI_BIAS) ? e.bias : nullptr;
  const float4 sw0 = epi_sw4(e, np);
  const float4 b0 = load_f4_or(bp, np, 0.0f);
  const float4 sw1 = GLU ? epi_sw4(e, np + 16) : sw0;
  const float4 b1 = GLU ? load_f4_or(bp, np + 16, 0.0f) : b0;
  uint2 g2 = make_uint2(0x3F803F80u, 0x3F803F80u);  // bf16 1.0 x 4
  if ((e.flags & IFX_EPI_GATE) && col_ok) g2 = *reinterpret_cast<const uint2*>(e.gate + c_out);
  const float sa_pre = tid < BM ? epi_sa(e, min(m0 + tid, e.M - 1)) : 0.0f;

  // DMA load i of a stage covers rows kRowsPerDma*blk .. +kRowsPerDma-1
  // (blk = wave*kLoads + i; weight rows first, then token rows). Rows past N/M
  // are clamped: computed, never stored. Addresses are formed per stage to keep
  // VGPRs free.
  const int lrow = lane / S::kChunks;
  const int lpos = lane % S::kChunks;
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_offset(smem) + wave * kLoads * 1024);
  const int64_t n_last = e.N - 1, m_last = e.M - 1;
  auto issue = [&](int kl) {  // local stage index kl: K stage kt0 + kl, ring slot kl % STAGES
    const int kt = kt0 + kl;
    const uint32_t buf = lds_base + (kl % STAGES) * kStage;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int blk = wave * kLoads + i;
      const int row = blk * kRowsPerDma + lrow;
      const int64_t k0 = static_cast<int64_t>(kt) * KB + ((lpos ^ S::f(row)) << 4);
      const uint8_t* p;
      if (blk * kRowsPerDma < BN) {  // wave-uniform
        p = W + min(n0 + row, n_last) * ldw + k0;
      } else {
        p = A + min(m0 + (row - BN), m_last) * lda + k0;
      }
      dma16(p, buf + i * 1024);
    }
  };

  v16f acc[kFN][kFM];
#pragma unroll
  for (int i = 0; i < kFN; ++i)
#pragma unroll
    for (int j = 0; j < kFM; ++j) acc[i][j] = v16f{};

  // 32x32x64 fragment of K step h of the stage: lane l supplies row l%32 and the
  // K bytes [64h + 32*(l/32), +32) = chunks 4h + 2*(l/32) + {0,1}.
  const int frow = lane & 31;
  const int fhalf = lane >> 5;
  auto compute = [&](const uint8_t* base) {
#pragma unroll
    for (int h = 0; h < kHalves; ++h) {
      const int c0 = 4 * h + 2 * fhalf;
      v8i af[kFM];
#pragma unroll
      for (int j = 0; j < kFM; ++j) {
        const int row = BN + wm * kWT + j * 32 + frow;
        af[j] = cat8(ld16(base + S::off(row, c0)), ld16(base + S::off(row, c0 + 1)));
      }
#pragma unroll
      for (int i = 0; i < kFN; ++i) {
        const int row = wn * (32 * kFN) + i * 32 + frow;
        const v8i wf = cat8(ld16(base + S::off(row, c0)), ld16(base + S::off(row, c0 + 1)));
#pragma unroll
        for (int j = 0; j < kFM; ++j) {
          acc[i][j] = mfma32(wf, af[j], acc[i][j]);
        }
      }
    }
  };

  if constexpr (FM == 4 || (FM == 2 && BM == 128)) {
    // Register-pipelined 4-wave form (wave tile 128 x 128 for 256-token tiles,
    // 64 x 128 for 128-token tiles; accumulators in AccVGPRs). A 128-byte stage holds two 32x32x64 K steps (halves); the
    // fragments of the next half are read from LDS into the other register
    // set while the MFMAs of the current half run, so the matrix pipe does not
    // wait on LDS latency. Per stage kt:
    //   half 0: MFMAs on (kt, 0), reads of (kt, 1);
    //   s_waitcnt lgkmcnt(0) (this wave is done reading slot kt) and vmcnt
    //   (its DMA of stage kt+1 landed; those of the STAGES-2 later stages may
    //   stay in flight); s_barrier (for every wave: stage kt+1 is in LDS and
    //   slot kt is free);
    //   half 1: MFMAs on (kt, 1), reads of (kt+1, 0), and the DMA of stage
    //   kt+STAGES into slot kt, one instruction after each MFMA.
    static_assert(KB == 128 && (STAGES == 2 || STAGES == 3) && kWaves == 4 && kFN >= 3 && kFN <= 4,
                  "4-wave layout");
    constexpr int kMF = kFN * kFM;        // MFMAs per half
    constexpr int kRd = 2 * (kFN + kFM);  // 16-byte LDS reads per half
    static_assert(kLoads <= kRd && kLoads % 2 == 0, "one DMA per LDS read");
    // DMA sources: a wave-uniform choice of operand and a 32-bit byte offset
    // per lane, formed per instruction (row clamp + 24-bit multiply-add) so no
    // address registers stay live; the launch guarantees both operands span
    // < 4 GiB with rows and row strides below 2^24. DMA i of a stage covers
    // tile rows 8 * (wave * kLoads + i) + lrow (weight rows first).
    static_assert(kRowsPerDma == 8, "128-byte rows");
    // Which 1 KB blocks (8 rows) of a stage wave `wave` fills: with kW3 every
    // wave takes BN / 32 weight blocks and BM / 32 token blocks (the same
    // split for all waves, so all wait for the same counts); otherwise blocks
    // wave * kLoads .. + kLoads - 1 of [weight blocks | token blocks].
    constexpr int kW4 = BN / 32, kA4 = BM / 32;  // kW3: weight / token DMAs per wave per stage
    static_assert(!kW3 || kW4 + kA4 == kLoads, "kW3 DMA split");
    const int iw = kW3 ? kW4 : BN / 8 - wave * kLoads;  // DMAs i < iw of this wave load weight rows
    uint32_t doff[kLoads];                  // per-lane byte offset of DMA i, stage kt0
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int blk = kW3 ? (i < kW4 ? wave * kW4 + i : BN / 8 + wave * kA4 + (i - kW4)) : wave * kLoads + i;
      const int r = blk * 8 + lrow;
      const bool isw = i < iw;
      const uint32_t row = static_cast<uint32_t>(isw ? min(n0 + r, n_last) : min(m0 + (r - BN), m_last));
      doff[i] = __umul24(row, static_cast<uint32_t>(isw ? ldw : lda)) +
                static_cast<uint32_t>(((lpos ^ lrow ^ (blk & 1)) << 4) + kt0 * KB);
    }
    const uint64_t wbase = reinterpret_cast<uintptr_t>(W), abase = reinterpret_cast<uintptr_t>(A);
    // LDS byte offsets (from smem) of stage kl's weight rows and token rows
    auto wslot = [&](int kl) -> uint32_t {
      return kW3 ? (kl % 3) * kWSlot : (kl % STAGES) * kStage;
    };
    auto aslot = [&](int kl) -> uint32_t {
      return kW3 ? 3 * kWSlot + (kl & 1) * kASlot : (kl % STAGES) * kStage + kWSlot;
    };
    // kW3: DMA index of issue slot m. The token rows are issued first and the
    // weight rows after them, so the weight rows are the newest in flight.
    auto dma_at = [](int m) { return kW3 ? (m < kA4 ? kW4 + m : m - kA4) : m; };
    // DMA i of this wave: weight rows of stage klw (i < iw) or token rows of
    // stage kla; block blk = wave * kLoads + i lands at row 8 * blk of its stage
    // (token rows counted from BN).
    // wdst / adst: this wave's LDS destination bases (lds_base + slot) of the
    // stages its weight / token DMAs fill, formed once per stage
    auto dma_one = [&](int klw, int kla, uint32_t wdst, uint32_t adst, int i) {
      const bool isw = i < iw;  // wave-uniform
      // branch-free wave-uniform choice of the operand base
      const uint64_t sel = static_cast<uint64_t>(-static_cast<int64_t>(isw));
      const uint8_t* base = reinterpret_cast<const uint8_t*>(abase ^ ((wbase ^ abase) & sel));
      const int kl = isw ? klw : kla;
      dma16s(base, doff[i] + static_cast<uint32_t>(kl) * KB, (isw ? wdst : adst) + i * 1024);
    };
    // bases such that DMA i lands at base + i * 1024
    const uint32_t smem_off = lds_offset(smem);
    auto wdst_of = [&](int kl) {
      return __builtin_amdgcn_readfirstlane(kW3 ? smem_off + wslot(kl) + wave * kW4 * 1024 : lds_base + wslot(kl));
    };
    auto adst_of = [&](int kl) {
      return __builtin_amdgcn_readfirstlane(kW3 ? smem_off + aslot(kl) + (wave * kA4 - kW4) * 1024
                                                : lds_base + aslot(kl) - kWSlot);
    };
    // 16-byte fragment halves: W fragments i at (2i, 2i+1), token fragments j at (2kFN+2j, 2kFN+2j+1)
    v4i fr[2][kRd];
    // Token fragments past M: a wave whose 32-token fragments j >= JV lie
    // wholly past the last token (the last token tile of an M that is not a
    // multiple of the tile) skips their LDS reads and MFMAs. JV is a
    // compile-time count (kFM, kFM / 2 or 0), the smallest that covers the
    // wave's tokens, so a partial tile costs fewer matrix-core cycles.
    // wp / ap: the stage's weight-row and token-row slots
    auto read_one = [&](const uint8_t* wp, const uint8_t* ap, v4i* f, int h, int r, auto jv_tag) {
      constexpr int JV = decltype(jv_tag)::value;
      const int ch = 4 * h + 2 * fhalf + (r & 1);
      if (r < 2 * kFN) {
        f[r] = ld16(wp + S::off(wn * (32 * kFN) + (r >> 1) * 32 + frow, ch));
      } else if ((r - 2 * kFN) >> 1 < JV) {
        f[r] = ld16(ap + S::off(wm * kWT + ((r - 2 * kFN) >> 1) * 32 + frow, ch));
      }
    };

    auto mfma_one = [&](const v4i* f, int m, auto jv_tag) {
      constexpr int JV = decltype(jv_tag)::value;
      const int i = m / kFM, j = m % kFM;
      if (j < JV)
        acc[i][j] = mfma32(cat8(f[2 * i], f[2 * i + 1]), cat8(f[2 * kFN + 2 * j], f[2 * kFN + 2 * j + 1]), acc[i][j]);
    };
    auto interleave = [](auto jv_tag) {  // keep the MFMA / LDS-read alternation
      constexpr int JV = decltype(jv_tag)::value;
      constexpr int kMFv = kFN * JV, kRdv = 2 * (kFN + JV);
#pragma unroll
      for (int m = 0; m < kMFv; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      if constexpr (kRdv > kMFv) __builtin_amdgcn_sched_group_barrier(0x100, kRdv - kMFv, 0);
    };
    using std::integral_constant;
    constexpr integral_constant<int, kFM> kAllFrags{};
    auto wait_lgkm0 = [] { __builtin_amdgcn_s_waitcnt(0xC07F); };  // lgkmcnt(0), visible to the compiler
    auto sync = [&] {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
    if constexpr (kW3) {
      // Weight rows three stages deep, token rows two. Stage kt's second half
      // issues the token rows of stage kt+2 and the weight rows of stage kt+3
      // (token DMAs first), both into the slots stage kt has just freed; the
      // barrier of stage kt then needs everything but the newest weight rows
      // (stage kt+2), which stay in flight: weight rows get two stages of lead.
      // Prologue order per wave: A0 W0 A1 W1 W2 (each its own DMAs only).
#pragma unroll
      for (int s = 0; s < 3; ++s) {
        const uint32_t wd = wdst_of(s), ad = adst_of(s);
#pragma unroll
        for (int m = 0; m < kLoads; ++m) {
          const int i = dma_at(m);
          if (i < iw) {
            if (s < nk) dma_one(s, 0, wd, ad, i);
          } else if (s < 2 && s < nk) {
            dma_one(0, s, wd, ad, i);
          }
        }
      }
      if (nk >= 3) wait_vmcnt<kLoads + kW4>();  // this wave's A1 W1 W2 may stay in flight
      else if (nk == 2) wait_vmcnt<kLoads>();
      else wait_vmcnt<0>();
    } else {
      // prologue: stages 0 .. STAGES-1 in flight, stage 0 landed
#pragma unroll
      for (int s = 0; s < STAGES; ++s)
        if (s < nk) {
          const uint32_t wd = wdst_of(s), ad = adst_of(s);
#pragma unroll
          for (int i = 0; i < kLoads; ++i) dma_one(s, s, wd, ad, i);
        }
      if (nk >= STAGES) wait_vmcnt<(STAGES - 1) * kLoads>();
      else wait_vmcnt<0>();
    }
    sync();
#pragma unroll
    for (int r = 0; r < kRd; ++r) read_one(smem + wslot(0), smem + aslot(0), fr[0], 0, r, kAllFrags);  // stage 0's half 0
    // kDma2: stage kt + STAGES exists (kW3: its token rows are issued here);
    // kDma3 (kW3): stage kt + 3 exists (its weight rows are issued here).
    auto stage = [&](int kt, auto dma2_tag, auto dma3_tag, auto jv) {
      constexpr bool kDma2 = decltype(dma2_tag)::value;
      constexpr bool kDma3 = decltype(dma3_tag)::value;
      const uint8_t* wcur = smem + wslot(kt);
      const uint8_t* acur = smem + aslot(kt);
      const uint8_t* wnxt = smem + wslot(kt + 1);  // after the last stage: a settled slot, unused
      const uint8_t* anxt = smem + aslot(kt + 1);
      wait_lgkm0();
#pragma unroll
      for (int m = 0; m < kRd; ++m) {
        if (m < kMF) mfma_one(fr[0], m, jv);
        read_one(wcur, acur, fr[1], 1, m, jv);
      }
      interleave(jv);
      wait_lgkm0();
      if constexpr (kW3) {
        // stage kt+1 landed; the weight rows of stage kt+2 may stay in flight
        if (kt + 2 < nk) wait_vmcnt<kW4>();
        else if (kt + 1 < nk) wait_vmcnt<0>();
      } else {
        if (kDma2 || kt + STAGES - 1 < nk) wait_vmcnt<(STAGES - 2) * kLoads>();  // stages up to kt+STAGES-1 issued
        else if (kt + 1 < nk) wait_vmcnt<0>();
      }
      sync();
      // DMA destinations: kW3 weight rows of stage kt+3 and token rows of
      // stage kt+2 (both the slots of stage kt); otherwise stage kt+STAGES
      const uint32_t wd = wdst_of(kW3 ? kt + 3 : kt + STAGES);
      const uint32_t ad = adst_of(kW3 ? kt + 2 : kt + STAGES);
#pragma unroll
      for (int m = 0; m < kRd; ++m) {
        if (m < kMF) mfma_one(fr[1], m, jv);
        read_one(wnxt, anxt, fr[0], 0, m, jv);
        if (m < kLoads) {
          if constexpr (kW3) {
            const int i = dma_at(m);
            if (i < iw) {
              if constexpr (kDma3) dma_one(kt + 3, 0, wd, ad, i);
            } else {
              if constexpr (kDma2) dma_one(0, kt + 2, wd, ad, i);
            }
          } else if constexpr (kDma2) {
            dma_one(kt + STAGES, kt + STAGES, wd, ad, m);
          }
        }
      }
      interleave(jv);
    };
    using std::false_type;
    using std::true_type;
    auto kloop = [&](auto jv) {
      int kt = 0;
      if constexpr (kW3) {
        for (; kt + 3 < nk; ++kt) stage(kt, true_type{}, true_type{}, jv);
        for (; kt + 2 < nk; ++kt) stage(kt, true_type{}, false_type{}, jv);
      } else {
        for (; kt + STAGES < nk; ++kt) stage(kt, true_type{}, false_type{}, jv);
      }
      for (; kt < nk; ++kt) stage(kt, false_type{}, false_type{}, jv);
    };
    // wave-uniform: 32-token fragments of this wave that hold a token < M
    const int64_t jv = (e.M - mw + 31) / 32;
    if (jv > kFM / 2) kloop(kAllFrags);
    else if (jv > 0) kloop(integral_constant<int, kFM / 2>{});
    else kloop(integral_constant<int, 0>{});
    wait_vmcnt<0>();  // no DMA may still write LDS when the epilogue reuses it
  } else {
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
      if (s < nk) issue(s);
    for (int kt = 0; kt < nk; ++kt) {
      // Loads of stages kt+1 .. kt+STAGES-2 may stay in flight.
      if (kt + STAGES - 2 < nk) wait_vmcnt<(STAGES - 2) * kLoads>();
      else wait_vmcnt<0>();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1);
      compute(smem + (kt % STAGES) * kStage);
    }
  }

  if (part.base) {
    // Split-K: store this slice's raw accumulators; splitk_reduce applies the
    // epilogue. Through the same LDS transpose, 128 packed columns per row.
    asm volatile("" ::: "memory");
    __syncthreads();
    float* tile = reinterpret_cast<float*>(smem) + wave * 32 * kPitch;
    const int64_t nw = n0 + wn * (32 * kFN);
    const int64_t mw = m0 + wm * kWT;
    const int col = (lane & 31) * 4;  // packed column of the wave tile (32 * kFN of them)
#pragma unroll
    for (int j = 0; j < kFM; ++j) {
#pragma unroll
      for (int i = 0; i < kFN; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<v4f*>(tile + frow * kPitch + i * 32 + 8 * q + 4 * fhalf) = quad(acc[i][j], q);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (col < 32 * kFN && nw + col < e.N) {
#pragma unroll 4
        for (int r = lane >> 5; r < 32; r += 2) {
          const int64_t m = mw + j * 32 + r;
          if (m < e.M)
            *reinterpret_cast<float4*>(part.base + (split * e.M + m) * part.ld + nw + col) =
                *reinterpret_cast<const float4*>(tile + r * kPitch + col);
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    return;
  }
  // Epilogue through LDS, one 32-token fragment row at a time.
  // (1) Raw fp32 accumulators go to this wave's private [token][packed column]
  //     tile (row pitch padded by 16 bytes: the 16 rows written by 16 lanes
  //     land in distinct banks).
  // (2) Each lane owns four consecutive output columns of the tile: their
  //     scales, bias and adaLN gate are loaded once, the tile's token scales
  //     are staged in LDS, and a fragment row's residual loads are all issued
  //     before its math. Every output row is written as one contiguous segment.
  // The epilogue flags are resolved once per workgroup into a compile-time
  // mode (activation, gate, residual; bf16 residual and output), so the row
  // loop carries no per-element branches; other flag sets take the
  // runtime-flag loop.
  // The barrier keeps the stage buffers alive until every wave is done with
  // its MFMAs and publishes the token scales.
  if constexpr (kW3) {
    // s_sa overlays the ring: every wave must be done reading its last stage
    asm volatile("" ::: "memory");
    __syncthreads();
  }
  static_assert(kWaves * 64 >= BM, "one token scale per thread");
  if (tid < BM) s_sa[tid] = sa_pre;
  asm volatile("" ::: "memory");
  __syncthreads();
  const float swa[4] = {sw0.x, sw0.y, sw0.z, sw0.w}, ba[4] = {b0.x, b0.y, b0.z, b0.w};
  const float swu[4] = {sw1.x, sw1.y, sw1.z, sw1.w}, bu[4] = {b1.x, b1.y, b1.z, b1.w};
  const float gta[4] = {__uint_as_float(g2.x << 16), __uint_as_float(g2.x & 0xFFFF0000u),
                        __uint_as_float(g2.y << 16), __uint_as_float(g2.y & 0xFFFF0000u)};
  float* tile = reinterpret_cast<float*>(smem) + wave * 32 * kPitch;
  const int r0 = lane / kLanesPerRow;

  // Mode bits: 1 GELU-tanh (GeGLU for GLU), 2 SiLU (SwiGLU), 4 gate,
  // 8 residual, 16 runtime flags (f32 residual or output, any combination).
  // NT (compile time): bf16 output rows stored nontemporally (e.nt_out); a
  // runtime choice per store split every row into its own basic block and
  // kept the rows' address arithmetic from being shared.
  auto rows = [&](auto mode_tag, auto nt_tag) __attribute__((always_inline)) {
    constexpr int MD = decltype(mode_tag)::value;
    constexpr bool NT = decltype(nt_tag)::value;
    constexpr bool kRt = (MD & 16) != 0;
    const int fl = e.flags;
    const bool act_gelu = kRt ? (fl & (GLU ? IFX_EPI_GEGLU : IFX_EPI_GELU_TANH)) != 0 : (MD & 1) != 0;
    const bool act_silu = kRt ? (fl & IFX_EPI_SWIGLU) != 0 : (MD & 2) != 0;
    const bool has_gate = kRt ? (fl & IFX_EPI_GATE) != 0 : (MD & 4) != 0;
    const bool has_res = kRt ? (fl & IFX_EPI_RESIDUAL) != 0 : (MD & 8) != 0;
    // Compile-time residual modes load every residual row of the wave tile
    // (bf16 x 4 per row and lane) before the first output store and wait for
    // them once. Vector-memory loads and stores share one completion counter,
    // so a residual load consumed after a store would wait for that store.
    // (4-wave 128 x 128 wave tiles only: their accumulators sit in AccVGPRs,
    // leaving the VGPRs of the K loop's fragments free for the residuals.)
    constexpr bool kPre = !kRt && (MD & 8) != 0 && kFM == 4;
    uint2 resv[kPre ? kFM : 1][kPre ? kRowIters : 1];
    if constexpr (kPre) {
      const uint16_t* rp = static_cast<const uint16_t*>(e.res) + (col_ok ? c_out : 0);
#pragma unroll
      for (int j = 0; j < kFM; ++j)
#pragma unroll
        for (int t = 0; t < kRowIters; ++t) {
          const int64_t m = min(mw + j * 32 + r0 + t * kRowsPerPass, e.M - 1);
          resv[j][t] = ld8_nt(rp + m * e.ldr);
        }
    }
#pragma unroll
    for (int j = 0; j < kFM; ++j) {
#pragma unroll
      for (int i = 0; i < kFN; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<v4f*>(tile + frow * kPitch + i * 32 + 8 * q + 4 * fhalf) = quad(acc[i][j], q);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if constexpr (kPre) {
        if (j == 0) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): every residual row has landed
      }
      const int64_t mrow = mw + j * 32 + r0;         // token of pass 0
      const int64_t left = e.M - (mw + j * 32);      // rows of this fragment row inside M
      // Rows that load their residuals here do so kResBatch rows at a time,
      // ahead of their math. The other modes walk all rows as one batch, with
      // no loop: the compiler waits for every outstanding
      // vector-memory operation (the previous fragment row's stores included)
      // at the entry of a loop that stores, which left each fragment row's
      // store latency exposed (8192x14336x3072 GELU 312 -> 302 us).
      constexpr bool kRowLoads = kRt || ((MD & 8) != 0 && !kPre);
      constexpr int kResBatch = !kRowLoads ? kRowIters : kRowIters < 8 ? kRowIters : 8;
      // A fragment row wholly inside M runs without per-row guards, so the
      // compiler can interleave the rows' arithmetic.
      auto emit = [&](auto full_tag) __attribute__((always_inline)) {
        constexpr bool kFull = decltype(full_tag)::value;
        uint16_t* orow = static_cast<uint16_t*>(e.out) + mrow * e.ldo + c_out;
        // one batch of rows at a time keeps the accumulator-holding 4-wave
        // kernel within its registers
#pragma unroll 1
        for (int t0 = 0; t0 < kRowIters; t0 += kResBatch) {
        float4 res[kResBatch];
#pragma unroll
        for (int tb = 0; tb < kResBatch; ++tb) {
          const int t = t0 + tb;
          const int r = r0 + t * kRowsPerPass;
          if constexpr (kRt) {
            res[tb] = (has_res && (kFull || r < left)) ? load_res4(e, mrow + t * kRowsPerPass, c_out)
                                            : make_float4(0.f, 0.f, 0.f, 0.f);
          } else if constexpr ((MD & 8) != 0) {
            uint2 rv;
            if constexpr (kPre) {
              rv = resv[j][t];
            } else {
              const uint16_t* rp = static_cast<const uint16_t*>(e.res) + c_out;
              rv = *reinterpret_cast<const uint2*>(rp + min(mrow + t * kRowsPerPass, e.M - 1) * e.ldr);
            }
            res[tb] = make_float4(__uint_as_float(rv.x << 16), __uint_as_float(rv.x & 0xFFFF0000u),
                                 __uint_as_float(rv.y << 16), __uint_as_float(rv.y & 0xFFFF0000u));
          }
        }
#pragma unroll
        for (int tb = 0; tb < kResBatch; ++tb) {
          const int t = t0 + tb;
          const int r = r0 + t * kRowsPerPass;
          if (kFull || r < left) {
            const float sa = s_sa[wm * kWT + j * 32 + r];
            const float4 v = *reinterpret_cast<const float4*>(tile + r * kPitch + pc);
            const float va[4] = {v.x, v.y, v.z, v.w};
            float y[4];
            if constexpr (GLU) {
              const float4 w = *reinterpret_cast<const float4*>(tile + r * kPitch + pc + 16);
              const float wa[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
              for (int u = 0; u < 4; ++u) {
                const float gv = va[u] * sa * swa[u] + ba[u];
                const float uv = wa[u] * sa * swu[u] + bu[u];
                y[u] = (act_silu ? silu(gv) : gelu_tanh(gv)) * uv;
              }
            } else {
#pragma unroll
              for (int u = 0; u < 4; ++u) {
                y[u] = va[u] * sa * swa[u] + ba[u];
                if (act_gelu) y[u] = gelu_tanh(y[u]);
              }
            }
            if (has_gate) {
#pragma unroll
              for (int u = 0; u < 4; ++u) y[u] = mul_rn(y[u], gta[u]);
            }
            if (has_res) {
              y[0] = res[tb].x + y[0];
              y[1] = res[tb].y + y[1];
              y[2] = res[tb].z + y[2];
              y[3] = res[tb].w + y[3];
            }
            {
              if constexpr (kRt) {
                epi_store4(e, mrow + t * kRowsPerPass, c_out, y);
              } else {
                uint2 o;
                o.x = pack_bf16x2(y[0], y[1]);
                o.y = pack_bf16x2(y[2], y[3]);
                uint16_t* op = orow + static_cast<int64_t>(t * kRowsPerPass) * e.ldo;
                if constexpr (NT) st8_nt(op, o);
                else *reinterpret_cast<uint2*>(op) = o;
              }
            }
          }
        }
        }
      };
      if (col_ok) {
        if (left >= 32) emit(std::true_type{});
        else emit(std::false_type{});
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
  };
  const int fl = e.flags;
  const bool plain_io = !(fl & (IFX_EPI_OUT_F32 | IFX_EPI_OUT_F16 | IFX_EPI_RES_F32));
  const int gr = ((fl & IFX_EPI_GATE) ? 4 : 0) | ((fl & IFX_EPI_RESIDUAL) ? 8 : 0);
  using std::integral_constant;
  auto run = [&](auto md) __attribute__((always_inline)) {
    if constexpr (decltype(md)::value == 16) {
      rows(md, std::false_type{});
    } else {
      if (e.nt_out) rows(md, std::true_type{});
      else rows(md, std::false_type{});
    }
  };
  if constexpr (GLU) {
    if (plain_io && gr == 0) {
      if (fl & IFX_EPI_SWIGLU) run(integral_constant<int, 2>{});
      else run(integral_constant<int, 1>{});
    } else {
      run(integral_constant<int, 16>{});
    }
  } else {
    const bool gl = (fl & IFX_EPI_GELU_TANH) != 0;
    if (!plain_io) run(integral_constant<int, 16>{});
    else if (gl && gr == 0) run(integral_constant<int, 1>{});
    else if (gl) run(integral_constant<int, 16>{});
    else if (gr == 0) run(integral_constant<int, 0>{});
    else if (gr == 8) run(integral_constant<int, 8>{});
    else if (gr == 12) run(integral_constant<int, 12>{});
    else run(integral_constant<int, 16>{});
  }
}

// Split-K finish: sums the K slices' partial accumulators in slice order
// (deterministic) and applies the full epilogue. One thread per four output
// columns of one token.
template <bool GLU>
__global__ __launch_bounds__(256) void splitk_reduce(Partials part, int ksplit, Epi e) {
  const int64_t n_out = GLU ? e.N / 2 : e.N;
  const int64_t groups = n_out / 4;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= e.M * groups) return;
  const int64_t m = idx / groups;
  const int64_t c = (idx - m * groups) * 4;                 // output column
  const int64_t ng = GLU ? (c >> 4) * 32 + (c & 15) : c;   // packed row of its (gate) group
  v4f a = v4f{0.f, 0.f, 0.f, 0.f}, u = a;
  const float* p0 = part.base + m * part.ld + ng;
  const int64_t slice = e.M * part.ld;
  int s = 0;
  // four slices' loads in flight at a time, added in slice order
  for (; s + 4 <= ksplit; s += 4) {
    v4f pa[4], pu[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      pa[q] = *reinterpret_cast<const v4f*>(p0 + (s + q) * slice);
      if constexpr (GLU) pu[q] = *reinterpret_cast<const v4f*>(p0 + (s + q) * slice + 16);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a += pa[q];
      if constexpr (GLU) u += pu[q];
    }
  }
  for (; s < ksplit; ++s) {
    a += *reinterpret_cast<const v4f*>(p0 + s * slice);
    if constexpr (GLU) u += *reinterpret_cast<const v4f*>(p0 + s * slice + 16);
  }
  float y[4];
  if constexpr (GLU) epi_pre_glu(e, a, u, ng, m, y);
  else epi_pre(e, a, ng, m, y);
  epi_finish4(e, m, c, y);
}

// ---------------------------------------------------------------------------
// Skinny kernel (M <= 64): weight streaming
// ---------------------------------------------------------------------------
//
// A workgroup owns a group of 16 weight rows (32 for GLU: a gate block and
// its up block) and the whole of K. Inside it the WAVES waves split the K
// steps (wave w takes steps w, w+WAVES, ...), each loading kSkUnroll steps of
// weight fragments (nontemporal: read once per call) and token fragments
// before issuing their MFMAs; partial sums are added in LDS in wave order.
// Shapes with few row groups spread over more CUs by token blocks (tsplit) or
// row halves (rhalves), never by splitting K: a K split needs a device-wide
// handoff of partial sums between workgroups, and its agent-scope
// release/acquire (a write-back and an invalidation of the XCD's L2) costs
// more than the split wins. Measured on MI355X with weights streamed from HBM,
// two K slices with an acquire-release ticket against one workgroup per group:
// 16x512x8192 8.9 / 7.6 us, 1x1024x16384 16.7 / 9.7, 8x2048x8192 19.4 / 7.8,
// 16x1536x6144 15.2 / 7.1; three and four slices lose more.

constexpr int kSkUnroll = 4;       // K steps whose loads are issued together per wave
constexpr int kSkMaxGroups = 256;  // row groups up to which a group may take two workgroups (row halves)

// The qkv_split epilogue of ifx_fp8_linear_qkv_rope (flag kEpiRopeQkv): the
// fused q|k|v weight rows are permuted per head so that packed rows
// 16k + 4g + {0, 1, 2, 3} hold head dims d, d + 1, d + HD/2, d + 1 + HD/2
// with d = 8k + 2g; the lane that owns those four outputs of a token applies
// the rotary pairs (d, d + HD/2) and (d + 1, d + 1 + HD/2) itself.
constexpr int kEpiRopeQkv = 1 << 20;  // internal flag, never accepted from callers

struct RopeQkv {
  const float* pos;       // position of token m at pos[m * ldpos]
  int64_t ldpos;
  const float* inv_freq;  // [HD/2] or null (no rotation)
  int64_t hq, hkv, hd;
  void* q;                // Q at q[m*sq_t + h*sq_h + d]
  int64_t sq_t, sq_h;
  void* k;                // K at k[(kv_base + m)*sk_t + h*sk_h + d]
  int64_t sk_t, sk_h;
  void* v;                // V likewise
  int64_t sv_t, sv_h;
  int64_t kv_base;
  const int32_t* kv_base_dev;  // device kv_base, or null
  int out_dtype;               // IFX_DTYPE_F16 / BF16 / F32
};

__device__ __forceinline__ void store_elem(int dtype, void* base, int64_t i, float v) {
  if (dtype == IFX_DTYPE_F32) static_cast<float*>(base)[i] = v;
  else if (dtype == IFX_DTYPE_F16) static_cast<_Float16*>(base)[i] = static_cast<_Float16>(v);
  else static_cast<__bf16*>(base)[i] = static_cast<__bf16>(v);
}

// y = the four outputs of token m at packed columns p .. p + 3 (p % 4 == 0).
__device__ __forceinline__ void rope_qkv_store(const RopeQkv& r, int64_t m, int64_t p, const float* y) {
  const int64_t head = p / r.hd, pq = p - head * r.hd, half = r.hd / 2;
  const int64_t d = 8 * (pq / 16) + 2 * ((pq % 16) / 4);
  float lo0 = y[0], lo1 = y[1], hi0 = y[2], hi1 = y[3];
  if (r.inv_freq && head < r.hq + r.hkv) {  // Q and K heads rotate
    const float ps = r.pos[m * r.ldpos];
    float s0, c0, s1, c1;
    sincosf(ps * r.inv_freq[d], &s0, &c0);
    sincosf(ps * r.inv_freq[d + 1], &s1, &c1);
    rotate_pair(lo0, hi0, c0, s0);
    rotate_pair(lo1, hi1, c1, s1);
  }
  void* dst;
  int64_t off;
  if (head < r.hq) {
    dst = r.q;
    off = m * r.sq_t + head * r.sq_h;
  } else {
    const int64_t krow = (r.kv_base_dev ? static_cast<int64_t>(*r.kv_base_dev) : r.kv_base) + m;
    if (head < r.hq + r.hkv) {
      dst = r.k;
      off = krow * r.sk_t + (head - r.hq) * r.sk_h;
    } else {
      dst = r.v;
      off = krow * r.sv_t + (head - r.hq - r.hkv) * r.sv_h;
    }
  }
  store_elem(r.out_dtype, dst, off + d, lo0);
  store_elem(r.out_dtype, dst, off + d + 1, lo1);
  store_elem(r.out_dtype, dst, off + half + d, hi0);
  store_elem(r.out_dtype, dst, off + half + d + 1, hi1);
}

struct SkArgs {
  RopeQkv rope;    // the qkv_split epilogue's arguments (flag kEpiRopeQkv)
};

struct SkinnyPlan {
  int mb;          // 16-token blocks per workgroup (1..4)
  int nbw;         // 16-row weight blocks per workgroup (1, or 2 for GLU)
  int64_t groups;  // row groups
  int waves;       // waves per workgroup (4, 8 or 16)
  int tsplit;      // workgroups along the tokens per group (each owns mb blocks)
  int rhalves;     // workgroups along the group's 16 weight rows (2: 8 rows each)
};

__host__ inline SkinnyPlan skinny_plan(int64_t M, int64_t N, int64_t K, bool glu) {
  SkinnyPlan p{};
  p.mb = static_cast<int>((M + 15) / 16);
  p.nbw = glu ? 2 : 1;
  p.groups = N / (16 * p.nbw);
  const int64_t ksteps = (K + kBK - 1) / kBK;
  // One token block per workgroup (grid.y over the blocks) when the row groups
  // alone leave CUs idle: the extra reads of each weight fragment hit L2, and
  // each workgroup's MFMA and load chain gets 1/mb as long. Measured (M = 50,
  // weights streamed from HBM): 50x1024x4096 10.9 -> 5.8 us, 50x2560x1024
  // 6.4 -> 4.9 us; GLU weights (32-row groups) and 256 or more groups lose or
  // break even (50x8192x1024 GeGLU 7.6 -> 9.1 us; 50x4096x1024 with its
  // weights L2/MALL-resident 4.7 -> 4.9 us, streamed from HBM 6.5 -> 5.6 us).
  p.tsplit = 1;
  if (p.mb > 1 && p.nbw == 1 && p.groups < 256) {
    p.tsplit = p.mb;
    p.mb = 1;
  }
  // GLU weights with four token blocks: two workgroups of two blocks each
  // (50x8192x1024 GeGLU 7.5 -> 6.5 us; one block each is slower, and so is
  // splitting two blocks: 32x8192x2048 SwiGLU 7.5 -> 7.7 us).
  if (p.nbw == 2 && p.mb == 4 && p.groups <= 256) {
    p.tsplit = 2;
    p.mb = 2;
  }
  // Too few row groups to reach every CU (one 16-token block): two
  // workgroups per group, each streaming 8 of its 16 weight rows (the other 8
  // MFMA rows are zeros and their outputs are not stored). The matrix cores
  // are idle here anyway; the weight stream spreads over twice the CUs.
  p.rhalves = 1;
  if (p.mb == 1 && p.tsplit == 1 && p.nbw == 1 && p.groups * 2 <= kSkMaxGroups) p.rhalves = 2;
  // Enough waves that every wave has at most kSkUnroll K steps
  // (one batch of loads in flight); 16 waves leave 128 VGPRs each, enough
  // for one 16 x 16 block only.
  int w = 4;
  const int wmax = p.nbw * p.mb == 1 ? 16 : 8;
  while (w < wmax && ksteps > static_cast<int64_t>(w) * kSkUnroll && 2 * w * p.nbw * p.mb <= 32) w *= 2;
  p.waves = w;
  return p;
}

// TILED: w is in the layout of ifx_fp8_pack_skinny (2 KB tile per 16-row block
// and 128-byte K step, zero-padded in K), so each weight load instruction of a
// wave reads 1 KB of contiguous memory.
template <int MB, int NBW, int WAVES, bool TILED, int RH = 1>
__global__ __launch_bounds__(WAVES * 64) void gemm_skinny(const uint8_t* __restrict__ A, int64_t lda,
                                                          const uint8_t* __restrict__ W, int64_t ldw,
                                                          int64_t K, Epi e, SkArgs sp) {
  __shared__ v4f red[WAVES][NBW][MB][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // RH > 1: RH workgroups split the group's 16 weight rows (16 / RH each)
  const int rh = RH == 1 ? 0 : static_cast<int>(blockIdx.x % RH);
  const int64_t grp = static_cast<int64_t>(blockIdx.x) / RH;  // row group
  const int64_t nrow0 = grp * (16 * NBW);
  const int frow = lane & 15;
  const int g = lane >> 4;
  // this lane's weight row is streamed here / its output rows are stored here
  const bool wmine = RH == 1 || frow / (16 / RH) == rh;
  const bool omine = RH == 1 || (4 * g) / (16 / RH) == rh;
  const int64_t ksteps = (K + kBK - 1) / kBK;
  const int64_t s_end = ksteps;
  const bool a_tiled = (e.flags & IFX_EPI_A_TILED) != 0;  // A in the skinny tile layout (lda unused)
  const int64_t mb0 = static_cast<int64_t>(blockIdx.y) * MB;  // first 16-token block of this workgroup

  const uint8_t* wrow[NBW];
#pragma unroll
  for (int b = 0; b < NBW; ++b) wrow[b] = W + (nrow0 + b * 16 + frow) * ldw + g * 32;
  const uint8_t* arow[MB];
#pragma unroll
  for (int j = 0; j < MB; ++j) {
    int64_t m = (mb0 + j) * 16 + frow;
    m = m < e.M ? m : e.M - 1;  // rows past M are computed, never stored
    arow[j] = A + m * lda + g * 32;
  }

  // Epilogue operands of the lanes that will finish token block j = wave,
  // fetched now so their latency hides under the weight stream.
  const int64_t m_epi = wave < MB ? (mb0 + wave) * 16 + frow : e.M;
  const int64_t mc = min(m_epi, e.M - 1);
  const int64_t c_epi = NBW == 2 ? (nrow0 >> 5) * 16 + 4 * g : nrow0 + 4 * g;  // output column
  float sa_epi = 1.0f, sw_epi[NBW][4], b_epi[NBW][4], gate_epi[4] = {1.f, 1.f, 1.f, 1.f}, res_epi[4] = {0.f, 0.f, 0.f, 0.f};
  if (wave < MB) {
    sa_epi = epi_sa(e, mc);
    const float* bp = (e.flags & IFX_EPI_BIAS) ? e.bias : nullptr;
#pragma unroll
    for (int b = 0; b < NBW; ++b) {
      const float4 w4 = epi_sw4(e, nrow0 + b * 16 + 4 * g);
      const float4 b4 = load_f4_or(bp, nrow0 + b * 16 + 4 * g, 0.0f);
      sw_epi[b][0] = w4.x; sw_epi[b][1] = w4.y; sw_epi[b][2] = w4.z; sw_epi[b][3] = w4.w;
      b_epi[b][0] = b4.x; b_epi[b][1] = b4.y; b_epi[b][2] = b4.z; b_epi[b][3] = b4.w;
    }
    if (e.flags & IFX_EPI_GATE) {
      const uint2 g2 = *reinterpret_cast<const uint2*>(e.gate + c_epi);
      gate_epi[0] = __uint_as_float(g2.x << 16); gate_epi[1] = __uint_as_float(g2.x & 0xFFFF0000u);
      gate_epi[2] = __uint_as_float(g2.y << 16); gate_epi[3] = __uint_as_float(g2.y & 0xFFFF0000u);
    }
    if (e.flags & IFX_EPI_RESIDUAL) {
      const float4 r4 = load_res4(e, mc, c_epi);
      res_epi[0] = r4.x; res_epi[1] = r4.y; res_epi[2] = r4.z; res_epi[3] = r4.w;
    }
  }

  v4f acc[NBW][MB];
#pragma unroll
  for (int b = 0; b < NBW; ++b)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[b][j] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int64_t s0 = wave; s0 < s_end; s0 += WAVES * kSkUnroll) {
    v8i wf[kSkUnroll][NBW];
    v8i af[kSkUnroll][MB];
#pragma unroll
    for (int u = 0; u < kSkUnroll; ++u) {
      const int64_t s = s0 + u * WAVES;
      const int64_t k0 = s * kBK + g * 32;
      const bool lo = s < s_end && k0 < K;  // K % 16 == 0: a 16-byte half is all in or all out
      const bool hi = s < s_end && k0 + 16 < K;
#pragma unroll
      for (int b = 0; b < NBW; ++b) {
        if constexpr (TILED) {
          const bool in = s < s_end && wmine;
          const uint8_t* p = W + ((grp * NBW + b) * ksteps + s) * 2048 + lane * 16;
          wf[u][b] = cat8(in ? ld16_nt(p) : v4i{0, 0, 0, 0}, in ? ld16_nt(p + 1024) : v4i{0, 0, 0, 0});
        } else {
          const uint8_t* p = wrow[b] + s * kBK;
          wf[u][b] = cat8(lo && wmine ? ld16_nt(p) : v4i{0, 0, 0, 0}, hi && wmine ? ld16_nt(p + 16) : v4i{0, 0, 0, 0});
        }
      }
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        const uint8_t* p = arow[j] + s * kBK;
        if (a_tiled) {  // workgroup-uniform
          const bool in = s < s_end;
          const uint8_t* t = A + ((mb0 + j) * ksteps + s) * 2048 + lane * 16;
          af[u][j] = cat8(in ? ld16(t) : v4i{0, 0, 0, 0}, in ? ld16(t + 1024) : v4i{0, 0, 0, 0});
        } else {
          af[u][j] = cat8(lo ? ld16(p) : v4i{0, 0, 0, 0}, hi ? ld16(p + 16) : v4i{0, 0, 0, 0});
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kSkUnroll; ++u)
#pragma unroll
      for (int b = 0; b < NBW; ++b)
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[b][j] = mfma16(wf[u][b], af[u][j], acc[b][j]);
  }

  // Cross-wave reduction in LDS, fixed order (wave 0, 1, ...): deterministic.
#pragma unroll
  for (int b = 0; b < NBW; ++b)
#pragma unroll
    for (int j = 0; j < MB; ++j) red[wave][b][j][lane] = acc[b][j];
  __syncthreads();
  // wave w finishes token block j = w (for w < MB)
  const int j = wave;
  v4f sum[NBW];
  if (wave < MB) {
#pragma unroll
    for (int b = 0; b < NBW; ++b) {
      sum[b] = red[0][b][j][lane];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) sum[b] += red[w][b][j][lane];
    }
  }

  if (wave < MB && m_epi < e.M && omine) {
    float y[4];
    if constexpr (NBW == 2) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float gv = sum[0][r] * sa_epi * sw_epi[0][r] + b_epi[0][r];
        const float uv = sum[1][r] * sa_epi * sw_epi[1][r] + b_epi[1][r];
        y[r] = ((e.flags & IFX_EPI_SWIGLU) ? silu(gv) : gelu_tanh(gv)) * uv;
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        y[r] = sum[0][r] * sa_epi * sw_epi[0][r] + b_epi[0][r];
        if (e.flags & IFX_EPI_GELU_TANH) y[r] = gelu_tanh(y[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (e.flags & IFX_EPI_GATE) y[r] = mul_rn(y[r], gate_epi[r]);
      if (e.flags & IFX_EPI_RESIDUAL) y[r] = res_epi[r] + y[r];
    }
    if (NBW == 1 && (e.flags & kEpiRopeQkv)) rope_qkv_store(sp.rope, m_epi, c_epi, y);
    else epi_store4(e, m_epi, c_epi, y);
  }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------

template <int BN, int BM, int WGN, int WGM, bool GLU>
int launch_lds(const uint8_t* a, int64_t lda, const uint8_t* w, int64_t ldw, int64_t K, const Epi& e,
               hipStream_t st) {
  const int64_t tiles_m = (e.M + BM - 1) / BM;
  const int64_t tiles_n = (e.N + BN - 1) / BN;
  const int64_t grid = tiles_m * tiles_n;
  if (grid > 0x7FFFFFFFLL) return IFX_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((gemm_lds<BN, BM, WGN, WGM, GLU>), dim3(static_cast<unsigned>(grid)),
                     dim3(WGN * WGM * 64), 0, st, a, lda, w, ldw, K, static_cast<int>(tiles_m), e);
  return launch_status();
}

// Large-M launch plan: tiles and, when there are too few tiles to fill the
// GPU, a K split (each slice at least 4 stages) finished by splitk_reduce.
struct BigPlan {
  int64_t tiles_m, tiles_n;
  int ksplit;
  int64_t kstages;  // K stages per slice
  size_t ws_bytes;  // fp32 partials of all slices
};

__host__ inline BigPlan big_plan(int64_t M, int64_t N, int64_t K, int bm, int bn, int kb) {
  BigPlan p{};
  p.tiles_m = (M + bm - 1) / bm;
  p.tiles_n = (N + bn - 1) / bn;
  const int64_t tiles = p.tiles_m * p.tiles_n;
  const int64_t nk = K / kb;
  int64_t s = 1;
  if (tiles < 192) {
    // As many slices as keep the grid within one workgroup per CU: a grid of
    // 1-2 workgroups per CU leaves the CUs that get two the critical path
    // (measured: 816x2048x16384 51 vs 57 us at 224 vs 336 workgroups;
    // 1024x2048x11008 44 vs 51 us at 256 vs 320).
    s = 256 / tiles;
    if (s > nk / 4) s = nk / 4;
    if (s < 1) s = 1;
  }
  p.kstages = (nk + s - 1) / s;
  p.ksplit = static_cast<int>((nk + p.kstages - 1) / p.kstages);
  p.ws_bytes = p.ksplit > 1 ? static_cast<size_t>(p.ksplit) * M * N * sizeof(float) : 0;
  return p;
}

template <int BM, int BN, int KB, int STAGES, int OCC, bool GLU, int FM = 2>
int launch_big(const uint8_t* a, int64_t lda, const uint8_t* w, int64_t ldw, int64_t K, const Epi& e,
               void* ws, size_t ws_bytes, hipStream_t st) {
  const BigPlan p = big_plan(e.M, e.N, K, BM, BN, KB);
  if (p.tiles_m * p.tiles_n * p.ksplit > 0x7FFFFFF0LL) return IFX_ERR_UNSUPPORTED;
  Partials part{nullptr, e.N, p.kstages};
  if (p.ksplit > 1) {
    if (!ws || ws_bytes < p.ws_bytes || !aligned16(ws)) return IFX_ERR_WORKSPACE;
    part.base = static_cast<float*>(ws);
  }
  const TileMap t = make_tile_map(p.tiles_m, p.tiles_n, p.ksplit);
  hipLaunchKernelGGL((gemm_big<BM, BN, KB, STAGES, OCC, GLU, FM>), dim3(static_cast<unsigned>(8 * t.per_xcd)), dim3(4 * BM / FM),
                     0, st, a, lda, w, ldw, K, t, e, part);
  if (p.ksplit > 1) {
    const int64_t threads = e.M * ((GLU ? e.N / 2 : e.N) / 4);
    hipLaunchKernelGGL((splitk_reduce<GLU>), dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, st,
                       part, p.ksplit, e);
  }
  return launch_status();
}

template <int MB, int NBW, int WAVES>
void launch_skinny_w(const SkinnyPlan& p, const uint8_t* a, int64_t lda, const uint8_t* w, int64_t ldw, int64_t K,
                     const Epi& e, const SkArgs& sp, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(p.groups * p.rhalves), static_cast<unsigned>(p.tsplit)),
      block(WAVES * 64);
  if constexpr (MB == 1 && NBW == 1) {
    if (p.rhalves == 2) {
      if (e.flags & IFX_EPI_W_TILED)
        hipLaunchKernelGGL((gemm_skinny<MB, NBW, WAVES, true, 2>), grid, block, 0, st, a, lda, w, ldw, K, e, sp);
      else
        hipLaunchKernelGGL((gemm_skinny<MB, NBW, WAVES, false, 2>), grid, block, 0, st, a, lda, w, ldw, K, e, sp);
      return;
    }
  }
  if (e.flags & IFX_EPI_W_TILED)
    hipLaunchKernelGGL((gemm_skinny<MB, NBW, WAVES, true>), grid, block, 0, st, a, lda, w, ldw, K, e, sp);
  else
    hipLaunchKernelGGL((gemm_skinny<MB, NBW, WAVES, false>), grid, block, 0, st, a, lda, w, ldw, K, e, sp);
}

template <int MB, int NBW>
void launch_skinny_mb(const SkinnyPlan& p, const uint8_t* a, int64_t lda, const uint8_t* w, int64_t ldw, int64_t K,
                      const Epi& e, const SkArgs& sp, hipStream_t st) {
  // 16 waves (128 VGPRs each) only for one 16 x 16 output block per workgroup:
  // more blocks' fragments do not fit without spilling
  if constexpr (NBW * MB == 1) {
    if (p.waves >= 16) {
      launch_skinny_w<MB, NBW, 16>(p, a, lda, w, ldw, K, e, sp, st);
      return;
    }
  }
  if constexpr (8 * NBW * MB <= 32) {
    if (p.waves >= 8) {
      launch_skinny_w<MB, NBW, 8>(p, a, lda, w, ldw, K, e, sp, st);
      return;
    }
  }
  launch_skinny_w<MB, NBW, 4>(p, a, lda, w, ldw, K, e, sp, st);
}

template <int NBW>
int launch_skinny(const SkinnyPlan& p, const uint8_t* a, int64_t lda, const uint8_t* w, int64_t ldw, int64_t K,
                  const Epi& e, hipStream_t st, const RopeQkv* rope = nullptr) {
  const SkArgs sp{rope ? *rope : RopeQkv{}};
  switch (p.mb) {
    case 1: launch_skinny_mb<1, NBW>(p, a, lda, w, ldw, K, e, sp, st); break;
    case 2: launch_skinny_mb<2, NBW>(p, a, lda, w, ldw, K, e, sp, st); break;
    case 3: launch_skinny_mb<3, NBW>(p, a, lda, w, ldw, K, e, sp, st); break;
    default: launch_skinny_mb<4, NBW>(p, a, lda, w, ldw, K, e, sp, st); break;
  }
  return launch_status();
}

constexpr int64_t kSkinnyMaxM = 64;

// One thread per 16-byte chunk of the tiled layout: chunk c = ((b * ks + s) *
// 2 + half) * 64 + l holds row 16b + l%16, K bytes s*128 + 32*(l/16) + 16*half
// + 0..15 (zero past K).
__global__ __launch_bounds__(256) void pack_skinny_kernel(const uint8_t* __restrict__ w, int64_t ldw, int64_t K,
                                                          int64_t ks, int64_t chunks, uint8_t* __restrict__ out) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (c >= chunks) return;
  const int l = static_cast<int>(c & 63);
  const int half = static_cast<int>((c >> 6) & 1);
  const int64_t bs = c >> 7;  // b * ks + s
  const int64_t b = bs / ks, st = bs - b * ks;
  const int64_t row = b * 16 + (l & 15);
  const int64_t k = st * kBK + 32 * (l >> 4) + 16 * half;
  v4i v{0, 0, 0, 0};
  if (k < K) v = *reinterpret_cast<const v4i*>(w + row * ldw + k);
  *reinterpret_cast<v4i*>(out + c * 16) = v;
}

// Large-M configurations (all with 128-byte K stages, so K % 128 == 0): see
// pick_big below.
constexpr int kBigKB = 128;

// Every M past the skinny range (M > 64) with K % 128 == 0 takes gemm_big; its
// small-grid configurations beat gemm_lds there by 3-5x (65x2048x2048 8.8 vs
// 33 us, 128x4096x8192 22.5 vs 97 us), so gemm_lds only serves K % 128 != 0.
inline bool big_path(int64_t M, int64_t K) { return M > kSkinnyMaxM && K % kBigKB == 0; }

// Large-M configuration for a shape:
//  * kWide / kWide192: 256 tokens x 256 (or 192) weight rows per workgroup, one
//    workgroup per CU. 256 x 256 tiles run the 4-wave register-pipelined form
//    (C5 up 8192x14336x3072 GELU 341 -> 317 us, C5 qkv 247 -> 224 us, C3 gate|up
//    73 -> 69 us against 8 waves of 128 x 64), or 8 waves when an operand
//    spans 4 GiB or more (32-bit DMA offsets); 256 x 192 tiles likewise. 192-row tiles are taken when they need
//    fewer tile rounds on the 256 CUs, weighted by tile height and efficiency:
//    e.g. an 8192 x 3072 output is 384 tiles of 256 rows (a half-empty second
//    round) but 512 tiles of 192 rows (two full rounds): 329 -> 302 us for
//    K = 14336; a GLU output of 1024 x 22016 is 344 tiles of 256 but 460 of 192.
//  * kSmall: fewer than 192 tiles of 256 x 256 and K <= 4096 -- 64 tokens x
//    128 weight rows, 128-byte stages, 4 waves of 64 x 32 (short MFMA chains
//    per wave: the loop is latency-bound at these sizes), a 3-stage ring, two
//    workgroups per CU, usually no split (1024 x 2560 x 2048: 28 us with split-K
//    narrow tiles, 15.7 us with 2 waves of 64 x 64 and 64-byte stages, 12.1 us
//    with a 2-stage ring; weights streamed from HBM with bias and residual,
//    2 -> 3 stages: 1024 x 2560 18.2 -> 15.5 us, 1024 x 2048 15.5 -> 12.3 us);
//  * kSmall32: as kSmall with 32-token tiles (2 waves of 64 x 32) when 64-token
//    tiles would give fewer than 256 workgroups (200 x 2560 x 2048 10.7 -> 8.8 us,
//    512 x 1024 x 2048 12.4 -> 10.6 us; at 256 or more the 64-token tiles win:
//    1024 x 2560 x 2048 12.2 against 15.2 us). A 4-stage ring when the grid fits
//    one workgroup per CU, else 3 stages and two per CU (streamed weights: 200 x
//    2560 x 2048 16.2 -> 10.5 us, 300 x 3072 x 3072 23.0 -> 14.4 us, 816 x 2048 x
//    2048 16.7 -> 14.0 us against 2 stages);
//  * kNarrow: fewer than 192 tiles and a longer K -- 128 tokens x 256 weight
//    rows, the register-pipelined 4 waves of 64 x 128 with a 3-stage ring
//    (144 KB) when the 32-bit DMA offsets fit (else 8 waves of 128 x 32, two
//    stages), 128-byte stages, plus split K. 816 x 2048 x 16384: 44.1 us with 8
//    waves, 42.8 pipelined with two stages, 41.0 with three; with the weights
//    streamed from HBM 52.0 -> 42.4 us (two -> three stages), 1024 x 2048 x 11008
//    44.2 -> 39.3 us. (44 us with 4 waves of 128 x 64 and 64-byte stages; the
//    64 x 128 / 32 x 128 tiles without a split, re-measured on the current
//    kernels: 1024 x 2048 x 11008 44.3 against 40.2 us, 816 x 2048 x 16384 56-60
//    against 43-45 us.)
enum class BigCfg { kWide, kWide192, kSmall, kSmall32, kNarrow };

inline BigCfg pick_big(int64_t M, int64_t N, int64_t K, bool glu) {
  const int64_t tm = (M + 255) / 256;
  const int64_t t256 = tm * ((N + 255) / 256);
  if (t256 < 192) {
    if (K > 4096) return BigCfg::kNarrow;
    return ((M + 63) / 64) * ((N + 127) / 128) < 256 ? BigCfg::kSmall32 : BigCfg::kSmall;
  }
  (void)glu;  // GLU tiles take the same shapes (16-row gate|up blocks divide 192)
  {
    const int64_t t192 = tm * ((N + 191) / 192);
    // a 192-row tile does ~15% less work per unit time than a 256-row one
    // (measured: 8192x9216x3072, 6 full rounds of 192 vs 4.5 of 256, is 2.5% slower)
    if (((t192 + 255) / 256) * 192 * 115 < ((t256 + 255) / 256) * 256 * 100) return BigCfg::kWide192;
  }
  return BigCfg::kWide;
}

// The 4-wave kernel forms DMA addresses as a 32-bit byte offset (row * ld, a
// 24-bit multiply) from a wave-uniform base: both operands must span < 4 GiB
// with rows and row strides below 2^24.
inline bool dma32_ok(int64_t M, int64_t N, int64_t lda, int64_t ldw) {
  constexpr int64_t k24 = int64_t(1) << 24, k32 = int64_t(1) << 32;
  return M < k24 && N < k24 && lda < k24 && ldw < k24 && M * lda < k32 && N * ldw < k32;
}

template <bool GLU>
int launch_large(const uint8_t* a, int64_t lda, const uint8_t* w, int64_t ldw, int64_t K, const Epi& e, void* ws,
                 size_t ws_bytes, hipStream_t st) {
  switch (pick_big(e.M, e.N, K, GLU)) {
    case BigCfg::kWide192:
      if (dma32_ok(e.M, e.N, lda, ldw))
        return launch_big<256, 192, 128, 2, 1, GLU, 4>(a, lda, w, ldw, K, e, ws, ws_bytes, st);
      if constexpr (!GLU) return launch_big<256, 192, 128, 2, 1, GLU>(a, lda, w, ldw, K, e, ws, ws_bytes, st);
      [[fallthrough]];  // operands past 4 GiB with GLU: 8 waves of 256 x 256 (no split at this size)
    case BigCfg::kWide:
      if (dma32_ok(e.M, e.N, lda, ldw))
        return launch_big<256, 256, 128, 2, 1, GLU, 4>(a, lda, w, ldw, K, e, ws, ws_bytes, st);
      return launch_big<256, 256, 128, 2, 1, GLU>(a, lda, w, ldw, K, e, ws, ws_bytes, st);
    case BigCfg::kSmall:
      return launch_big<64, 128, 128, 3, 2, GLU, 1>(a, lda, w, ldw, K, e, ws, ws_bytes, st);
    case BigCfg::kSmall32: {
      // a grid that fits one workgroup per CU takes a 4-stage ring (80 KB);
      // larger grids 3 stages, two workgroups per CU
      const BigPlan p = big_plan(e.M, e.N, K, 32, 128, 128);
      if (p.tiles_m * p.tiles_n * p.ksplit <= 256)
        return launch_big<32, 128, 128, 4, 1, GLU, 1>(a, lda, w, ldw, K, e, ws, ws_bytes, st);
      return launch_big<32, 128, 128, 3, 2, GLU, 1>(a, lda, w, ldw, K, e, ws, ws_bytes, st);
    }
    default:
      if (dma32_ok(e.M, e.N, lda, ldw))
        return launch_big<128, 256, 128, 3, 1, GLU, 2>(a, lda, w, ldw, K, e, ws, ws_bytes, st);
      return launch_big<128, 256, 128, 2, 1, GLU, 1>(a, lda, w, ldw, K, e, ws, ws_bytes, st);
  }
}

}  // namespace
}  // namespace ifx

using namespace ifx;

extern "C" {

size_t ifx_fp8_linear_workspace_size(int64_t M, int64_t N, int64_t K, int epilogue) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  if (M <= kSkinnyMaxM) return 0;  // the skinny kernel needs no workspace
  if (!big_path(M, K)) return 0;
  switch (pick_big(M, N, K, (epilogue & (IFX_EPI_GEGLU | IFX_EPI_SWIGLU)) != 0)) {
    case BigCfg::kWide192: return big_plan(M, N, K, 256, 192, 128).ws_bytes;
    case BigCfg::kWide: return big_plan(M, N, K, 256, 256, 128).ws_bytes;
    case BigCfg::kSmall: return big_plan(M, N, K, 64, 128, 128).ws_bytes;
    case BigCfg::kSmall32: return big_plan(M, N, K, 32, 128, 128).ws_bytes;
    default: return big_plan(M, N, K, 128, 256, 128).ws_bytes;
  }
}

}  // extern "C"

namespace {

// Checks shared by ifx_fp8_linear and ifx_quant_linear (everything but the
// activation operand); IFX_OK when the call may proceed.
int check_linear(const void* w, int64_t ldw, const float* sw, const float* bias, const void* residual, int64_t ldr,
                 const void* gate, int epilogue, const void* out, int64_t ldo, int64_t M, int64_t N, int64_t K) {
  constexpr int kKnown = IFX_EPI_BIAS | IFX_EPI_GELU_TANH | IFX_EPI_GEGLU | IFX_EPI_SWIGLU |
                         IFX_EPI_RESIDUAL | IFX_EPI_GATE | IFX_EPI_OUT_F32 | IFX_EPI_RES_F32 |
                         IFX_EPI_SCALAR_SA | IFX_EPI_SCALAR_SW | IFX_EPI_W_TILED | IFX_EPI_A_TILED |
                         IFX_EPI_OUT_F16;
  if (epilogue & ~kKnown) return IFX_ERR_INVALID;
  if ((epilogue & IFX_EPI_OUT_F32) && (epilogue & IFX_EPI_OUT_F16)) return IFX_ERR_INVALID;
  const bool glu = (epilogue & (IFX_EPI_GEGLU | IFX_EPI_SWIGLU)) != 0;
  const bool tiled = (epilogue & IFX_EPI_W_TILED) != 0;
  // the tile layouts serve M <= 64
  if ((tiled || (epilogue & IFX_EPI_A_TILED)) && M > kSkinnyMaxM) return IFX_ERR_UNSUPPORTED;
  if ((epilogue & IFX_EPI_GEGLU) && (epilogue & IFX_EPI_SWIGLU)) return IFX_ERR_INVALID;
  if (glu && (epilogue & IFX_EPI_GELU_TANH)) return IFX_ERR_INVALID;
  if (M < 0 || N <= 0 || K <= 0 || N % 16 != 0 || K % 16 != 0) return IFX_ERR_INVALID;
  if (glu && N % 32 != 0) return IFX_ERR_INVALID;
  const int64_t n_out = glu ? N / 2 : N;
  if ((!tiled && ldw < K) || ldo < n_out) return IFX_ERR_INVALID;
  if (M == 0) return IFX_OK;
  if (!w || !out) return IFX_ERR_INVALID;
  if ((epilogue & IFX_EPI_BIAS) && !bias) return IFX_ERR_INVALID;
  if ((epilogue & IFX_EPI_GATE) && !gate) return IFX_ERR_INVALID;
  if (epilogue & IFX_EPI_RESIDUAL) {
    if (!residual || ldr < n_out || ldr % 8 != 0 || !aligned16(residual)) return IFX_ERR_INVALID;
  }
  if (!aligned16(w) || !aligned16(out) || (!tiled && ldw % 16 != 0) || ldo % 8 != 0) return IFX_ERR_ALIGN;
  if ((sw && !(epilogue & IFX_EPI_SCALAR_SW) && !aligned16(sw)) || (bias && !aligned16(bias)) ||
      (gate && (reinterpret_cast<uintptr_t>(gate) & 7u)))
    return IFX_ERR_ALIGN;
  return IFX_OK;
}

// Large-M outputs of at least this many bytes are stored nontemporally, so
// that they do not displace the operands that later kernels find in the
// 256 MB memory-side cache.
constexpr int64_t kNtOutBytes = int64_t(32) << 20;

inline size_t round256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

// Workspace of ifx_quant_linear: the GEMM's own workspace first (split-K
// partials), then the e4m3 copy of x (row stride K), the per-token scales and
// the per-tensor amax partials.
struct QlWorkspace {
  size_t gemm, q, scale, partial, total;
};

QlWorkspace ql_workspace(int64_t M, int64_t N, int64_t K, int epilogue, int scale_mode) {
  QlWorkspace w{};
  w.gemm = round256(ifx_fp8_linear_workspace_size(M, N, K, epilogue));
  w.q = round256(static_cast<size_t>(M) * K);
  w.scale = round256(static_cast<size_t>(M) * sizeof(float));
  w.partial = scale_mode == IFX_SCALE_TENSOR ? round256(ifx_quant_tensor_workspace_size(M * K)) : 0;
  w.total = w.gemm + w.q + w.scale + w.partial;
  return w;
}

}  // namespace

extern "C" {

int ifx_fp8_linear(const void* a, int64_t lda, const float* sa, const void* w, int64_t ldw,
                   const float* sw, const float* bias, const void* residual, int64_t ldr,
                   const void* gate, int epilogue, void* out, int64_t ldo, int64_t M, int64_t N,
                   int64_t K, void* workspace, size_t ws_bytes, void* stream) {
  const int rc = check_linear(w, ldw, sw, bias, residual, ldr, gate, epilogue, out, ldo, M, N, K);
  if (rc != IFX_OK) return rc;
  const bool a_tiled = (epilogue & IFX_EPI_A_TILED) != 0;
  if (!a_tiled && lda < K) return IFX_ERR_INVALID;
  if (M == 0) return IFX_OK;
  if (!a) return IFX_ERR_INVALID;
  if (!aligned16(a) || (!a_tiled && lda % 16 != 0)) return IFX_ERR_ALIGN;
  const bool glu = (epilogue & (IFX_EPI_GEGLU | IFX_EPI_SWIGLU)) != 0;

  Epi e{sa, sw, bias, residual, ldr, static_cast<const uint16_t*>(gate), out, ldo, epilogue, M, N};
  const uint8_t* A = static_cast<const uint8_t*>(a);
  const uint8_t* Wt = static_cast<const uint8_t*>(w);
  hipStream_t st = static_cast<hipStream_t>(stream);

  if (M <= kSkinnyMaxM) {
    const SkinnyPlan p = skinny_plan(M, N, K, glu);
    return glu ? launch_skinny<2>(p, A, lda, Wt, ldw, K, e, st) : launch_skinny<1>(p, A, lda, Wt, ldw, K, e, st);
  }
  if (big_path(M, K)) {
    const int64_t out_bytes = M * (glu ? N / 2 : N) * static_cast<int64_t>(sizeof(uint16_t));
    e.nt_out = out_bytes >= kNtOutBytes;
    return glu ? launch_large<true>(A, lda, Wt, ldw, K, e, workspace, ws_bytes, st)
               : launch_large<false>(A, lda, Wt, ldw, K, e, workspace, ws_bytes, st);
  }
  // Grids under one round of 256 x 128 tiles take 64 x 64 tiles (4 waves of
  // 32 x 32): 100x2560x2064 35.5 -> 10.5 us, 1000x2048x2064 39.5 -> 16.8 us.
  if (((M + 127) / 128) * ((N + 255) / 256) < 256)
    return glu ? launch_lds<64, 64, 2, 2, true>(A, lda, Wt, ldw, K, e, st)
               : launch_lds<64, 64, 2, 2, false>(A, lda, Wt, ldw, K, e, st);
  return glu ? launch_lds<256, 128, 2, 2, true>(A, lda, Wt, ldw, K, e, st)
             : launch_lds<256, 128, 2, 2, false>(A, lda, Wt, ldw, K, e, st);
}

int ifx_fp8_linear_qkv_rope(const void* a, int64_t lda, const float* sa, const void* w, int64_t ldw,
                            const float* sw, const float* bias, int flags, const float* pos, int64_t ldpos,
                            const float* inv_freq, int64_t heads_q, int64_t heads_kv, int64_t head_dim,
                            void* q_out, int64_t sq_t, int64_t sq_h, void* k_out, int64_t sk_t, int64_t sk_h,
                            void* v_out, int64_t sv_t, int64_t sv_h, int out_dtype, int64_t kv_base,
                            const int32_t* kv_base_dev, int64_t M, int64_t K, void* workspace, size_t ws_bytes,
                            void* stream) {
  constexpr int kAllowed = IFX_EPI_BIAS | IFX_EPI_W_TILED | IFX_EPI_A_TILED;
  (void)workspace;  // the skinny kernel needs none (ifx_fp8_linear_workspace_size is 0 for M <= 64)
  (void)ws_bytes;
  if (flags & ~kAllowed) return IFX_ERR_INVALID;
  if (out_dtype != IFX_DTYPE_BF16 && out_dtype != IFX_DTYPE_F16 && out_dtype != IFX_DTYPE_F32) return IFX_ERR_INVALID;
  if (heads_q <= 0 || heads_kv <= 0 || head_dim <= 0 || head_dim % 16 != 0 || kv_base < 0) return IFX_ERR_INVALID;
  if (head_dim > 256) return IFX_ERR_UNSUPPORTED;
  if (M > kSkinnyMaxM) return IFX_ERR_UNSUPPORTED;  // the register epilogue is the skinny kernel's
  const int64_t N = (heads_q + 2 * heads_kv) * head_dim;
  // check_linear validates the operands; the Q buffer stands in for `out`
  // (its own layout is checked below)
  const int rc = check_linear(w, ldw, sw, bias, nullptr, 0, nullptr, flags, q_out, N, M, N, K);
  if (rc != IFX_OK) return rc;
  const bool a_tiled = (flags & IFX_EPI_A_TILED) != 0;
  if (!a_tiled && lda < K) return IFX_ERR_INVALID;
  if (inv_freq && (!pos || ldpos < 1)) return IFX_ERR_INVALID;
  if (sq_h < head_dim || sq_t < heads_q * sq_h || sk_h < head_dim || sv_h < head_dim) return IFX_ERR_INVALID;
  if (sk_t < heads_kv * sk_h || sv_t < heads_kv * sv_h) return IFX_ERR_INVALID;
  if (M == 0) return IFX_OK;
  if (!a || !k_out || !v_out) return IFX_ERR_INVALID;
  if (!aligned16(a) || (!a_tiled && lda % 16 != 0)) return IFX_ERR_ALIGN;
  Epi e{sa, sw, bias, nullptr, 0, nullptr, q_out, N, flags | kEpiRopeQkv, M, N};
  const RopeQkv r{pos, ldpos, inv_freq, heads_q, heads_kv, head_dim, q_out, sq_t, sq_h, k_out, sk_t, sk_h,
                  v_out, sv_t, sv_h, kv_base, kv_base_dev, out_dtype};
  const SkinnyPlan p = skinny_plan(M, N, K, false);
  return launch_skinny<1>(p, static_cast<const uint8_t*>(a), lda, static_cast<const uint8_t*>(w), ldw, K, e,
                          static_cast<hipStream_t>(stream), &r);
}

size_t ifx_fp8_skinny_tiled_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || N % 16 != 0 || K % 16 != 0) return 0;
  return static_cast<size_t>(N / 16) * ((K + kBK - 1) / kBK) * 2048;
}

int ifx_fp8_pack_skinny(const void* w, int64_t ldw, int64_t N, int64_t K, void* w_out, void* stream) {
  if (N <= 0 || K <= 0 || N % 16 != 0 || K % 16 != 0 || ldw < K) return IFX_ERR_INVALID;
  if (!w || !w_out) return IFX_ERR_INVALID;
  if (!aligned16(w) || !aligned16(w_out) || ldw % 16 != 0) return IFX_ERR_ALIGN;
  const int64_t ks = (K + kBK - 1) / kBK;
  const int64_t chunks = (N / 16) * ks * 128;
  if ((chunks + 255) / 256 > 0x7FFFFFFFLL) return IFX_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(pack_skinny_kernel, dim3(static_cast<unsigned>((chunks + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(w), ldw, K, ks, chunks,
                     static_cast<uint8_t*>(w_out));
  return launch_status();
}

size_t ifx_quant_linear_workspace_size(int64_t M, int64_t N, int64_t K, int epilogue, int scale_mode) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return ql_workspace(M, N, K, epilogue, scale_mode).total;
}

}  // extern "C"

namespace {
// Contract checks of ifx_quant_linear that do not involve the workspace, shared
// with ifx_quant_linear_noalloc so that a rejected call launches nothing.
int check_quant_linear(const void* x, int64_t ldx, int scale_mode, const void* w, int64_t ldw, const float* sw,
                       const float* bias, const void* residual, int64_t ldr, const void* gate, int epilogue,
                       void* out, int64_t ldo, int64_t M, int64_t N, int64_t K) {
  if (scale_mode != IFX_SCALE_ROW && scale_mode != IFX_SCALE_TENSOR) return IFX_ERR_INVALID;
  if (epilogue & IFX_EPI_SCALAR_SA) return IFX_ERR_INVALID;  // the scale is computed here
  const int rc = check_linear(w, ldw, sw, bias, residual, ldr, gate, epilogue, out, ldo, M, N, K);
  if (rc != IFX_OK) return rc;
  if (ldx < K) return IFX_ERR_INVALID;
  if (M == 0) return IFX_OK;
  if (!x) return IFX_ERR_INVALID;
  if (!aligned16(x) || ldx % 8 != 0) return IFX_ERR_ALIGN;
  if (scale_mode == IFX_SCALE_TENSOR && ldx != K) return IFX_ERR_UNSUPPORTED;
  return IFX_OK;
}
}  // namespace

extern "C" {

int ifx_quant_linear(const void* x, int64_t ldx, int scale_mode, const void* w, int64_t ldw, const float* sw,
                     const float* bias, const void* residual, int64_t ldr, const void* gate, int epilogue,
                     void* out, int64_t ldo, int64_t M, int64_t N, int64_t K, float* a_scale, void* workspace,
                     size_t ws_bytes, void* stream) {
  const int rc = check_quant_linear(x, ldx, scale_mode, w, ldw, sw, bias, residual, ldr, gate, epilogue, out, ldo,
                                    M, N, K);
  if (rc != IFX_OK || M == 0) return rc;
  // the stand-alone quantizer into the workspace, then the GEMM
  const QlWorkspace ql = ql_workspace(M, N, K, epilogue, scale_mode);
  if (!workspace || ws_bytes < ql.total || (reinterpret_cast<uintptr_t>(workspace) & 255u)) return IFX_ERR_WORKSPACE;
  uint8_t* base = static_cast<uint8_t*>(workspace);
  void* gws = base;
  uint8_t* q = base + ql.gemm;
  float* sa = a_scale ? a_scale : reinterpret_cast<float*>(base + ql.gemm + ql.q);
  void* partial = base + ql.gemm + ql.q + ql.scale;
  int r;
  if (scale_mode == IFX_SCALE_TENSOR)
    r = ifx_quant_tensor_bf16(x, M * K, q, sa, partial, ql.partial, stream);
  else
    r = ifx_quant_rows(x, IFX_DTYPE_BF16, ldx, M, K, q, K, sa, stream);
  if (r != IFX_OK) return r;
  const int flags = epilogue | (scale_mode == IFX_SCALE_TENSOR ? IFX_EPI_SCALAR_SA : 0);
  return ifx_fp8_linear(q, K, sa, w, ldw, sw, bias, residual, ldr, gate, flags, out, ldo, M, N, K, gws, ql.gemm,
                        stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// ifx_quant_linear_noalloc: ifx_quant_linear on a library-owned scratch buffer
// ---------------------------------------------------------------------------
//
// For callers that cannot allocate (code under HIP graph capture, serving
// loops that forbid hipMalloc). The workspace of ifx_quant_linear (split-K
// partials, the e4m3 copy of x, the scales) lives in `scratch`, a
// file-scope device array: every GPU the library runs on holds its own copy
// (at its own address) until the process ends. Host code never passes the
// array's name to a kernel (in host code it names a host-side shadow); it uses
// the device address that hipGetSymbolAddress returns, looked up once per
// device with that device current.

namespace {

constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// Device address of this device's `scratch`, or nullptr (status in *rc).
void* scratch_ptr(int* rc) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *rc = static_cast<int>(e);
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *rc = IFX_ERR_UNSUPPORTED;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *rc = e != hipSuccess ? static_cast<int>(e) : IFX_ERR_UNSUPPORTED;
      return nullptr;
    }
    g_scratch[dev] = p;
  }
  *rc = IFX_OK;
  return g_scratch[dev];
}

}  // namespace

extern "C" {

size_t ifx_quant_linear_noalloc_max_bytes(void) { return kScratchBytes; }

int ifx_quant_linear_noalloc(const void* x, int64_t ldx, int scale_mode, const void* w, int64_t ldw,
                             const float* sw, const float* bias, const void* residual, int64_t ldr,
                             const void* gate, int epilogue, void* out, int64_t ldo, int64_t M, int64_t N,
                             int64_t K, float* a_scale, void* stream) {
  if (M < 0 || N <= 0 || K <= 0) return IFX_ERR_INVALID;
  // every contract check before the scratch is touched: a rejected call launches nothing
  int rc = check_quant_linear(x, ldx, scale_mode, w, ldw, sw, bias, residual, ldr, gate, epilogue, out, ldo, M, N, K);
  if (rc != IFX_OK || M == 0) return rc;
  const size_t need = ql_workspace(M, N, K, epilogue, scale_mode).total;
  if (need > kScratchBytes) return IFX_ERR_SCRATCH;
  void* ws = scratch_ptr(&rc);
  if (!ws) return rc;
  return ifx_quant_linear(x, ldx, scale_mode, w, ldw, sw, bias, residual, ldr, gate, epilogue, out, ldo, M, N, K,
                          a_scale, ws, kScratchBytes, stream);
}

}  // extern "C"
