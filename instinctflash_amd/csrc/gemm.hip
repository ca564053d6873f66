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
// Kernels
//  * gemm_lds  (M > 64): BN x BM workgroup tile, BK = 128 bytes of K per stage,
//    A and W tiles double-buffered in LDS (16-byte chunks XOR-swizzled by row so
//    the fragment reads are bank-conflict free), global loads of stage k+1 in
//    flight while stage k runs on the matrix cores, epilogue from registers.
//  * gemm_skinny (M <= 64): bandwidth-bound on the weight stream. One workgroup
//    owns 16 (32 for GLU) weight rows and a K range; every wave streams weight
//    fragments straight from HBM into MFMA registers (no LDS staging), partial
//    sums are reduced across waves in LDS and, when K is split across
//    workgroups, across workgroups through a workspace: the last workgroup to
//    finish a row group (atomic ticket) adds the partials in split order and
//    runs the epilogue, so results are deterministic; it also resets the ticket,
//    so the workspace stays zeroed between calls.

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
};

__device__ __forceinline__ float4 load_f4_or(const float* p, int64_t i, float dflt) {
  if (!p) return make_float4(dflt, dflt, dflt, dflt);
  return *reinterpret_cast<const float4*>(p + i);
}

// y (four consecutive output columns c..c+3 of row m, after activation) ->
// gate, residual, store.
__device__ __forceinline__ void epi_finish4(const Epi& e, int64_t m, int64_t c, float* y) {
  if (e.flags & IFX_EPI_GATE) {
    const uint2 g = *reinterpret_cast<const uint2*>(e.gate + c);
    y[0] *= __uint_as_float(g.x << 16);
    y[1] *= __uint_as_float(g.x & 0xFFFF0000u);
    y[2] *= __uint_as_float(g.y << 16);
    y[3] *= __uint_as_float(g.y & 0xFFFF0000u);
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
  if (e.flags & IFX_EPI_OUT_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(e.out) + m * e.ldo + c) = make_float4(y[0], y[1], y[2], y[3]);
  } else {
    uint2 o;
    o.x = pack_bf16x2(y[0], y[1]);
    o.y = pack_bf16x2(y[2], y[3]);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(e.out) + m * e.ldo + c) = o;
  }
}

// Plain epilogue for one lane's D fragment: rows n..n+3 of W, token m.
__device__ __forceinline__ void epi_store(const Epi& e, const v4f acc, int64_t n, int64_t m) {
  if (m >= e.M || n >= e.N) return;
  const float sa = e.sa ? e.sa[m] : 1.0f;
  const float4 sw = load_f4_or(e.sw, n, 1.0f);
  const float4 b = load_f4_or((e.flags & IFX_EPI_BIAS) ? e.bias : nullptr, n, 0.0f);
  float y[4] = {acc[0] * sa * sw.x + b.x, acc[1] * sa * sw.y + b.y, acc[2] * sa * sw.z + b.z,
                acc[3] * sa * sw.w + b.w};
  if (e.flags & IFX_EPI_GELU_TANH) {
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = gelu_tanh(y[r]);
  }
  epi_finish4(e, m, n, y);
}

// GLU epilogue: `ng` is the packed row of the gate fragment, the up fragment is
// 16 packed rows later; output column = (ng / 32) * 16 + (ng % 16).
__device__ __forceinline__ void epi_store_glu(const Epi& e, const v4f accg, const v4f accu, int64_t ng,
                                              int64_t m) {
  if (m >= e.M || ng >= e.N) return;
  const float sa = e.sa ? e.sa[m] : 1.0f;
  const float4 swg = load_f4_or(e.sw, ng, 1.0f);
  const float4 swu = load_f4_or(e.sw, ng + 16, 1.0f);
  const float* bp = (e.flags & IFX_EPI_BIAS) ? e.bias : nullptr;
  const float4 bg = load_f4_or(bp, ng, 0.0f);
  const float4 bu = load_f4_or(bp, ng + 16, 0.0f);
  const float g[4] = {accg[0] * sa * swg.x + bg.x, accg[1] * sa * swg.y + bg.y,
                      accg[2] * sa * swg.z + bg.z, accg[3] * sa * swg.w + bg.w};
  const float u[4] = {accu[0] * sa * swu.x + bu.x, accu[1] * sa * swu.y + bu.y,
                      accu[2] * sa * swu.z + bu.z, accu[3] * sa * swu.w + bu.w};
  float y[4];
  const bool swiglu = (e.flags & IFX_EPI_SWIGLU) != 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) y[r] = (swiglu ? silu(g[r]) : gelu_tanh(g[r])) * u[r];
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

// byte offset of 16-byte chunk `ch` of tile row `row` (XOR swizzle by row).
__device__ __forceinline__ int swz(int row, int ch) { return row * kBK + ((ch ^ (row & 7)) << 4); }

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
// Skinny kernel (M <= 64): weight streaming, split-K
// ---------------------------------------------------------------------------

constexpr int kSkWaves = 4;
constexpr int kSkUnroll = 4;  // K steps whose loads are issued together per wave

struct SkinnyPlan {
  int mb;         // 16-token blocks (1..4)
  int nbw;        // 16-row weight blocks per workgroup (1, or 2 for GLU)
  int64_t groups; // workgroups along N
  int splits;     // workgroups along K
  int64_t ksteps; // 128-byte K steps in total
  int64_t steps_per_split;
  size_t ws_bytes;
};

// Workspace layout (fixed for every shape, so a call never finds another call's
// partial sums where its tickets live): [tickets: kTicketBytes][partials].
// Split-K is only used when there are fewer than kMaxTicketGroups row groups.
constexpr int64_t kMaxTicketGroups = 1024;
constexpr size_t kTicketBytes = kMaxTicketGroups * sizeof(uint32_t);

__host__ inline SkinnyPlan skinny_plan(int64_t M, int64_t N, int64_t K, bool glu) {
  SkinnyPlan p{};
  p.mb = static_cast<int>((M + 15) / 16);
  p.nbw = glu ? 2 : 1;
  p.groups = N / (16 * p.nbw);
  p.ksteps = (K + kBK - 1) / kBK;
  // Aim for >= 256 workgroups (one per CU) while giving every wave at least
  // two K steps of its own.
  int64_t s = (256 + p.groups - 1) / p.groups;
  const int64_t smax = p.ksteps / (2 * kSkWaves);
  if (s > smax) s = smax;
  if (s < 1 || p.groups > kMaxTicketGroups) s = 1;
  p.steps_per_split = (p.ksteps + s - 1) / s;
  p.splits = static_cast<int>((p.ksteps + p.steps_per_split - 1) / p.steps_per_split);
  if (p.splits > 1) {
    const size_t partial = static_cast<size_t>(p.splits) * p.groups * p.nbw * p.mb * 64 * 4 * sizeof(float);
    p.ws_bytes = kTicketBytes + partial;
  }
  return p;
}

template <int MB, int NBW>
__global__ __launch_bounds__(kSkWaves * 64) void gemm_skinny(const uint8_t* __restrict__ A, int64_t lda,
                                                             const uint8_t* __restrict__ W, int64_t ldw,
                                                             int64_t K, int64_t steps_per_split, int splits,
                                                             uint32_t* tickets, float* partials, Epi e) {
  __shared__ v4f red[kSkWaves][NBW][MB][64];
  __shared__ int last_flag;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t grp = blockIdx.x;
  const int split = blockIdx.y;
  const int64_t nrow0 = grp * (16 * NBW);
  const int frow = lane & 15;
  const int g = lane >> 4;

  const int64_t ksteps = (K + kBK - 1) / kBK;
  const int64_t s_begin = split * steps_per_split;
  int64_t s_end = s_begin + steps_per_split;
  s_end = s_end < ksteps ? s_end : ksteps;

  const uint8_t* wrow[NBW];
#pragma unroll
  for (int b = 0; b < NBW; ++b) wrow[b] = W + (nrow0 + b * 16 + frow) * ldw + g * 32;
  const uint8_t* arow[MB];
#pragma unroll
  for (int j = 0; j < MB; ++j) {
    int64_t m = j * 16 + frow;
    m = m < e.M ? m : e.M - 1;
    arow[j] = A + m * lda + g * 32;
  }

  v4f acc[NBW][MB];
#pragma unroll
  for (int b = 0; b < NBW; ++b)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[b][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // Wave w takes K steps s_begin+w, +kSkWaves, ... in groups of kSkUnroll whose
  // loads are all issued before the first MFMA of the group.
  for (int64_t s0 = s_begin + wave; s0 < s_end; s0 += kSkWaves * kSkUnroll) {
    v8i wf[kSkUnroll][NBW];
    v8i af[kSkUnroll][MB];
#pragma unroll
    for (int u = 0; u < kSkUnroll; ++u) {
      const int64_t s = s0 + u * kSkWaves;
      const int64_t k0 = s * kBK + g * 32;
      const bool ok = s < s_end;
      const bool lo = ok && k0 < K;       // K % 16 == 0: each 16-byte half is all-in or all-out
      const bool hi = ok && k0 + 16 < K;
#pragma unroll
      for (int b = 0; b < NBW; ++b) {
        const uint8_t* p = wrow[b] + s * kBK;
        const v4i x0 = lo ? ld16_nt(p) : v4i{0, 0, 0, 0};
        const v4i x1 = hi ? ld16_nt(p + 16) : v4i{0, 0, 0, 0};
        wf[u][b] = cat8(x0, x1);
      }
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        const uint8_t* p = arow[j] + s * kBK;
        const v4i x0 = lo ? ld16(p) : v4i{0, 0, 0, 0};
        const v4i x1 = hi ? ld16(p + 16) : v4i{0, 0, 0, 0};
        af[u][j] = cat8(x0, x1);
      }
    }
#pragma unroll
    for (int u = 0; u < kSkUnroll; ++u)
#pragma unroll
      for (int b = 0; b < NBW; ++b)
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[b][j] = mfma16(wf[u][b], af[u][j], acc[b][j]);
  }

  // Cross-wave reduction in LDS (fixed order: wave 0..3).
#pragma unroll
  for (int b = 0; b < NBW; ++b)
#pragma unroll
    for (int j = 0; j < MB; ++j) red[wave][b][j][lane] = acc[b][j];
  __syncthreads();
  // Wave w finalizes fragment pairs (b, j) with (b*MB + j) % kSkWaves == w.
  constexpr int kFrags = NBW * MB;

  if (splits > 1) {
    // Publish this split's partial sums, then take a ticket.
    for (int f = wave; f < kFrags; f += kSkWaves) {
      const int b = f / MB, j = f % MB;
      v4f s = red[0][b][j][lane];
#pragma unroll
      for (int w = 1; w < kSkWaves; ++w) s += red[w][b][j][lane];
      float* dst = partials + ((((static_cast<int64_t>(split) * gridDim.x + grp) * NBW + b) * MB + j) * 64 + lane) * 4;
      *reinterpret_cast<v4f*>(dst) = s;
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const uint32_t t = atomicAdd(tickets + grp, 1u);
      last_flag = (t == static_cast<uint32_t>(splits - 1));
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    for (int f = wave; f < kFrags; f += kSkWaves) {
      const int b = f / MB, j = f % MB;
      v4f s = v4f{0.f, 0.f, 0.f, 0.f};
      for (int sp = 0; sp < splits; ++sp) {
        const float* src = partials + ((((static_cast<int64_t>(sp) * gridDim.x + grp) * NBW + b) * MB + j) * 64 + lane) * 4;
        s += __builtin_nontemporal_load(reinterpret_cast<const v4f*>(src));
      }
      red[0][b][j][lane] = s;
    }
    if (tid == 0) tickets[grp] = 0u;
  } else {
    for (int f = wave; f < kFrags; f += kSkWaves) {
      const int b = f / MB, j = f % MB;
      v4f s = red[0][b][j][lane];
#pragma unroll
      for (int w = 1; w < kSkWaves; ++w) s += red[w][b][j][lane];
      red[0][b][j][lane] = s;
    }
  }
  __syncthreads();
  const int64_t m_base = frow;
  if constexpr (NBW == 2) {
    // GLU: block 0 = gate rows, block 1 = up rows.
    for (int j = wave; j < MB; j += kSkWaves)
      epi_store_glu(e, red[0][0][j][lane], red[0][1][j][lane], nrow0 + 4 * g, m_base + j * 16);
  } else {
    for (int j = wave; j < MB; j += kSkWaves) epi_store(e, red[0][0][j][lane], nrow0 + 4 * g, m_base + j * 16);
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

template <int MB, int NBW>
void launch_skinny_mb(const SkinnyPlan& p, const uint8_t* a, int64_t lda, const uint8_t* w, int64_t ldw,
                      int64_t K, uint32_t* tickets, float* partials, const Epi& e, hipStream_t st) {
  hipLaunchKernelGGL((gemm_skinny<MB, NBW>), dim3(static_cast<unsigned>(p.groups), p.splits),
                     dim3(kSkWaves * 64), 0, st, a, lda, w, ldw, K, p.steps_per_split, p.splits, tickets,
                     partials, e);
}

template <int NBW>
int launch_skinny(const SkinnyPlan& p, const uint8_t* a, int64_t lda, const uint8_t* w, int64_t ldw,
                  int64_t K, void* ws, const Epi& e, hipStream_t st) {
  uint32_t* tickets = static_cast<uint32_t*>(ws);
  float* partials = nullptr;
  if (p.splits > 1) partials = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kTicketBytes);
  switch (p.mb) {
    case 1: launch_skinny_mb<1, NBW>(p, a, lda, w, ldw, K, tickets, partials, e, st); break;
    case 2: launch_skinny_mb<2, NBW>(p, a, lda, w, ldw, K, tickets, partials, e, st); break;
    case 3: launch_skinny_mb<3, NBW>(p, a, lda, w, ldw, K, tickets, partials, e, st); break;
    default: launch_skinny_mb<4, NBW>(p, a, lda, w, ldw, K, tickets, partials, e, st); break;
  }
  return launch_status();
}

constexpr int64_t kSkinnyMaxM = 64;

}  // namespace
}  // namespace ifx

using namespace ifx;

extern "C" {

size_t ifx_fp8_linear_workspace_size(int64_t M, int64_t N, int64_t K, int epilogue) {
  if (M <= 0 || M > kSkinnyMaxM || N <= 0 || K <= 0) return 0;
  const bool glu = (epilogue & (IFX_EPI_GEGLU | IFX_EPI_SWIGLU)) != 0;
  return skinny_plan(M, N, K, glu).ws_bytes;
}

int ifx_fp8_linear(const void* a, int64_t lda, const float* sa, const void* w, int64_t ldw,
                   const float* sw, const float* bias, const void* residual, int64_t ldr,
                   const void* gate, int epilogue, void* out, int64_t ldo, int64_t M, int64_t N,
                   int64_t K, void* workspace, size_t ws_bytes, void* stream) {
  constexpr int kKnown = IFX_EPI_BIAS | IFX_EPI_GELU_TANH | IFX_EPI_GEGLU | IFX_EPI_SWIGLU |
                         IFX_EPI_RESIDUAL | IFX_EPI_GATE | IFX_EPI_OUT_F32 | IFX_EPI_RES_F32;
  if (epilogue & ~kKnown) return IFX_ERR_INVALID;
  const bool glu = (epilogue & (IFX_EPI_GEGLU | IFX_EPI_SWIGLU)) != 0;
  if ((epilogue & IFX_EPI_GEGLU) && (epilogue & IFX_EPI_SWIGLU)) return IFX_ERR_INVALID;
  if (glu && (epilogue & IFX_EPI_GELU_TANH)) return IFX_ERR_INVALID;
  if (M < 0 || N <= 0 || K <= 0 || N % 16 != 0 || K % 16 != 0) return IFX_ERR_INVALID;
  if (glu && N % 32 != 0) return IFX_ERR_INVALID;
  const int64_t n_out = glu ? N / 2 : N;
  if (lda < K || ldw < K || ldo < n_out) return IFX_ERR_INVALID;
  if (M == 0) return IFX_OK;
  if (!a || !w || !out) return IFX_ERR_INVALID;
  if ((epilogue & IFX_EPI_BIAS) && !bias) return IFX_ERR_INVALID;
  if ((epilogue & IFX_EPI_GATE) && !gate) return IFX_ERR_INVALID;
  if (epilogue & IFX_EPI_RESIDUAL) {
    if (!residual || ldr < n_out || ldr % 8 != 0 || !aligned16(residual)) return IFX_ERR_INVALID;
  }
  if (!aligned16(a) || !aligned16(w) || !aligned16(out) || lda % 16 != 0 || ldw % 16 != 0 || ldo % 8 != 0)
    return IFX_ERR_ALIGN;
  if ((sw && !aligned16(sw)) || (bias && !aligned16(bias)) || (gate && (reinterpret_cast<uintptr_t>(gate) & 7u)))
    return IFX_ERR_ALIGN;

  Epi e{sa, sw, bias, residual, ldr, static_cast<const uint16_t*>(gate), out, ldo, epilogue, M, N};
  const uint8_t* A = static_cast<const uint8_t*>(a);
  const uint8_t* Wt = static_cast<const uint8_t*>(w);
  hipStream_t st = static_cast<hipStream_t>(stream);

  if (M <= kSkinnyMaxM) {
    const SkinnyPlan p = skinny_plan(M, N, K, glu);
    if (p.splits > 1 && (!workspace || ws_bytes < p.ws_bytes)) return IFX_ERR_WORKSPACE;
    return glu ? launch_skinny<2>(p, A, lda, Wt, ldw, K, workspace, e, st)
               : launch_skinny<1>(p, A, lda, Wt, ldw, K, workspace, e, st);
  }
  return glu ? launch_lds<256, 128, 2, 2, true>(A, lda, Wt, ldw, K, e, st)
             : launch_lds<256, 128, 2, 2, false>(A, lda, Wt, ldw, K, e, st);
}

}  // extern "C"
