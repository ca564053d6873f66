// Attention for short robotics sequences (non-causal, or causal with an
// offset) on gfx950 matrix cores, with split-KV partials and a combine kernel
// that can quantize each token's full output row to FP8 E4M3 -- the producer of
// the output projection's A operand.
//
// Reference: instinctflash/kernels/attention.py:23-213 (`attention`,
// `SplitWorkspace`, the combine kernel with fused per-token FP8 output). Same
// semantics: grouped-query heads fold into query rows (row = token * group +
// head-in-group), query row t sees keys [0, limit_t) with
// limit_t = kv_len (+ kv_extra[t]) (min causal_offset + t + 1), kv_len may be
// read from device memory (a captured graph follows it), kv_index makes key n
// the cache row kv_index[n]. The FP8 output uses this package's per-row
// quantization recipe (1e-12 floor, scale = amax * fl32(1/448), IEEE division)
// instead of the Triton 1e-8 floor and 448/amax multiply.
//
// Design. A 256-lane workgroup owns 128 query rows of one KV head (4 waves x 32
// rows) and one split of the keys. Per block of 64 keys the workgroup stages K
// and V row-major in LDS (16-byte copies; the next block's loads are in flight
// during the current block's matrix work); every wave then computes
//   S^T = K . Q^T      (v_mfma_f32_32x32x16_{bf16,f16}; keys are MFMA rows,
//                       queries MFMA columns, so lane l owns query l%32 and 16
//                       of its 32 keys per 32-key tile)
// so the online softmax needs no cross-lane traffic beyond one swap between
// the two lane halves for the running max, and
//   O^T = V^T . P^T    (P^T is the lane's own probabilities, packed to 16 bit;
//                       the MFMA K slots of a lane half h are keys
//                       8q0 + 4h + {0..3} and 8q0 + 8 + 4h + {0..3}, which both
//                       operands use, so no shuffling of P is needed; the V^T
//                       operand comes from the row-major V block through the
//                       gfx950 transposing LDS read ds_read_b64_tr_b16)
// keeping O^T in registers (lane = query, 16 head dims per 32-dim tile).

#include <type_traits>

#include "ifx_abi.h"
#include "ifx_device.h"
#include "ifx_quant.h"

namespace ifx {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kAttnThreads = 256;
constexpr int kRowsPerWg = 128;  // 4 waves x 32 query rows
constexpr int kBlockN = 64;      // keys per LDS block
typedef short s16x4_t __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 (measured on gfx950): within each group of 16 lanes, lane
// i receives element k (k = 0..3) = the (i % 4)-th 16-bit element at the
// address of group lane 4k + i / 4. Group lane j therefore addresses row
// kb + j / 4, columns c0 + 4 * (j % 4) .. +3 of a row-major tile, and lane i gets
// the 4 rows kb..kb+3 of column c0 + i.
__device__ __forceinline__ u32x2_t lds_read_tr16(const uint16_t* p) {
  const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4_t*)(const_cast<uint16_t*>(p)));
  return __builtin_bit_cast(u32x2_t, v);
}

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t sqb, sqt, sqh, skb, skt, skh, svb, svt, svh, sob, sot, soh;
  int64_t n_rows;   // Tq * group
  int64_t D;
  int64_t n_keys;   // addressable keys: Tk, or the length of kv_index
  int64_t Tk;       // cache rows (kv_index entries are clamped into it)
  int group;
  int Hkv;
  int kv_len_static;
  const int32_t* kv_len;    // device kv_len or null
  const int32_t* kv_extra;  // [Tq] or null
  int causal;
  int causal_offset;
  const int32_t* kv_index;  // or null
  float qk_scale;           // scale * log2(e)
  int splits;
  uint16_t* po;  // [splits, B, Hkv, n_rows, 32 * DT] partial outputs / their own l, 16-bit (operand type)
  float* pm;  // [splits, B, Hkv, n_rows] running max (log2 domain)
  float* pl;  // [splits, B, Hkv, n_rows] softmax denominators
};

template <bool BF16>
struct Mfma;

template <>
struct Mfma<true> {
  static __device__ __forceinline__ v16f run(u32x4_t a, u32x4_t b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    const bf2 v = {static_cast<__bf16>(x), static_cast<__bf16>(y)};
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ float to_f32(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }
};

template <>
struct Mfma<false> {
  static __device__ __forceinline__ v16f run(u32x4_t a, u32x4_t b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 v = {static_cast<_Float16>(x), static_cast<_Float16>(y)};
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ float to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
  }
};

// DT: 32-dim tiles of the head (D <= 32 * DT); D16 = ceil(D / 16) MFMA K chunks.
// Heads up to 128 dims run two workgroups per CU (<= 256 VGPRs), so one
// workgroup's softmax overlaps the other's matrix work; wider heads need the
// registers of one workgroup per CU.
template <bool BF16, int DT>
__global__ __launch_bounds__(kAttnThreads, DT <= 4 ? 2 : 1) void attn_kernel(AttnArgs a) {
  using MF = Mfma<BF16>;
  constexpr int kDP = 32 * DT;        // padded head dim of V^T / O
  constexpr int kKPitch = kDP + 8;    // bf16 elements per K row (pitch 4 dwords off a bank multiple)
  constexpr int kVPitch = kDP + 16;   // per V row (8 dwords off: 4 rows x 32 bytes of a transposing read)
  // K and V blocks; after the key loop the same memory stages the partial rows
  constexpr int kTp = 36;  // floats per transpose row (32 + 4: rows start in different banks)
  constexpr int kKV = kBlockN * (kKPitch + kVPitch);
  constexpr int kTr = 4 * 32 * kTp * 2;  // 4 waves x 32 x kTp floats, in 16-bit units
  __shared__ __attribute__((aligned(16))) uint16_t kv_lds[kKV > kTr ? kKV : kTr];
  uint16_t* const k_lds = kv_lds;
  uint16_t* const v_lds = kv_lds + kBlockN * kKPitch;
  __shared__ int s_end[4];
  __shared__ int s_min[4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;  // this lane's query (MFMA column)
  const int half = lane >> 5;
  const int kvh = blockIdx.y / a.splits;
  const int split = blockIdx.y % a.splits;
  const int64_t b = blockIdx.z;
  const int D = static_cast<int>(a.D);

  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerWg + wave * 32 + col;
  const bool row_ok = row < a.n_rows;
  const int64_t tok = row_ok ? row / a.group : 0;
  const int head = kvh * a.group + static_cast<int>(row_ok ? row % a.group : 0);

  // Q^T fragments (MFMA B operand): query `col`, dims 16c + 8*half .. +7;
  // issued first, their latency overlaps the key-range reduction below
  u32x4_t qf[2 * DT];
#pragma unroll
  for (int c = 0; c < 2 * DT; ++c) {
    const int d = 16 * c + 8 * half;
    if (row_ok && d < D)
      qf[c] = *reinterpret_cast<const u32x4_t*>(a.q + b * a.sqb + tok * a.sqt + head * a.sqh + d);
    else
      qf[c] = u32x4_t{0u, 0u, 0u, 0u};
  }

  // visible keys of this row; the workgroup's key range [start, end) and the
  // bound below which every row sees every key (blocks under it skip masking)
  int lim = 0;
  if (row_ok) {
    lim = a.kv_len ? a.kv_len[0] : a.kv_len_static;
    if (a.kv_extra) lim += a.kv_extra[tok];
    if (a.causal) lim = min(lim, static_cast<int>(tok) + a.causal_offset + 1);
    lim = max(0, min(lim, static_cast<int>(a.n_keys)));
  }
  {
    const uint32_t wmax = wave_max_u32(static_cast<uint32_t>(lim));
    const uint32_t wmin = ~wave_max_u32(~static_cast<uint32_t>(row_ok ? lim : 0x7FFFFFFF));
    if (lane == 0) {
      s_end[wave] = static_cast<int>(wmax);
      s_min[wave] = static_cast<int>(wmin);
    }
  }
  __syncthreads();
  int end = max(max(s_end[0], s_end[1]), max(s_end[2], s_end[3]));
  const int full_below = min(min(s_min[0], s_min[1]), min(s_min[2], s_min[3]));
  int start = 0;
  if (a.splits > 1) {
    const int per = ((end + a.splits - 1) / a.splits + kBlockN - 1) / kBlockN * kBlockN;
    start = split * per;
    end = min(end, start + per);
  }

  v16f acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = v16f{};
  float m_run = -__builtin_inff();
  float l_run = 0.0f;

  const uint16_t* kbase = a.k + b * a.skb + static_cast<int64_t>(kvh) * a.skh;
  const uint16_t* vbase = a.v + b * a.svb + static_cast<int64_t>(kvh) * a.svh;
  const int tk = static_cast<int>(a.Tk);
  auto key_row = [&](int n) -> int64_t {
    const int r = a.kv_index ? a.kv_index[n] : n;
    return r < 0 ? 0 : (r >= tk ? tk - 1 : r);
  };

  // K / V blocks go global -> registers -> LDS. The loads of block n0 + 64 are
  // issued before the matrix work of block n0, so their latency is hidden;
  // addresses are clamped into range (no branches), out-of-range pieces are
  // zeroed when written to LDS.
  constexpr int kCpr = kDP / 8;                           // 16-byte chunks per padded row
  constexpr int kKL = kBlockN * kCpr / kAttnThreads;      // chunks of K (and of V) per thread (= DT)
  static_assert(kBlockN * kCpr % kAttnThreads == 0, "staging");
  u32x4_t kreg[kKL], vreg[kKL];
  auto fetch = [&](int n0) {
#pragma unroll
    for (int i = 0; i < kKL; ++i) {
      const int c = tid + i * kAttnThreads;
      const int64_t r = key_row(min(n0 + c / kCpr, end - 1));
      const int dc = 8 * (c % kCpr) < D ? 8 * (c % kCpr) : 0;
      kreg[i] = *reinterpret_cast<const u32x4_t*>(kbase + r * a.skt + dc);
      vreg[i] = *reinterpret_cast<const u32x4_t*>(vbase + r * a.svt + dc);
    }
  };
  // Pieces past `end` or past D are zeroed: K so that masked scores stay finite,
  // V so that a zero probability never meets a non-finite value.
  auto stage = [&](int n0) {
#pragma unroll
    for (int i = 0; i < kKL; ++i) {
      const int c = tid + i * kAttnThreads;
      const int n = c / kCpr, dc = c % kCpr;
      const bool ok = n0 + n < end && 8 * dc < D;
      *reinterpret_cast<u32x4_t*>(k_lds + n * kKPitch + 8 * dc) = ok ? kreg[i] : u32x4_t{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4_t*>(v_lds + n * kVPitch + 8 * dc) = ok ? vreg[i] : u32x4_t{0u, 0u, 0u, 0u};
    }
  };

  // Heads over 128 dims have no registers to spare for the next block's data:
  // they load each block right before staging it.
  constexpr bool kPrefetch = DT <= 4;
  if (kPrefetch && start < end) fetch(start);
  for (int n0 = start; n0 < end; n0 += kBlockN) {
    if (!kPrefetch) fetch(n0);
    stage(n0);
    __syncthreads();
    if (kPrefetch && n0 + kBlockN < end) fetch(n0 + kBlockN);

    // ---- S^T = K . Q^T for the two 32-key tiles (two independent MFMA chains)
    v16f s[2] = {v16f{}, v16f{}};
    // all 2 * DT chunks of the padded head: dims past D are zero in Q and K
#pragma unroll
    for (int c = 0; c < 2 * DT; ++c) {
      // at most 4 chunks of K fragments in registers ahead of their MFMAs
      if (c % 4 == 0) asm volatile("" ::: "memory");
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const u32x4_t kf = *reinterpret_cast<const u32x4_t*>(k_lds + (32 * t + col) * kKPitch + 16 * c + 8 * half);
        s[t] = MF::run(kf, qf[c], s[t]);
      }
    }
    // ---- online softmax (log2 domain); lane holds keys n0 + 32t + 8q + 4*half + r
    float mblk = -__builtin_inff();
    if (n0 + kBlockN <= full_below && n0 + kBlockN <= end) {  // workgroup-uniform: no key masked
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          s[t][i] = s[t][i] * a.qk_scale;
          mblk = fmaxf(mblk, s[t][i]);
        }
    } else {
      const int lim_b = min(lim, end) - n0 - 4 * half;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float x = 32 * t + 8 * (i >> 2) + (i & 3) < lim_b ? s[t][i] * a.qk_scale : -__builtin_inff();
          s[t][i] = x;
          mblk = fmaxf(mblk, x);
        }
    }
    mblk = fmaxf(mblk, __shfl_xor(mblk, 32, 64));
    // The reference max only moves when a score exceeds it by more than 2^8
    // (probabilities then stay <= 256, exact in the 16-bit P operand's range),
    // so the accumulators are rarely rescaled; l and O share the reference, so
    // the normalized result is the same.
    const float m_new = mblk > m_run + 8.0f ? fmaxf(m_run, mblk) : m_run;
    const float m_use = m_new == -__builtin_inff() ? 0.0f : m_new;
    float psum = 0.0f;
    uint32_t pk[2][2][4];  // [tile][q0 pair][packed pairs]
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const float p0 = __builtin_amdgcn_exp2f(s[t][i] - m_use), p1 = __builtin_amdgcn_exp2f(s[t][i + 1] - m_use);
        psum = psum + p0 + p1;
        pk[t][i >> 3][(i & 7) >> 1] = MF::pack2(p0, p1);
      }
    // rescale only when some row's reference moved (the rescale is by 1 otherwise)
    if (__any(m_new != m_run)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      l_run = l_run * alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] = acc[dt][i] * alpha;
    }
    l_run = l_run + psum;
    m_run = m_new;

    // ---- O^T += V^T . P^T: 16 keys per MFMA (tile t, q0 pair); DT independent chains.
    // The V^T operand of lane L (16-lane group g = L / 16, j = L % 16): head dim
    // 32dt + 16(g % 2) + j, keys kb..kb+3 and kb+8..kb+11, kb = 32t + 16qp + 4(g / 2).
    {
      const int g = lane >> 4, j = lane & 15;
      const int vr = 4 * (g >> 1) + (j >> 2), vc = 16 * (g & 1) + 4 * (j & 3);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int qp = 0; qp < 2; ++qp) {
          if (DT > 4) asm volatile("" ::: "memory");  // bound the V fragments read ahead (registers)
          const u32x4_t pf = u32x4_t{pk[t][qp][0], pk[t][qp][1], pk[t][qp][2], pk[t][qp][3]};
          const uint16_t* vbk = v_lds + (32 * t + 16 * qp + vr) * kVPitch + vc;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const u32x2_t lo = lds_read_tr16(vbk + 32 * dt);
            const u32x2_t hi = lds_read_tr16(vbk + 8 * kVPitch + 32 * dt);
            acc[dt] = MF::run(u32x4_t{lo[0], lo[1], hi[0], hi[1]}, pf, acc[dt]);
          }
        }
    }
    __syncthreads();  // the LDS block is refilled next
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (a.splits > 1) {
    // Partial rows are stored normalized by their own l, in the operands'
    // 16-bit type (|O/l| <= max |V|; half the bytes of fp32 to write here and to
    // read in the combine). They leave through LDS, 32 head dims at a time: each
    // wave writes its 32 x 32 block there (lane = query row) and stores it back
    // row-major, 16 rows x 64 contiguous bytes per store instruction instead of
    // 32 rows x 16 bytes. The block buffers are free after the loop.
    const int64_t wrow0 = static_cast<int64_t>(blockIdx.x) * kRowsPerWg + wave * 32;
    const int64_t pbase = ((static_cast<int64_t>(split) * gridDim.z + b) * a.Hkv + kvh) * a.n_rows;
    if (row_ok && half == 0) {
      a.pm[pbase + row] = m_run;
      a.pl[pbase + row] = l_tot;
    }
    constexpr int kTp16 = 20;  // 32-bit words per LDS row: 16 (32 dims) + 4 (16-byte aligned rows)
    uint32_t* tb = reinterpret_cast<uint32_t*>(kv_lds) + wave * 32 * kTp16;
    const float inv_l = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    const int sr = lane >> 2, sc = 4 * (lane & 3);  // store: rows sr + 16k, words sc..sc+3 (dims 2sc..)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<u32x2_t*>(tb + col * kTp16 + 4 * q + 2 * half) =
            u32x2_t{MF::pack2(acc[dt][4 * q] * inv_l, acc[dt][4 * q + 1] * inv_l),
                    MF::pack2(acc[dt][4 * q + 2] * inv_l, acc[dt][4 * q + 3] * inv_l)};
      u32x4_t v[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) v[k] = *reinterpret_cast<const u32x4_t*>(tb + (sr + 16 * k) * kTp16 + sc);
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int64_t r = wrow0 + sr + 16 * k;
        if (r < a.n_rows) *reinterpret_cast<u32x4_t*>(a.po + (pbase + r) * kDP + 32 * dt + 2 * sc) = v[k];
      }
    }
    return;
  }
  if (!row_ok) return;
  const float inv = 1.0f / l_tot;
  uint16_t* orow = a.o + b * a.sob + tok * a.sot + head * a.soh;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int d = 32 * dt + 8 * q + 4 * half;
      if (d < D) {
        const uint32_t w0 = MF::pack2(acc[dt][4 * q] * inv, acc[dt][4 * q + 1] * inv);
        const uint32_t w1 = MF::pack2(acc[dt][4 * q + 2] * inv, acc[dt][4 * q + 3] * inv);
        *reinterpret_cast<u32x2_t*>(orow + d) = u32x2_t{w0, w1};
      }
    }
}

// Split-KV combine for one (batch, token): merge the partial softmax states of
// every head of the token, write O (optional) and, with q8, quantize the whole
// token row [Hq * D] per token (this package's recipe). The per-(head, split)
// weights exp2(m_s - m) / l are formed once in LDS; the row's values stay in
// registers between the two passes (Hq * D <= 256 * kCombineVpt).
constexpr int kCombineVpt = 32;
constexpr int kCombineMaxW = 1024;  // Hq * splits

// ks > 0: q8 in the skinny tile layout (ks K steps; the grid covers 16*ceil(Tq/16)
// token rows and the padding rows / K padding are written as zeros).
template <bool BF16, int NT>
__global__ __launch_bounds__(NT) void attn_combine_kernel(AttnArgs a, int64_t kdp, int64_t Hq,
                                                                    uint8_t* q8, int64_t ldq8, float* q8s, int64_t ks,
                                                                    int64_t Tq) {
  using MF = Mfma<BF16>;
  __shared__ uint32_t red[NT / 64];
  __shared__ float wgt[kCombineMaxW];
  const int64_t b = blockIdx.x;
  const int64_t tok = blockIdx.y;
  const int D = static_cast<int>(a.D);
  const int S = a.splits;
  const int H = static_cast<int>(Hq);
  if (tok >= Tq) {  // tile-layout padding row (workgroup-uniform)
    for (int64_t i = threadIdx.x; i < ks * 16; i += NT)
      *reinterpret_cast<uint2*>(q8 + tile_offset(tok, 8 * i, ks)) = make_uint2(0u, 0u);
    return;
  }
  const int64_t nb = gridDim.x;
  // per (head, split): the partial row's index, its softmax state in LDS
  __shared__ float pl_s[kCombineMaxW];
  __shared__ int64_t off_s[kCombineMaxW];
  for (int i = threadIdx.x; i < H * S; i += NT) {
    const int h = i / S, sp = i - (i / S) * S;
    const int64_t pr = ((sp * nb + b) * a.Hkv + h / a.group) * a.n_rows + tok * a.group + h % a.group;
    off_s[i] = pr * kdp;
    wgt[i] = a.pm[pr];
    pl_s[i] = a.pl[pr];
  }
  __syncthreads();
  // per head: the max over splits, then the normalized split weights
  for (int h = threadIdx.x; h < H; h += NT) {
    float m = -__builtin_inff();
    for (int sp = 0; sp < S; ++sp) m = fmaxf(m, wgt[h * S + sp]);
    float l = 0.0f;
    for (int sp = 0; sp < S; ++sp) {
      const float w = __builtin_amdgcn_exp2f(wgt[h * S + sp] - m);
      wgt[h * S + sp] = w;
      l = l + w * pl_s[h * S + sp];
    }
    const float inv = 1.0f / l;
    // the stored partials are O_s / l_s: weight exp2(m_s - m) * l_s / l
    for (int sp = 0; sp < S; ++sp) wgt[h * S + sp] = wgt[h * S + sp] * pl_s[h * S + sp] * inv;
  }
  __syncthreads();
  // the merged row in groups of 4 head dims; the partials of up to 16 splits of
  // a group are loaded together (addresses clamped, weights zeroed past S)
  constexpr int kG = kCombineVpt / 4;  // groups per thread
  const int groups = H * D / 4;
  float4 val[kG];
  uint32_t amax = 0;
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    const int e4 = threadIdx.x + j * NT;
    val[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e4 >= groups) continue;
    const int h = (4 * e4) / D, d = 4 * e4 - h * D;
    float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < S; s0 += 16) {
      float4 pv[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int sp = min(s0 + u, S - 1);
        const u32x2_t r = *reinterpret_cast<const u32x2_t*>(a.po + off_s[h * S + sp] + d);
        pv[u] = make_float4(MF::to_f32(static_cast<uint16_t>(r[0])), MF::to_f32(static_cast<uint16_t>(r[0] >> 16)),
                            MF::to_f32(static_cast<uint16_t>(r[1])), MF::to_f32(static_cast<uint16_t>(r[1] >> 16)));
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float w = s0 + u < S ? wgt[h * S + s0 + u] : 0.0f;
        o4.x = o4.x + w * pv[u].x;
        o4.y = o4.y + w * pv[u].y;
        o4.z = o4.z + w * pv[u].z;
        o4.w = o4.w + w * pv[u].w;
      }
    }
    val[j] = o4;
    if (a.o) {
      uint16_t* op = a.o + b * a.sob + tok * a.sot + h * a.soh + d;
      *reinterpret_cast<uint2*>(op) = make_uint2(MF::pack2(o4.x, o4.y), MF::pack2(o4.z, o4.w));
    }
    const uint32_t m1 = max(abs_bits(o4.x), abs_bits(o4.y)), m2 = max(abs_bits(o4.z), abs_bits(o4.w));
    amax = max(amax, max(m1, m2));
  }
  if (!q8) return;  // uniform
  amax = wave_max_u32(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) amax = amax > red[w] ? amax : red[w];
  const float sc = scale_from_amax_bits(amax);
  if (threadIdx.x == 0) q8s[tok] = sc;
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    const int e4 = threadIdx.x + j * NT;
    if (e4 < groups) {
      uint8_t* qp = ks > 0 ? q8 + tile_offset(tok, 4 * e4, ks) : q8 + tok * ldq8 + 4 * e4;
      qp[0] = static_cast<uint8_t>(q1(val[j].x, sc));
      qp[1] = static_cast<uint8_t>(q1(val[j].y, sc));
      qp[2] = static_cast<uint8_t>(q1(val[j].z, sc));
      qp[3] = static_cast<uint8_t>(q1(val[j].w, sc));
    }
  }
  if (ks > 0)  // K padding of the tile layout
    for (int64_t i = groups / 2 + threadIdx.x; i < ks * 16; i += NT)
      *reinterpret_cast<uint2*>(q8 + tile_offset(tok, 8 * i, ks)) = make_uint2(0u, 0u);
}

template <bool BF16, int DT>
void launch_attn(const AttnArgs& a, int64_t B, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((a.n_rows + kRowsPerWg - 1) / kRowsPerWg),
                  static_cast<unsigned>(a.Hkv * a.splits), static_cast<unsigned>(B));
  hipLaunchKernelGGL((attn_kernel<BF16, DT>), grid, dim3(kAttnThreads), 0, st, a);
}

template <bool BF16>
void dispatch_attn(const AttnArgs& a, int64_t B, int dt, hipStream_t st) {
  switch (dt) {
    case 1: launch_attn<BF16, 1>(a, B, st); break;
    case 2: launch_attn<BF16, 2>(a, B, st); break;
    case 3: launch_attn<BF16, 3>(a, B, st); break;
    case 4: launch_attn<BF16, 4>(a, B, st); break;
    case 5: launch_attn<BF16, 5>(a, B, st); break;
    case 6: launch_attn<BF16, 6>(a, B, st); break;
    case 7: launch_attn<BF16, 7>(a, B, st); break;
    default: launch_attn<BF16, 8>(a, B, st); break;
  }
}

}  // namespace
}  // namespace ifx

using namespace ifx;

extern "C" {

size_t ifx_attention_workspace_size(int64_t B, int64_t Tq, int64_t Hq, int64_t Hkv, int64_t D, int splits) {
  if (B <= 0 || Tq <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || D <= 0 || D > 256 || splits <= 1) return 0;
  const int64_t rows = static_cast<int64_t>(splits) * B * Hkv * Tq * (Hq / Hkv);
  const int64_t dp = (D + 31) / 32 * 32;
  return static_cast<size_t>(rows) * (dp * sizeof(uint16_t) + 2 * sizeof(float));
}

int ifx_attention(const void* q, const void* k, const void* v, void* o, int dtype, int64_t B, int64_t Tq,
                  int64_t Hq, int64_t Tk, int64_t Hkv, int64_t D, const int64_t* q_strides,
                  const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides, int64_t kv_len,
                  const int32_t* kv_len_dev, const int32_t* kv_extra, int causal, int64_t causal_offset,
                  const int32_t* kv_index, int64_t n_index, float scale, int splits, void* workspace,
                  size_t ws_bytes, void* q8, int64_t ldq8, float* q8_scale, void* stream) {
  if (dtype != IFX_DTYPE_BF16 && dtype != IFX_DTYPE_F16) return IFX_ERR_INVALID;
  if (B < 0 || Tq < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || Tk <= 0 || D <= 0 || D % 8 != 0) return IFX_ERR_INVALID;
  if (D > 256) return IFX_ERR_UNSUPPORTED;
  if (!q_strides || !k_strides || !v_strides || splits < 1 || splits > 64) return IFX_ERR_INVALID;
  if (kv_index && n_index <= 0) return IFX_ERR_INVALID;
  if (kv_len < 0 || causal_offset < -(int64_t(1) << 30) || causal_offset > (int64_t(1) << 30) ||
      Tk > 0x7FFFFFFFLL || n_index > 0x7FFFFFFFLL)
    return IFX_ERR_INVALID;
  if (q8 && (splits < 2 || B != 1 || !q8_scale || (ldq8 != IFX_LD_TILED && ldq8 < Hq * D))) return IFX_ERR_INVALID;
  const int64_t q8_ks = q8 && ldq8 == IFX_LD_TILED ? (Hq * D + 127) / 128 : 0;
  if (q8_ks > 0 && (Tq > 64 || (Hq * D) % 16 != 0 || !aligned16(q8))) return IFX_ERR_UNSUPPORTED;
  if (Hq * D > static_cast<int64_t>(kAttnThreads) * kCombineVpt || Hq * splits > kCombineMaxW)
    return IFX_ERR_UNSUPPORTED;
  if (splits == 1 && !o) return IFX_ERR_INVALID;
  if (splits > 1 && (!workspace || ws_bytes < ifx_attention_workspace_size(B, Tq, Hq, Hkv, D, splits)))
    return IFX_ERR_WORKSPACE;
  if (splits > 1 && !aligned16(workspace)) return IFX_ERR_ALIGN;  // 16-byte partial-row stores
  if (o && !o_strides) return IFX_ERR_INVALID;
  if (B == 0 || Tq == 0) return IFX_OK;
  if (!q || !k || !v) return IFX_ERR_INVALID;
  // 16-byte row pieces: base pointers and every row stride must keep 8-element alignment
  for (const int64_t* s : {q_strides, k_strides, v_strides})
    for (int i = 0; i < 3; ++i)
      if (s[i] % 8 != 0) return IFX_ERR_ALIGN;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v)) return IFX_ERR_ALIGN;
  if (o) {
    for (int i = 0; i < 3; ++i)
      if (o_strides[i] % 4 != 0) return IFX_ERR_ALIGN;
    if (reinterpret_cast<uintptr_t>(o) & 7u) return IFX_ERR_ALIGN;
  }

  const int64_t group = Hq / Hkv;
  const int dt = static_cast<int>((D + 31) / 32);
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = static_cast<uint16_t*>(o);
  a.sqb = q_strides[0]; a.sqt = q_strides[1]; a.sqh = q_strides[2];
  a.skb = k_strides[0]; a.skt = k_strides[1]; a.skh = k_strides[2];
  a.svb = v_strides[0]; a.svt = v_strides[1]; a.svh = v_strides[2];
  if (o) { a.sob = o_strides[0]; a.sot = o_strides[1]; a.soh = o_strides[2]; }
  a.n_rows = Tq * group;
  a.D = D;
  a.n_keys = kv_index ? n_index : Tk;
  a.Tk = Tk;
  a.group = static_cast<int>(group);
  a.Hkv = static_cast<int>(Hkv);
  a.kv_len_static = static_cast<int>(kv_len < a.n_keys ? kv_len : a.n_keys);
  a.kv_len = kv_len_dev;
  a.kv_extra = kv_extra;
  a.causal = causal ? 1 : 0;
  a.causal_offset = static_cast<int>(causal_offset);
  a.kv_index = kv_index;
  a.qk_scale = scale * 1.4426950408889634f;
  a.splits = splits;
  if (splits > 1) {
    const int64_t rows = static_cast<int64_t>(splits) * B * Hkv * a.n_rows;
    a.po = static_cast<uint16_t*>(workspace);
    a.pm = reinterpret_cast<float*>(a.po + rows * 32 * dt);
    a.pl = a.pm + rows;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bf = dtype == IFX_DTYPE_BF16;
  if (bf) dispatch_attn<true>(a, B, dt, st);
  else dispatch_attn<false>(a, B, dt, st);
  if (splits > 1) {
    const dim3 grid(static_cast<unsigned>(B), static_cast<unsigned>(q8_ks > 0 ? (Tq + 15) / 16 * 16 : Tq));
    // Few tokens (fewer workgroups than CUs): one 4-dim group per lane, so more
    // of the partial rows (written by other XCDs) are in flight per CU
    // (pi05 chunk, 51 tokens: 18.8 -> 18.2 us); many tokens: 256 lanes (the
    // 800-token prefix is 4.6 us slower with 512).
    const int64_t groups = B * Tq < 128 ? Hq * D / 4 : 0;
    auto launch = [&](auto bf_tag, auto nt_tag) {
      constexpr bool kBf = decltype(bf_tag)::value;
      constexpr int kNt = decltype(nt_tag)::value;
      hipLaunchKernelGGL((attn_combine_kernel<kBf, kNt>), grid, dim3(kNt), 0, st, a, int64_t(32 * dt), Hq,
                         static_cast<uint8_t*>(q8), ldq8, q8_scale, q8_ks, Tq);
    };
    using std::integral_constant;
    if (bf) {
      if (groups > 512) launch(integral_constant<bool, true>{}, integral_constant<int, 1024>{});
      else if (groups > 256) launch(integral_constant<bool, true>{}, integral_constant<int, 512>{});
      else launch(integral_constant<bool, true>{}, integral_constant<int, 256>{});
    } else {
      if (groups > 512) launch(integral_constant<bool, false>{}, integral_constant<int, 1024>{});
      else if (groups > 256) launch(integral_constant<bool, false>{}, integral_constant<int, 512>{});
      else launch(integral_constant<bool, false>{}, integral_constant<int, 256>{});
    }
  }
  return launch_status();
}

}  // extern "C"
