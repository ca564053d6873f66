/*
 * ifx_fp8.h -- C ABI of the MI355X (gfx950) FP8 projection path.
 *
 * One shared library (libifx_fp8.so) exports these entry points. Every pointer
 * argument is a DEVICE pointer except where noted; `stream` is a hipStream_t
 * (NULL = the null stream). No entry point allocates memory, synchronises the
 * host, or keeps mutable global state: the caller owns every buffer, so a call
 * may be captured into a HIP graph. (The one exception, ifx_quant_linear_noalloc,
 * works in a fixed scratch array that the library holds per GPU.) Calls on distinct streams are independent,
 * except that a workspace buffer must not be shared by calls that may overlap.
 *
 * Return value: IFX_OK (0), a negative IFX_ERR_* for an argument the library
 * rejects before launching anything, or a positive hipError_t from the launch.
 *
 * Data formats
 *   e4m3  : OCP FP8 E4M3FN bytes (torch.float8_e4m3fn), NaN = 0x7F/0xFF.
 *   bf16  : bfloat16 bit patterns.
 *   scale : float32. Row m of a quantized tensor dequantizes as q[m,:] * scale[m].
 *   Strides (ld*) are in ELEMENTS of the tensor they describe.
 *
 * The quantization recipe (reference: instinctflash/kernels/fp8.py:30-37, with
 * the device scalar-division semantics pinned by instinctflash/runtime/
 * fp8_pack.py:83-91 and tests/test_sm89_fp8.py:48-56) is, per row m:
 *   amax[m]  = max_k |x[m,k]|            (NaN if any element is NaN)
 *   scale[m] = max(amax[m], 1e-12f) * fl32(1/448)
 *   q[m,k]   = e4m3_rne(clamp(x[m,k] / scale[m], -448, 448))   (IEEE division)
 */
#ifndef IFX_FP8_H
#define IFX_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IFX_ABI_VERSION 3

/* status codes (negative = rejected before launch) */
#define IFX_OK 0
#define IFX_ERR_INVALID (-1)     /* a size, stride or flag is out of contract   */
#define IFX_ERR_ALIGN (-2)       /* a pointer/stride breaks 16-byte alignment    */
#define IFX_ERR_WORKSPACE (-3)   /* workspace missing or smaller than required   */
#define IFX_ERR_UNSUPPORTED (-4) /* shape not supported by any kernel variant    */
#define IFX_ERR_SCRATCH (-5)     /* needs more than the library's fixed scratch  */

/* source dtypes for the quantizers */
#define IFX_DTYPE_BF16 0
#define IFX_DTYPE_F32 1
#define IFX_DTYPE_F16 2 /* outputs of ifx_qkv_split; ifx_attention operands */

/* activation selector for gated_act_quant (reference kernels/activation.py:15-16) */
#define IFX_ACT_GELU_TANH 0
#define IFX_ACT_SILU 1

/* fp8_linear epilogue flags (bitmask). Evaluation order per output element:
 *   y = acc[m,n] * sa[m] * sw[n]                     (sa / sw NULL => 1)
 *   y = y + bias[n]                                  IFX_EPI_BIAS
 *   y = gelu_tanh(y)                                 IFX_EPI_GELU_TANH
 *   h = act(y_gate) * y_up                           IFX_EPI_GEGLU / IFX_EPI_SWIGLU
 *       (weights packed with gate/up rows interleaved in blocks of 16, output
 *        width N/2; see ifx_fp8_pack_glu)
 *   y = y * gate[n]                                  IFX_EPI_GATE   (adaLN gate, bf16 [N_out])
 *   y = residual[m,n] + y                            IFX_EPI_RESIDUAL
 *   out[m,n] = round(y)                              bf16; f32 with IFX_EPI_OUT_F32, fp16 with IFX_EPI_OUT_F16
 * residual is bf16 unless IFX_EPI_RES_F32. out may alias residual (in-place update).
 * IFX_EPI_SCALAR_SA / IFX_EPI_SCALAR_SW: sa / sw point to ONE f32 shared by all
 * tokens / weight rows (per-tensor scales, reference runtime/torch_fp8_linear.py:75-78).
 */
#define IFX_EPI_NONE 0
#define IFX_EPI_BIAS 1
#define IFX_EPI_GELU_TANH 2
#define IFX_EPI_GEGLU 4
#define IFX_EPI_SWIGLU 8
#define IFX_EPI_RESIDUAL 16
#define IFX_EPI_GATE 32
#define IFX_EPI_OUT_F32 64
#define IFX_EPI_RES_F32 128
#define IFX_EPI_SCALAR_SA 256
#define IFX_EPI_SCALAR_SW 512
/* w is in the skinny tile layout written by ifx_fp8_pack_skinny (M <= 64 only;
 * ldw is ignored). Not an epilogue option, but carried in the same flags. */
#define IFX_EPI_W_TILED 1024
/* a is in the skinny tile layout written by ifx_quant_rows_tiled (M <= 64 only;
 * lda is ignored). */
#define IFX_EPI_A_TILED 2048
/* out is fp16 (the attention operands of the GR00T / SigLIP engines; not with IFX_EPI_OUT_F32). */
#define IFX_EPI_OUT_F16 4096

int ifx_abi_version(void);
/* Host pointer to a static string describing a status code. */
const char* ifx_status_string(int status);

/*
 * Per-row dynamic quantization of x [M,K] (bf16 or f32) to e4m3 q [M,K] and
 * scale [M] with the recipe above.
 * Replaces: the activation quantizer the engines run before every FP8 GEMM
 * (reference instinctflash/kernels/norm.py:127-158 `row_quant`, recipe of
 * kernels/fp8.py:30-37) and, with IFX_DTYPE_F32, `quantize_weight`'s per-output-
 * channel pass (kernels/fp8.py:30-37; rows = output channels).
 */
int ifx_quant_rows(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                   void* q, int64_t ldq, float* scale, void* stream);

/*
 * Whole-tensor (per-tensor) dynamic quantization of a contiguous bf16 tensor of
 * `count` elements: one scale for all elements, same recipe, NaN anywhere =>
 * NaN scale. `partial` is a caller-provided device workspace of
 * ifx_quant_tensor_workspace_size(count) bytes.
 * Replaces: instinctflash/runtime/fp8_pack.py:83-91 `dynamic_pack_bf16_e4m3`.
 */
size_t ifx_quant_tensor_workspace_size(int64_t count);
int ifx_quant_tensor_bf16(const void* x, int64_t count, void* q, float* scale, void* partial,
                          size_t partial_bytes, void* stream);

/*
 * Pack a contiguous bf16 tensor with a FIXED device scale (one f32 element):
 * q[i] = e4m3_rne(clamp(x[i] / *scale, -448, 448)).
 * Replaces: instinctflash/runtime/fp8_pack.py:48-60 `pack_bf16_e4m3`.
 */
int ifx_pack_tensor_bf16(const void* x, int64_t count, const float* scale, void* q, void* stream);

/*
 * Row stride value selecting the skinny tile layout of ifx_quant_rows_tiled for
 * the e4m3 output of ifx_row_quant, ifx_gated_act_quant, ifx_moe_act_quant,
 * ifx_residual_norm_quant and ifx_attention's q8 (M <= 64 rows, K % 16 == 0,
 * 16-byte aligned; ifx_quant_rows_tiled_bytes(M, K) bytes): the layout the
 * M <= 64 GEMM reads with 1 KB contiguous loads (IFX_EPI_A_TILED).
 */
#define IFX_LD_TILED 0

/* Flags of ifx_row_quant. */
#define IFX_RQ_GELU 1 /* gelu_tanh after the affine terms */
#define IFX_RQ_F16 2  /* x holds fp16 (default bf16) */
#define IFX_RQ_F32 4  /* x holds float32 (the GR00T engine's encoder rows, engines/groot_n17/engine.py:144) */

/*
 * Consumer-side producer of the next FP8 operand from a raw bf16 (or fp16,
 * float32) accumulator:
 *   v = x[m,k] * row[m] * col[k] + bias[k]   (NULL factors are skipped)
 *   v = gelu_tanh(v) with IFX_RQ_GELU
 *   (q[m,:], scale[m]) = quantize(v) with the recipe above (FP32 v, no bf16 rounding).
 * Replaces: instinctflash/kernels/norm.py:150-158 `row_quant` (which the pi05
 * engine also applies to its fp16 attention output, engines/pi05/engine.py:205).
 */
int ifx_row_quant(const void* x, int64_t ldx, int64_t M, int64_t K, const float* row,
                  const float* col, const float* bias, int flags, void* q, int64_t ldq,
                  float* scale, void* stream);

/*
 * Gated activation + requantization from a raw bf16 gate|up accumulator gu [M,2F]:
 *   g = gu[m,f]*row[m]*col[f], u = gu[m,F+f]*row[m]*col[F+f], h = act(g)*u
 *   (q[m,:F], scale[m]) = quantize(h) with the recipe above.
 * Replaces: instinctflash/kernels/activation.py:46-56 `gated_act_quant`.
 */
int ifx_gated_act_quant(const void* gu, int64_t ldgu, int64_t M, int64_t F, const float* row,
                        const float* col, int act, void* q, int64_t ldq, float* scale, void* stream);

/*
 * Routed SwiGLU of a concatenated-experts gate|up accumulator gu [M, 2F] (bf16):
 *   h[m,k] = silu(g * row[m] * col[k]) * (u * row[m] * col[F+k]) * wr
 *   wr = route_w[m, min(k / group, E-1)] for k < n_routed, 1 for k >= n_routed
 *   (the shared expert's columns); q, scale = per-row E4M3 of h (recipe of
 *   ifx_quant_rows). row [M] / col [2F] f32 or NULL; route_w f32 [M, E].
 * Replaces: instinctflash/kernels/activation.py:131-137 `moe_act_quant`
 * (kernel :103-128), with this package's quantization recipe.
 */
int ifx_moe_act_quant(const void* gu, int64_t ldgu, int64_t M, int64_t F, const float* row, const float* col,
                      const float* route_w, int64_t E, int64_t group, int64_t n_routed, void* q, int64_t ldq,
                      float* scale, void* stream);

/*
 * y[m,d] = x[m,d] * row[m] * col[d] + bias[d] in float32 (one rounding per
 * operation, in that order); x and y each bf16, f16 or f32 (x_dtype, y_dtype).
 * Replaces: instinctflash/kernels/norm.py:178-185 `dequant_rows` (any float dtypes).
 */
int ifx_dequant_rows(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t D, const float* row,
                     const float* col, const float* bias, void* y, int y_dtype, int64_t ldy,
                     void* stream);

/*
 * FP8 x FP8 GEMM with fp32 accumulation and fused epilogue:
 *   acc[m,n] = sum_k a[m,k] * w[n,k]      a e4m3 [M,K] (lda), w e4m3 [N,K] (ldw)
 *   out = epilogue(acc)  (flags above; out [M, N_out], N_out = N/2 for GLU else N)
 * Contract: N % 16 == 0 (N % 32 for GLU), K % 16 == 0, a/w/out 16-byte aligned,
 * lda/ldw multiples of 16, ldo/ldr multiples of 8. sa: f32 [M] or NULL,
 * sw: f32 [N] or NULL, bias: f32 [N] or NULL, gate: bf16 [N_out] or NULL.
 * workspace: at least ifx_fp8_linear_workspace_size(M,N,K,epilogue) bytes of
 * 16-byte aligned device memory, used when the GEMM (M > 64) splits K across
 * workgroups because it has too few output tiles to fill the GPU: the slices'
 * fp32 partial sums, added by a second launch. The size is 0 (NULL allowed)
 * otherwise, and always for M <= 64. No initialisation is needed; one
 * workspace serves any sequence of calls and shapes. Calls that may overlap
 * must not share a workspace.
 * With sa = sw = NULL and epilogue 0 this is the raw-accumulator GEMM of
 * instinctflash/kernels/fp8.py:50-53 `gemm` (torch._scaled_mm with unit scales,
 * bf16 out). With scales and flags it fuses the consumers
 * kernels/norm.py:161-175 (dequant_rows), :45-58 (residual/gated residual),
 * :135-144 (gelu), kernels/activation.py:26-40 (GeGLU/SwiGLU),
 * kernels/rope.py:36-45 and kernels/wan.py:27-31 (rescale + bias).
 */
size_t ifx_fp8_linear_workspace_size(int64_t M, int64_t N, int64_t K, int epilogue);
int ifx_fp8_linear(const void* a, int64_t lda, const float* sa, const void* w, int64_t ldw,
                   const float* sw, const float* bias, const void* residual, int64_t ldr,
                   const void* gate, int epilogue, void* out, int64_t ldo, int64_t M, int64_t N,
                   int64_t K, void* workspace, size_t ws_bytes, void* stream);

/* Flags of ifx_residual_norm_quant. */
#define IFX_RNQ_WRITE_RES 1 /* store the updated residual (only with delta) */
#define IFX_RNQ_LAYERNORM 2 /* mean-centred LayerNorm instead of RMS norm */

/*
 * Pre-norm producer, one pass per row of res [M, D] (res_dtype F32 or BF16,
 * row stride ldres elements):
 *   if delta:  x = res + (delta * delta_row[m] * delta_col + bias) * gate,
 *              stored back to res in its dtype with IFX_RNQ_WRITE_RES (the
 *              stored value is the one normalized), else x = res
 *   y = x / sqrt(mean(x^2) + eps)                  (RMS), or with IFX_RNQ_LAYERNORM
 *   y = (x - mean) / sqrt(mean((x - mean)^2) + eps)
 *   y = y * weight + beta;  y = y * (1 + mod_scale) + mod_shift
 *   q, q_scale = per-row E4M3 of y (recipe of ifx_quant_rows); y stored if y != NULL
 * delta: [M, D] BF16 or F32 raw accumulator (NULL: no residual update).
 * delta_row [M], delta_col/bias/weight/beta [D]: f32, each may be NULL.
 * gate, mod_scale, mod_shift: f32 [D], or tables [n, D] whose row mod_index[m]
 * (int32 [M]) is used when mod_index != NULL; mod_scale and mod_shift come
 * together. q: e4m3 [M, ldq] (NULL: no quantization; q_scale [M] f32 then).
 * D % 8 == 0, D <= 16384; res/delta/y 16-byte aligned with row strides that
 * are multiples of 8 elements; vectors 16-byte aligned.
 * Replaces: instinctflash/kernels/norm.py:97-123 `residual_norm_quant` (kernel
 * :25-94), with this package's quantization recipe (1e-12 floor, reciprocal
 * scale, IEEE division) instead of the Triton 1e-8 floor / 448/amax multiply.
 * MoE router option (norm.py:84-94): with router_w != NULL the routing weights
 * of ifx_moe_router are computed from the FP32 y row (before any bf16 store)
 * and written to route_w [M, router_E]; router_bias [router_E] f32,
 * router_E <= 256. Equal to ifx_moe_router on an F32 y, bit for bit.
 */
int ifx_residual_norm_quant(void* res, int res_dtype, int64_t ldres, const void* delta, int delta_dtype,
                            int64_t lddelta, const float* delta_row, const float* delta_col, const float* bias,
                            const float* gate, const float* weight, const float* beta, const float* mod_scale,
                            const float* mod_shift, const int32_t* mod_index, int flags, float eps, void* q,
                            int64_t ldq, float* q_scale, void* y, int y_dtype, int64_t ldy, const float* router_w,
                            const float* router_bias, float* route_w, int64_t router_E, int router_top_k,
                            float router_scale, int64_t M, int64_t D, void* stream);

/*
 * Sigmoid top-k MoE router over x [M, D] (BF16 or F32, row stride ldx):
 *   logits = x . gate_w^T (gate_w f32 [E, D]); s = 1 / (1 + exp(-logits))
 *   the top_k experts by s + e_bias (e_bias f32 [E]; equal values: lowest
 *   expert index first) get route_w[m, e] = s[e] / (sum of chosen s + 1e-20) * scale,
 *   every other expert 0.  route_w f32 [M, E].  D <= 16384, E <= 256.
 * Replaces: instinctflash/kernels/activation.py:91-100 `moe_router` (kernel :71-88).
 */
int ifx_moe_router(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t D, const float* gate_w,
                   const float* e_bias, float* route_w, int64_t E, int top_k, float scale, void* stream);

/*
 * Split a fused QKV accumulator qkv [T, (HQ + 2*HKV) * HD] (BF16 or F32, row
 * stride ldqkv) into Q, K, V heads:
 *   x = qkv * row[t] * col + bias            (row [T], col/bias [(HQ+2HKV)*HD] f32; each may be NULL)
 *   Q, K heads: x = x / sqrt(mean(x^2) + eps) * q_norm|k_norm  (per head; both NULL or both [HD])
 *   Q, K heads: rotary on pairs (i, i + HD/2), angle = pos[t * ldpos + sections[i]] * inv_freq[i]
 *               (f32 pos table, int32 sections [HD/2] or NULL = column 0; inv_freq [HD/2] or NULL = none)
 *   store Q at q_out[t*sq_t + h*sq_h + d], K / V at k_out / v_out[(kv_base + t)*s*_t + h*s*_h + d]
 * out_dtype: IFX_DTYPE_BF16, IFX_DTYPE_F16 or IFX_DTYPE_F32 for all three;
 * kv_base_dev: NULL, or a device int32 read in place of kv_base. HD even, <= 256.
 * Replaces: instinctflash/kernels/rope.py:89-116 `qkv_split` (kernel :21-80).
 */
int ifx_qkv_split(const void* qkv, int qkv_dtype, int64_t ldqkv, const float* row, const float* col,
                  const float* bias, const float* q_norm, const float* k_norm, float eps, const float* inv_freq,
                  const float* pos, int64_t ldpos, const int32_t* sections, void* q_out, int64_t sq_t,
                  int64_t sq_h, void* k_out, int64_t sk_t, int64_t sk_h, void* v_out, int64_t sv_t, int64_t sv_h,
                  int out_dtype, int64_t kv_base, const int32_t* kv_base_dev, int64_t T, int64_t HQ, int64_t HKV,
                  int64_t HD, void* stream);

/*
 * FP8 QKV projection with the qkv_split work in the GEMM's epilogue (M <= 64):
 *   y = a . w^T * sa[m] * sw[n] (+ bias[n])           (fp32, never rounded to bf16)
 *   Q, K heads: rotary on pairs (i, i + HD/2), angle = pos[t * ldpos] * inv_freq[i]
 *   Q at q_out[t*sq_t + h*sq_h + d]; K / V at k_out / v_out[(kv_base + t)*s*_t + h*s*_h + d]
 * w [N = (heads_q + 2*heads_kv) * head_dim, K] has its rows reordered per head:
 * packed row 16k + 4g + r of a head holds head dim d + (r & 1) + (r >= 2 ? HD/2 : 0),
 * d = 8k + 2g (sw and bias in the same order); it may then be tiled
 * (IFX_EPI_W_TILED, ifx_fp8_pack_skinny). flags: IFX_EPI_BIAS, IFX_EPI_W_TILED,
 * IFX_EPI_A_TILED only. head_dim % 16 == 0, <= 256; inv_freq NULL = no rotation;
 * kv_base_dev: NULL or a device int32 read in place of kv_base; out_dtype BF16, F16
 * or F32. workspace / ws_bytes: unused (M <= 64 needs none); NULL / 0 allowed.
 * Replaces: the pair ifx_fp8_linear (raw accumulator, reference
 * instinctflash/kernels/fp8.py:50-53 `gemm`) + ifx_qkv_split (reference
 * instinctflash/kernels/rope.py:89-116) at decode / action-chunk sizes; the
 * reference has no single call for it.
 */
int ifx_fp8_linear_qkv_rope(const void* a, int64_t lda, const float* sa, const void* w, int64_t ldw,
                            const float* sw, const float* bias, int flags, const float* pos, int64_t ldpos,
                            const float* inv_freq, int64_t heads_q, int64_t heads_kv, int64_t head_dim,
                            void* q_out, int64_t sq_t, int64_t sq_h, void* k_out, int64_t sk_t, int64_t sk_h,
                            void* v_out, int64_t sv_t, int64_t sv_h, int out_dtype, int64_t kv_base,
                            const int32_t* kv_base_dev, int64_t M, int64_t K, void* workspace, size_t ws_bytes,
                            void* stream);

/*
 * Wan DiT QKV consumer: raw [rows, parts * D] (BF16 or F32, D = heads * head_dim,
 * parts = 1 + (k_pool != NULL) + (v_pool != NULL): Q, then K, then V columns):
 *   x = raw * row[r] * col + bias               (per part, columns of that part)
 *   Q / K: x = x / sqrt(mean(x^2) + eps) * q_norm|k_norm   (over the full D; skipped if NULL)
 *   Q / K: rotary on adjacent pairs (2j, 2j+1) of every head,
 *          angle = pos[t * ldpos + sections[j]] * inv_freq[j] (j < head_dim/2; inv_freq NULL = none)
 *   store Q at q_out[r * sq + c]; K / V at pool[b * s_b + slot * s_s + c], slot = slots[t] (or t)
 * with t = r % tokens, b = r / tokens. As in the reference launch, part 1 is K:
 * a V pool without a K pool is not written. head_dim % 8 == 0, <= 256; D <= 16384;
 * 16-byte aligned bases and strides that are multiples of 8 elements.
 * Replaces: instinctflash/kernels/wan.py:84-116 `wan_qkv` (kernel :19-81).
 */
int ifx_wan_qkv(const void* raw, int raw_dtype, int64_t ldraw, const float* row, const float* col,
                const float* bias, const float* q_norm, const float* k_norm, float eps, const float* inv_freq,
                const float* pos, int64_t ldpos, const int32_t* sections, void* q_out, int64_t sq, void* k_pool,
                int64_t sk_b, int64_t sk_s, void* v_pool, int64_t sv_b, int64_t sv_s, const int32_t* slots,
                int out_dtype, int64_t rows, int64_t tokens, int64_t heads, int64_t head_dim, void* stream);

/* Activation scaling of ifx_quant_linear. */
#define IFX_SCALE_ROW 0    /* one scale per token (row) */
#define IFX_SCALE_TENSOR 1 /* one scale for the whole [M, K] activation */

/*
 * Quantize bf16 activations x [M, K] (row stride ldx elements, ldx % 8 == 0,
 * 16-byte aligned) to E4M3 with the recipe of ifx_quant_rows (IFX_SCALE_ROW) or
 * ifx_quant_tensor_bf16 (IFX_SCALE_TENSOR) into the workspace, then run
 * ifx_fp8_linear on the result with the same weight / epilogue arguments: two
 * launches, the output bit-identical to those two calls in sequence.
 * IFX_SCALE_TENSOR needs ldx == K (else IFX_ERR_UNSUPPORTED).
 * workspace: ifx_quant_linear_workspace_size(...) bytes, 256-byte aligned, no
 * initialisation needed; calls that may overlap must not share one.
 * a_scale: NULL, or [M] f32 (IFX_SCALE_ROW) / [1] f32 (IFX_SCALE_TENSOR) that
 * receives the activation scales. IFX_EPI_SCALAR_SA is rejected (the scale is
 * computed here); IFX_EPI_SCALAR_SW is honoured.
 * Replaces: the body of ThorFP8Linear.forward (runtime/torch_fp8_linear.py:
 * 66-78: dynamic_pack_bf16_e4m3 + torch._scaled_mm with per-tensor scales) and
 * the engines' producer-quant -> gemm pair (kernels/norm.py:150-176 row_quant
 * feeding kernels/fp8.py:50-53 gemm).
 */
size_t ifx_quant_linear_workspace_size(int64_t M, int64_t N, int64_t K, int epilogue, int scale_mode);
int ifx_quant_linear(const void* x, int64_t ldx, int scale_mode, const void* w, int64_t ldw, const float* sw,
                     const float* bias, const void* residual, int64_t ldr, const void* gate, int epilogue,
                     void* out, int64_t ldo, int64_t M, int64_t N, int64_t K, float* a_scale, void* workspace,
                     size_t ws_bytes, void* stream);

/*
 * ifx_quant_rows for M <= 64 rows (K % 16 == 0, K <= 16384) writing q in the
 * skinny tile layout of ifx_fp8_pack_skinny (tokens in place of weight rows:
 * block j = rows 16j..16j+15), zero-filled past M and K, so a following
 * ifx_fp8_linear with IFX_EPI_A_TILED reads 1 KB contiguous per load
 * instruction. Same bytes and scales as ifx_quant_rows, only placed
 * differently. q holds ifx_quant_rows_tiled_bytes(M, K) bytes, 16-byte aligned.
 * No counterpart in the reference (a layout of this build).
 */
size_t ifx_quant_rows_tiled_bytes(int64_t M, int64_t K);
int ifx_quant_rows_tiled(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, void* q, float* scale,
                         void* stream);

/*
 * Repack an e4m3 weight [N, K] (row stride ldw; N % 16 == 0, K % 16 == 0) into
 * the skinny tile layout read by ifx_fp8_linear with IFX_EPI_W_TILED: for each
 * block of 16 rows b and each 128-byte K step s, one contiguous 2 KB tile
 * T[b * ks + s] (ks = ceil(K / 128)); lane l (0..63) of the matrix-core
 * fragment finds its 32 K bytes [32*(l/16), +32) of row 16b + l%16 at tile
 * bytes [16l, 16l+16) and [1024+16l, +16), so every load instruction of the
 * M <= 64 kernel reads 1 KB of contiguous memory. K is zero-padded to 128 * ks.
 * Apply after ifx_fp8_pack_glu for GLU weights (row blocks of the packed
 * order). w_out holds ifx_fp8_skinny_tiled_bytes(N, K) bytes; scales and bias
 * are unchanged. No counterpart in the reference (a layout of this build).
 */
size_t ifx_fp8_skinny_tiled_bytes(int64_t N, int64_t K);
int ifx_fp8_pack_skinny(const void* w, int64_t ldw, int64_t N, int64_t K, void* w_out, void* stream);

/*
 * Repack a gate|up weight (rows [0,F) gate, [F,2F) up; e4m3 [2F,K] + f32 scale
 * [2F] + optional f32 bias [2F]) into the interleaved layout the GLU epilogue
 * reads: packed rows 32j..32j+15 = gate rows 16j..16j+15, rows 32j+16..32j+31 =
 * up rows 16j..16j+15. Device-to-device, F % 16 == 0. bias/bias_out may be NULL.
 * Replaces: the weight layout `gated_act_quant` assumes (kernels/activation.py:24-25).
 */
int ifx_fp8_pack_glu(const void* w, const float* scale, const float* bias, int64_t F, int64_t K,
                     void* w_out, float* scale_out, float* bias_out, void* stream);

/*
 * Attention over q [B, Tq, Hq, D], k / v [B, Tk, Hkv, D] (dtype BF16 or F16,
 * strides in elements given as {batch, token, head}, last dimension contiguous,
 * multiples of 8; D % 8 == 0, D <= 256, Hq % Hkv == 0): grouped-query heads
 * share their KV head (group = Hq / Hkv). Query token t sees keys [0, limit_t):
 *   limit_t = kv_len (or kv_len_dev[0] read on the device when non-NULL)
 *             + kv_extra[t] (int32 [Tq], when non-NULL)
 *             then min(limit_t, t + causal_offset + 1) when causal,
 *   clamped to the addressable keys (Tk, or n_index with kv_index).
 * With kv_index (int32 [n_index]) key n is cache row kv_index[n].
 * o [B, Tq, Hq, D] (o_strides) = softmax(q k^T * scale) v per head.
 * splits > 1 spreads each row block's keys over `splits` workgroups, keeping
 * partial softmax states in `workspace` (ifx_attention_workspace_size bytes,
 * 16-byte aligned (else IFX_ERR_ALIGN), no zero-fill needed; partial rows normalized by their own softmax sum, in the
 * operands' 16-bit type), then merges them; o may then be NULL, and with q8 != NULL
 * (B == 1) every token's full output row [Hq * D] is also quantized per token to
 * e4m3 q8 [Tq, ldq8] with q8_scale [Tq] (this package's recipe, as
 * ifx_quant_rows). Hq * D <= 8192.
 * Replaces: instinctflash/kernels/attention.py:159-213 `attention` (kernel :23-92,
 * combine with fused FP8 output :113-147, SplitWorkspace :150-159).
 */
size_t ifx_attention_workspace_size(int64_t B, int64_t Tq, int64_t Hq, int64_t Hkv, int64_t D, int splits);
int ifx_attention(const void* q, const void* k, const void* v, void* o, int dtype, int64_t B, int64_t Tq,
                  int64_t Hq, int64_t Tk, int64_t Hkv, int64_t D, const int64_t* q_strides,
                  const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides, int64_t kv_len,
                  const int32_t* kv_len_dev, const int32_t* kv_extra, int causal, int64_t causal_offset,
                  const int32_t* kv_index, int64_t n_index, float scale, int splits, void* workspace,
                  size_t ws_bytes, void* q8, int64_t ldq8, float* q8_scale, void* stream);

/*
 * ifx_quant_linear without a workspace argument: the same launches, bit-identical output, but
 * the workspace is a fixed scratch array inside the library
 * (ifx_quant_linear_noalloc_max_bytes() = 64 MiB per GPU, held from the first
 * call on that GPU until the process ends). No allocation of any kind.
 * Rejects with IFX_ERR_SCRATCH a call whose ifx_quant_linear_workspace_size
 * exceeds the scratch (about M * K bytes of e4m3 plus the split-K partials).
 * The scratch is looked up on the CURRENT device (hipGetDevice), which must be
 * the device of `stream` and of every operand. All calls on one GPU share its
 * scratch: calls that may overlap on one GPU (distinct streams without
 * ordering) race and must not be issued. a_scale as for ifx_quant_linear.
 * No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, serving loops and harnesses that forbid hipMalloc).
 */
size_t ifx_quant_linear_noalloc_max_bytes(void);
int ifx_quant_linear_noalloc(const void* x, int64_t ldx, int scale_mode, const void* w, int64_t ldw,
                             const float* sw, const float* bias, const void* residual, int64_t ldr,
                             const void* gate, int epilogue, void* out, int64_t ldo, int64_t M, int64_t N,
                             int64_t K, float* a_scale, void* stream);

/*
 * Measurement helpers (no counterpart in the reference; used by bench.py to
 * record the shader clock under load). ifx_sclk_probe launches one wave that
 * spins for `wall_ticks` ticks of the constant-rate wall clock and writes
 * out[0] = shader-clock cycles elapsed, out[1] = wall-clock ticks elapsed
 * (uint64 [2], device, 16-byte aligned). ifx_wall_clock_khz reports the wall
 * clock's rate (host int) for the current device.
 */
int ifx_sclk_probe(void* out, int64_t wall_ticks, void* stream);
int ifx_wall_clock_khz(int* khz);

#ifdef __cplusplus
}
#endif

#endif /* IFX_FP8_H */
