"""CPU oracle of the FP8 projection path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker (or, for bench.py, as the timed CPU
baseline). The product (instinctflash_amd/) never imports it.

Parts
  * quantizer: plain C restatement (ifx_oracle.c, built by the Makefile here)
    of instinctflash/kernels/fp8.py:30-37 with the device scale arithmetic of
    instinctflash/runtime/fp8_pack.py:63-91. Pinned in tests/test_oracle.py by
    the reference's known-answer scale (tests/test_sm89_fp8.py:48-56), by
    byte-equality with torch's own CPU E4M3 cast over every finite bf16 pattern
    and the reference's fixed midpoint scales (scripts/qualify_sm89_fp8.py:61),
    by NaN/inf propagation, and by a brute-force nearest-value search.
  * e4m3_decode: the OCP E4M3FN value table, pinned against torch's decoder.
  * ref_linear: dequantize-then-fp32-matmul (benchmarks/native/fp8_probe.py:36)
    followed by the epilogue math of kernels/norm.py:45-58,135-144,161-175 and
    kernels/activation.py:26-40. Pinned by fp64 brute force, closed forms and
    torch's independent GELU/SiLU implementations.
  * residual_norm: the pre-norm producer of kernels/norm.py:25-94 (residual
    update in float32 in the reference's operation order, norm in float64).
    Pinned in tests/test_oracle.py by the reference's own test expectation
    (tests/test_gi_kernels.py:93-112: the update equals res + (delta*dr*dc +
    b)*gate to 1e-4, and the rsqrt-normalized row), by closed forms (a constant
    row normalizes to +-1 / 0, unit-RMS rows are fixed points of RMS norm) and by
    torch.nn.functional.layer_norm / rms_norm.
  * qkv_split: the QKV split of kernels/rope.py:21-80 (rescale, per-head q/k
    RMSNorm, rotary with float32 angles). Pinned by the reference's own test
    expectation (tests/test_gi_kernels.py:58-90) evaluated with torch, by the
    rotation invariants (pair norms preserved, position 0 = identity, angle
    additivity) and by unit RMS of normalized heads.
  * wan_qkv: the Wan QKV consumer of kernels/wan.py:19-81 (full-width q/k
    RMSNorm, interleaved-pair rotary). Pinned against qkv_split under the
    channel permutation that turns interleaved pairs into split halves, against
    torch.nn.functional.rms_norm over the full width, and by the rotation
    invariants.
  * moe_router / moe_act: the MoE routing of kernels/activation.py:71-137
    (sigmoid top-k router, routed SwiGLU with per-expert column weights).
    moe_router is pinned by the reference test's own construction
    (tests/test_gi_kernels.py:179-192: torch.topk + scatter + renormalize), by
    a brute-force search over every top_k-subset of experts and by the
    invariants (weights sum to scale, E - top_k zeros, bias moves selection but
    not weights); moe_act by the reference test's repeat_interleave
    construction of the column weights (:193-203), by reduction to the plain
    SwiGLU with unit weights, and by linearity in the routing weight.
  * attention: softmax attention with per-row key limits (kernels/attention.py:
    23-92, split combine :113-147) in float64. Pinned by the reference test's
    own formulation (tests/test_gi_kernels.py:22-30: repeat_interleave of KV
    heads, einsum, masked softmax) evaluated with torch, by
    torch.nn.functional.scaled_dot_product_attention with a boolean mask, and by
    closed forms (one visible key returns its value row; equal scores return
    the mean of the visible value rows).
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libifx_oracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        P, I64 = ctypes.c_void_p, ctypes.c_int64
        lib.oracle_e4m3.restype = ctypes.c_uint8
        lib.oracle_e4m3.argtypes = [ctypes.c_float]
        for name in ("oracle_quant_rows_f32", "oracle_quant_rows_bf16"):
            getattr(lib, name).restype = None
            getattr(lib, name).argtypes = [P, I64, I64, I64, P, I64, P]
        lib.oracle_pack_bf16.restype = None
        lib.oracle_pack_bf16.argtypes = [P, I64, ctypes.c_float, P]
        lib.oracle_quant_tensor_bf16.restype = None
        lib.oracle_quant_tensor_bf16.argtypes = [P, I64, P, P]
        _lib = lib
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------------------
# quantizer
# ---------------------------------------------------------------------------

def quant_rows(x: np.ndarray):
    """x: uint16 (bf16 bit patterns) or float32 [M, K] -> (q uint8 [M, K], scale float32 [M])."""
    x = np.ascontiguousarray(x)
    M, K = x.shape
    q = np.empty((M, K), np.uint8)
    s = np.empty((M,), np.float32)
    if x.dtype == np.uint16:
        load().oracle_quant_rows_bf16(_p(x), K, M, K, _p(q), K, _p(s))
    elif x.dtype == np.float32:
        load().oracle_quant_rows_f32(_p(x), K, M, K, _p(q), K, _p(s))
    else:
        raise TypeError(f"unsupported dtype {x.dtype}")
    return q, s


def pack_fixed(x_bf16: np.ndarray, scale: float) -> np.ndarray:
    x = np.ascontiguousarray(x_bf16.reshape(-1))
    q = np.empty(x.shape, np.uint8)
    load().oracle_pack_bf16(_p(x), x.size, float(scale), _p(q))
    return q.reshape(x_bf16.shape)


def quant_tensor(x_bf16: np.ndarray):
    x = np.ascontiguousarray(x_bf16.reshape(-1))
    q = np.empty(x.shape, np.uint8)
    s = np.empty((1,), np.float32)
    load().oracle_quant_tensor_bf16(_p(x), x.size, _p(q), _p(s))
    return q.reshape(x_bf16.shape), s


def e4m3(values) -> np.ndarray:
    lib = load()
    v = np.asarray(values, np.float32).reshape(-1)
    return np.array([lib.oracle_e4m3(float(f)) for f in v], np.uint8)


# ---------------------------------------------------------------------------
# value tables and conversions
# ---------------------------------------------------------------------------

def _decode_table() -> np.ndarray:
    t = np.empty(256, np.float32)
    for c in range(256):
        sign = -1.0 if c & 0x80 else 1.0
        e, m = (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            t[c] = np.nan
        elif e == 0:
            t[c] = sign * m * 2.0 ** -9
        else:
            t[c] = sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


E4M3_VALUES = _decode_table()


def e4m3_decode(q: np.ndarray) -> np.ndarray:
    return E4M3_VALUES[np.asarray(q, np.uint8)]


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even FP32 -> bf16 bit patterns (NaN kept quiet)."""
    u = np.ascontiguousarray(f, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(f, np.float32))
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


# ---------------------------------------------------------------------------
# GEMM + epilogue
# ---------------------------------------------------------------------------

def gelu_tanh(x):
    x = np.asarray(x, np.float32)
    return (0.5 * x * (1.0 + np.tanh(np.float32(0.7978845608028654) * (x + np.float32(0.044715) * x ** 3)))).astype(np.float32)


def silu(x):
    x = np.asarray(x, np.float32)
    return (x / (1.0 + np.exp(-x))).astype(np.float32)


def ref_linear(qa, sa, qw, sw, bias=None, act=None, residual=None, gate=None, acc_dtype=np.float32):
    """Dequantize-then-matmul reference (benchmarks/native/fp8_probe.py:36).

    qa uint8 [M,K] / sa [M] (None = 1); qw uint8 [N,K] / sw [N] (None = 1), gate|up
    weights in the reference layout (rows [0,F) gate, [F,2F) up). act in
    {None, 'gelu_tanh', 'geglu', 'swiglu'}. gate/residual are float arrays
    (bf16 values widened). Returns float32 [M, N_out] before output rounding.
    """
    a = e4m3_decode(qa).astype(acc_dtype)
    w = e4m3_decode(qw).astype(acc_dtype)
    if sa is not None:
        a = a * np.asarray(sa, acc_dtype)[:, None]
    if sw is not None:
        w = w * np.asarray(sw, acc_dtype)[:, None]
    y = (a @ w.T).astype(np.float32)
    if bias is not None:
        y = y + np.asarray(bias, np.float32)[None, :]
    if act == "gelu_tanh":
        y = gelu_tanh(y)
    elif act in ("geglu", "swiglu"):
        F = y.shape[1] // 2
        g, u = y[:, :F], y[:, F:]
        y = (gelu_tanh(g) if act == "geglu" else silu(g)) * u
    elif act is not None:
        raise ValueError(act)
    if gate is not None:
        y = y * np.asarray(gate, np.float32)[None, :]
    if residual is not None:
        y = np.asarray(residual, np.float32) + y
    return y.astype(np.float32)


def parity_stats(out: np.ndarray, ref: np.ndarray):
    """(max|d| / rms(ref), cosine) -- the GEMM acceptance metrics."""
    o = np.asarray(out, np.float64).reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    rms = float(np.sqrt(np.mean(r * r))) or 1.0
    d = float(np.max(np.abs(o - r))) if o.size else 0.0
    den = float(np.linalg.norm(o) * np.linalg.norm(r))
    cos = float(np.dot(o, r) / den) if den else 1.0
    return d / rms, cos


def residual_norm(res, delta=None, delta_row=None, delta_col=None, bias=None, gate=None, write_res=True,
                  layernorm=False, weight=None, beta=None, mod_scale=None, mod_shift=None, mod_index=None,
                  eps=1e-6, res_bf16=False):
    """Pre-norm producer of instinctflash/kernels/norm.py:25-94, restated.

    res: float32 [M, D] values (for res_bf16, the float32 widening of the bf16
    input). Returns (res_out float32 [M, D], y float64 [M, D]):
      * res_out: the residual update in float32, operation by operation in the
        reference's order (norm.py:46-56): d = delta*row; d = d*col; d = d+bias;
        d = d*gate; x = res + d -- every step one IEEE float32 rounding, so a
        device kernel without contraction reproduces it bit for bit; with
        res_bf16 and write_res the stored value is rounded to bf16 (RNE) and that
        rounded value is normalized (norm.py:56-57);
      * y: the normalization (norm.py:58-66) and affine / adaptive terms
        (:67-74) in float64 from res_out (RMS: x * 1/sqrt(mean(x^2) + eps);
        LayerNorm: (x - mean) * 1/sqrt(mean((x - mean)^2) + eps)).
    gate / mod_scale / mod_shift are [D], or [n, D] tables indexed by mod_index.
    """
    f32 = np.float32
    x = np.asarray(res, dtype=f32).copy()
    M, D = x.shape

    def rows_of(t):
        t = np.asarray(t, dtype=f32)
        if mod_index is None:
            return np.broadcast_to(t.reshape(1, D), (M, D))
        return t.reshape(-1, D)[np.asarray(mod_index, dtype=np.int64)]

    if delta is not None:
        d = np.asarray(delta, dtype=f32).copy()
        if delta_row is not None:
            d = (d * np.asarray(delta_row, dtype=f32)[:, None]).astype(f32)
        if delta_col is not None:
            d = (d * np.asarray(delta_col, dtype=f32)[None, :]).astype(f32)
        if bias is not None:
            d = (d + np.asarray(bias, dtype=f32)[None, :]).astype(f32)
        if gate is not None:
            d = (d * rows_of(gate)).astype(f32)
        x = (x + d).astype(f32)
        if res_bf16 and write_res:
            x = bf16_to_f32(f32_to_bf16(x))
    xd = x.astype(np.float64)
    if layernorm:
        xd = xd - xd.mean(axis=1, keepdims=True)
    y = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + float(f32(eps)))
    if weight is not None:
        y = y * np.asarray(weight, dtype=np.float64)[None, :]
    if beta is not None:
        y = y + np.asarray(beta, dtype=np.float64)[None, :]
    if mod_scale is not None:
        y = y * (1.0 + rows_of(mod_scale).astype(np.float64)) + rows_of(mod_shift).astype(np.float64)
    return x, y


def qkv_split(qkv, HQ, HKV, HD, row=None, col=None, bias=None, inv_freq=None, pos=None, sections=None,
              q_norm=None, k_norm=None, eps=1e-6):
    """QKV split of instinctflash/kernels/rope.py:21-80, restated.

    Rescale in float32 in the reference's order (x*row, *col, +bias); per-head
    RMSNorm of Q and K in float64 (x / sqrt(mean(x^2) + eps) * w); rotary with
    the reference's float32 angle pos[t, section[i]] * inv_freq[i] (:60-64) and
    float64 cos/sin, split-half pairing (i, i + HD/2). Returns float64
    (q [T, HQ, HD], k [T, HKV, HD], v [T, HKV, HD])."""
    f32 = np.float32
    x = np.asarray(qkv, dtype=f32)
    T = x.shape[0]
    if row is not None:
        x = (x * np.asarray(row, f32)[:, None]).astype(f32)
    if col is not None:
        x = (x * np.asarray(col, f32)[None, :]).astype(f32)
    if bias is not None:
        x = (x + np.asarray(bias, f32)[None, :]).astype(f32)
    x = x.astype(np.float64).reshape(T, HQ + 2 * HKV, HD)
    qk = x[:, :HQ + HKV]
    if q_norm is not None:
        rs = 1.0 / np.sqrt((qk * qk).mean(axis=2, keepdims=True) + float(f32(eps)))
        w = np.concatenate([np.broadcast_to(np.asarray(q_norm, np.float64), (HQ, HD)),
                            np.broadcast_to(np.asarray(k_norm, np.float64), (HKV, HD))])
        qk = qk * rs * w[None]
    if inv_freq is not None:
        half = HD // 2
        sec = np.zeros(half, np.int64) if sections is None else np.asarray(sections, np.int64)
        p = np.asarray(pos, f32)[:, sec]                                   # [T, half]
        ang = (p * np.asarray(inv_freq, f32)[None, :]).astype(f32).astype(np.float64)
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        lo, hi = qk[..., :half], qk[..., half:]
        qk = np.concatenate([lo * c - hi * s, hi * c + lo * s], axis=2)
    v = x[:, HQ + HKV:]
    return qk[:, :HQ], qk[:, HQ:], v


def wan_qkv(raw, heads, head_dim, tokens, parts=3, row=None, col=None, bias=None, q_norm=None, k_norm=None,
            inv_freq=None, pos=None, sections=None, eps=1e-6):
    """Wan QKV consumer of instinctflash/kernels/wan.py:19-81, restated.

    Per part p (0 = Q, 1 = K, 2 = V; columns p*D..(p+1)*D): rescale in float32 in
    the reference's order (x*row, *col, +bias); Q and K RMS-normalized over the
    full width D in float64 (x / sqrt(mean(x^2) + eps) * w); Q and K rotated on
    adjacent pairs (2j, 2j+1) of every head with the float32 angle
    pos[t, section[j]] * inv_freq[j], t = row % tokens. Returns float64 parts
    [rows, D] in order."""
    f32 = np.float32
    H, HD = heads, head_dim
    D = H * HD
    x = np.asarray(raw, dtype=f32)[:, :parts * D]
    rows = x.shape[0]
    if row is not None:
        x = (x * np.asarray(row, f32)[:, None]).astype(f32)
    if col is not None:
        x = (x * np.asarray(col, f32)[None, :parts * D]).astype(f32)
    if bias is not None:
        x = (x + np.asarray(bias, f32)[None, :parts * D]).astype(f32)
    out = []
    t = np.arange(rows) % tokens
    for p in range(parts):
        xp = x[:, p * D:(p + 1) * D].astype(np.float64)
        w = (q_norm if p == 0 else k_norm) if p < 2 else None
        if w is not None:
            xp = xp / np.sqrt((xp * xp).mean(axis=1, keepdims=True) + float(f32(eps))) * np.asarray(w, np.float64)
        if inv_freq is not None and p < 2:
            half = HD // 2
            sec = np.zeros(half, np.int64) if sections is None else np.asarray(sections, np.int64)
            ang = (np.asarray(pos, f32)[t][:, sec] * np.asarray(inv_freq, f32)[None, :]).astype(f32).astype(np.float64)
            c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
            y = xp.reshape(rows, H, half, 2)
            e, o = y[..., 0], y[..., 1]
            xp = np.stack([e * c - o * s, e * s + o * c], axis=-1).reshape(rows, D)
        out.append(xp)
    return out


def moe_router(x, gate_w, e_bias, top_k, scale):
    """Sigmoid top-k router of instinctflash/kernels/activation.py:71-88, restated.

    logits = x . gate_w^T and s = sigmoid(logits) in float64; the top_k experts
    by s + e_bias (equal scores: lowest expert index first, as the repeated
    argmax of :82-85) get s / (sum of chosen s + 1e-20) * scale, the others 0.
    Returns (route_w float64 [M, E], sel float64 [M, E] the selection scores)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(gate_w, np.float64)
    sg = 1.0 / (1.0 + np.exp(-(x @ w.T)))
    sel = sg + np.asarray(e_bias, np.float64)[None, :]
    M, E = sel.shape
    out = np.zeros((M, E))
    order = np.argsort(-sel, axis=1, kind="stable")[:, :top_k]
    rows = np.arange(M)[:, None]
    out[rows, order] = sg[rows, order]
    out = out / (out.sum(axis=1, keepdims=True) + 1e-20) * scale
    return out, sel


def moe_act(gu, row, col, route_w, experts, group, n_routed):
    """Routed SwiGLU of instinctflash/kernels/activation.py:103-128, restated in
    float32 in the reference's order: g = gu_g*row*col_g, u = gu_u*row*col_u,
    h = silu(g) * u * wr, wr = route_w[m, min(c // group, experts - 1)] for
    c < n_routed else 1. gu: float32 [M, 2F]. Returns h float32 [M, F]."""
    f32 = np.float32
    gu = np.asarray(gu, f32)
    F = gu.shape[1] // 2
    r = np.asarray(row, f32)[:, None]
    c = np.asarray(col, f32)[None, :]
    g = (gu[:, :F] * r).astype(f32) * c[:, :F]
    u = (gu[:, F:] * r).astype(f32) * c[:, F:]
    cols = np.arange(F)
    grp = np.minimum(cols // group, experts - 1)
    wr = np.where(cols[None, :] < n_routed, np.asarray(route_w, f32)[:, grp], f32(1.0)).astype(f32)
    return ((silu(g.astype(f32)) * u).astype(f32) * wr).astype(f32)


def attention(q, k, v, limits, scale, kv_index=None):
    """Attention of instinctflash/kernels/attention.py:23-92, restated in float64.

    q [B, Tq, Hq, D], k / v [B, Tk, Hkv, D] (any float dtype; Hq = group * Hkv,
    query head h reads KV head h // group); limits int [Tq]: token t sees keys
    [0, limits[t]); with kv_index key n is row kv_index[n] of k / v. Returns
    float64 [B, Tq, Hq, D] = softmax(q . k^T * scale) . v over the visible keys."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    if kv_index is not None:
        idx = np.asarray(kv_index, np.int64)
        k, v = k[:, idx], v[:, idx]
    B, Tq, Hq, D = q.shape
    g = Hq // k.shape[2]
    kk = np.repeat(k, g, axis=2)
    vv = np.repeat(v, g, axis=2)
    s = np.einsum("bqhd,bkhd->bhqk", q, kk) * scale
    n = np.arange(kk.shape[1])
    visible = n[None, :] < np.asarray(limits)[:, None]
    s = np.where(visible[None, None], s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.einsum("bhqk,bkhd->bqhd", p, vv)
