"""Pins of the CPU oracle (CPU only, no GPU).

The oracle is only trusted because these checks tie it to things it did not
compute itself:
  * the reference's known-answer scale (tests/test_sm89_fp8.py:48-56);
  * torch's own CPU E4M3 cast and the reference's torch formulation of the
    recipe (tests/test_sm89_fp8.py:242-254, tests/test_dynamic_fp8_pack.py:15-18),
    over every finite bf16 pattern, the reference's fixed midpoint scales
    (scripts/qualify_sm89_fp8.py:61), its shapes/magnitudes and non-finite cases;
  * a brute-force nearest-value search over the OCP E4M3 value set;
  * closed forms and torch's independent GELU/SiLU for the GEMM reference;
  * the committed golden fixtures (tests/golden/fp8_golden.npz).
Each check is chosen so that a plausible slip (true division instead of the
reciprocal, ties away from zero, a dropped bias, a transposed operand, swapped
gate/up halves) fails it.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "fp8_golden.npz"
FIXED_SCALES = (1.0, 1.0 + 2.0 ** -23, 1.0 - 2.0 ** -24, 2.0 ** -16, 1.0 / 448.0)


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def all_finite_bf16():
    pat = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    return pat[torch.isfinite(pat)].contiguous()


def torch_recipe(x):
    """The reference recipe in torch CPU ops, with the device scalar semantics."""
    scale = x.float().abs().amax(dim=1).clamp_min(1e-12) * torch.tensor(1.0 / 448.0, dtype=torch.float32)
    q = (x.float() / scale[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).numpy(), scale.numpy()


def nan_equal_bytes(a, b):
    a, b = np.asarray(a, np.uint8), np.asarray(b, np.uint8)
    na, nb = (a & 0x7F) == 0x7F, (b & 0x7F) == 0x7F
    return np.array_equal(na, nb) and np.array_equal(a[~na], b[~nb])


# ---------------------------------------------------------------------------
# scale arithmetic
# ---------------------------------------------------------------------------

def test_known_answer_scale():
    _, s = oracle.quant_rows(bits(torch.full((1, 16), 0.0361328125, dtype=torch.bfloat16)))
    assert s.view(np.uint32)[0] == 0x38A92493
    # true division (the CPU-only form) would give 0x38A92492: the oracle must not.
    assert (np.float32(0.0361328125) / np.float32(448.0)).view(np.uint32) == 0x38A92492


def test_scale_floor_and_zero_rows():
    q, s = oracle.quant_rows(np.zeros((2, 16), np.float32))
    assert np.all(q == 0)
    assert s.view(np.uint32)[0] == (np.float32(1e-12) * (np.float32(1) / np.float32(448))).view(np.uint32)


def test_nonfinite_propagation_matches_torch():
    for bad in (float("nan"), float("inf"), -float("inf")):
        x = torch.ones((4, 64), dtype=torch.bfloat16)
        x[1, 3] = bad
        q, s = oracle.quant_rows(bits(x))
        tq, ts = torch_recipe(x)
        assert np.array_equal(np.isnan(s), np.isnan(ts))
        assert np.array_equal(s[~np.isnan(s)], ts[~np.isnan(ts)])
        assert nan_equal_bytes(q, tq)


# ---------------------------------------------------------------------------
# E4M3 rounding
# ---------------------------------------------------------------------------

def test_decode_table_matches_torch():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    t = oracle.E4M3_VALUES
    assert np.array_equal(np.isnan(t), np.isnan(codes))
    assert np.array_equal(t[~np.isnan(t)], codes[~np.isnan(codes)])


def test_encode_matches_torch_cast_on_all_bf16_and_midpoints():
    fin = all_finite_bf16().float().numpy()
    vals = np.clip(fin, -448, 448)
    # every E4M3 value, the exact midpoints between neighbours and one fp32 ulp either side
    pos = np.unique(oracle.E4M3_VALUES[~np.isnan(oracle.E4M3_VALUES)]).astype(np.float32)
    mids = ((pos[1:].astype(np.float64) + pos[:-1]) / 2).astype(np.float32)
    near = np.concatenate([mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf))])
    vals = np.concatenate([vals, pos, -pos, near, -near]).astype(np.float32)
    ours = oracle.e4m3(vals)
    theirs = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, theirs)


def test_encode_is_nearest_ties_to_even_by_brute_force():
    pos = np.unique(oracle.E4M3_VALUES[~np.isnan(oracle.E4M3_VALUES)]).astype(np.float64)
    pos = pos[pos >= 0]
    rng = np.random.default_rng(7)
    mids = (pos[1:] + pos[:-1]) / 2
    vals = np.concatenate([rng.uniform(0, 448, 4000), 2.0 ** rng.uniform(-14, -6, 2000), mids, pos]).astype(np.float32)
    got = oracle.E4M3_VALUES[oracle.e4m3(vals)].astype(np.float64)
    for v, gv in zip(vals.astype(np.float64), got):
        d = np.abs(pos - v)
        best = pos[d == d.min()]
        if best.size == 2:  # tie: the even code (mantissa LSB 0)
            codes = [int(np.nonzero(oracle.E4M3_VALUES == b)[0][0]) for b in best]
            best = [b for b, c in zip(best, codes) if c % 2 == 0]
        assert gv == best[0], (v, gv, best)


def test_sign_and_special_codes():
    assert list(oracle.e4m3([0.0, -0.0, 448.0, -448.0, 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -10, np.nan])) == \
        [0x00, 0x80, 0x7E, 0xFE, 0x01, 0x00, 0x02, 0x7F]


# ---------------------------------------------------------------------------
# full per-row recipe vs torch's formulation
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape,mag", [((40, 2048), 1.0), ((256, 5120), 1.0), ((1, 16), 0.0),
                                       ((1, 16), 1e-20), ((1, 16), 1e30)])
def test_rows_match_torch_recipe(shape, mag):
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(shape, generator=g) * mag).to(torch.bfloat16)
    q, s = oracle.quant_rows(bits(x))
    tq, ts = torch_recipe(x)
    assert np.array_equal(s.view(np.uint32), ts.view(np.uint32))
    assert np.array_equal(q, tq)


def test_all_bf16_patterns_match_torch_recipe():
    fin = all_finite_bf16()
    for x in (fin.reshape(1, -1), fin.reshape(255, 256)):
        q, s = oracle.quant_rows(bits(x))
        tq, ts = torch_recipe(x)
        assert np.array_equal(s.view(np.uint32), ts.view(np.uint32))
        assert np.array_equal(q, tq)


@pytest.mark.parametrize("scale", FIXED_SCALES)
def test_fixed_scale_pack_matches_torch(scale):
    fin = all_finite_bf16()
    st = torch.tensor([scale], dtype=torch.float32)
    tq = (fin.float() / st).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(oracle.pack_fixed(bits(fin), float(st.item())), tq)


def test_per_tensor_matches_reference_formulation():
    # tests/test_dynamic_fp8_pack.py:15-18, with the device reciprocal scale
    g = torch.Generator().manual_seed(1)
    x = torch.randn((40, 2048), generator=g).to(torch.bfloat16)
    q, s = oracle.quant_tensor(bits(x))
    es = x.abs().amax().float().clamp_min(1e-12).reshape(1) * torch.tensor(1.0 / 448.0)
    eq = (x.float() / es).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert s.view(np.uint32)[0] == es.numpy().view(np.uint32)[0]
    assert np.array_equal(q, eq)


def test_f32_weights_match_quantize_weight_recipe():
    g = torch.Generator().manual_seed(2)
    w = torch.randn((32, 1000), generator=g) * 0.02
    w[4] = 0
    q, s = oracle.quant_rows(w.numpy())
    tq, ts = torch_recipe(w)
    assert np.array_equal(q, tq) and np.array_equal(s.view(np.uint32), ts.view(np.uint32))


# ---------------------------------------------------------------------------
# GEMM reference
# ---------------------------------------------------------------------------

def _small(seed=3, M=6, N=32, K=64):
    g = torch.Generator().manual_seed(seed)
    qa, sa = oracle.quant_rows(bits(torch.randn((M, K), generator=g).to(torch.bfloat16)))
    qw, sw = oracle.quant_rows((torch.randn((N, K), generator=g) * 0.02).numpy())
    return qa, sa, qw, sw, g


def test_ref_linear_matches_fp64_brute_force():
    qa, sa, qw, sw, _ = _small()
    A = oracle.e4m3_decode(qa).astype(np.float64) * sa[:, None]
    W = oracle.e4m3_decode(qw).astype(np.float64) * sw[:, None]
    exact = np.array([[sum(A[m, k] * W[n, k] for k in range(A.shape[1])) for n in range(W.shape[0])]
                      for m in range(A.shape[0])])
    ref = oracle.ref_linear(qa, sa, qw, sw)
    assert np.allclose(ref, exact, rtol=1e-5, atol=1e-6)
    # a transposed operand or missing row scale is caught by the acceptance metric
    bad = oracle.ref_linear(qa, None, qw, sw)
    assert oracle.parity_stats(bad, ref)[0] > 2e-2


def test_ref_linear_identity_closed_form():
    # W = I (scale 1): out = dequantized activations exactly
    K = 32
    qa, sa, _, _, _ = _small(K=K, N=K)
    eye = np.zeros((K, K), np.uint8)
    eye[np.arange(K), np.arange(K)] = 0x38  # e4m3 1.0
    out = oracle.ref_linear(qa, sa, eye, np.ones(K, np.float32))
    assert np.array_equal(out, (oracle.e4m3_decode(qa) * sa[:, None]).astype(np.float32))


def test_activations_match_torch():
    x = np.linspace(-8, 8, 4001, dtype=np.float32)
    tg = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    ts = torch.nn.functional.silu(torch.from_numpy(x)).numpy()
    assert np.allclose(oracle.gelu_tanh(x), tg, rtol=1e-5, atol=1e-6)
    assert np.allclose(oracle.silu(x), ts, rtol=1e-5, atol=1e-6)
    assert oracle.gelu_tanh(np.float32(0.0)) == 0.0


def test_glu_halves_and_epilogue_order():
    qa, sa, qw, sw, g = _small(N=64)
    y = oracle.ref_linear(qa, sa, qw, sw)
    gg, uu = torch.from_numpy(y[:, :32]), torch.from_numpy(y[:, 32:])
    geglu = (torch.nn.functional.gelu(gg, approximate="tanh") * uu).numpy()
    assert np.allclose(oracle.ref_linear(qa, sa, qw, sw, act="geglu"), geglu, rtol=1e-6, atol=1e-7)
    swapped = (torch.nn.functional.gelu(uu, approximate="tanh") * gg).numpy()
    assert oracle.parity_stats(swapped, geglu)[0] > 2e-2
    # residual + gate * (y + bias): the gate scales the projection, not the residual
    bias = np.linspace(-1, 1, 64).astype(np.float32)
    res = np.ones((y.shape[0], 64), np.float32)
    gate = np.full(64, 0.5, np.float32)
    got = oracle.ref_linear(qa, sa, qw, sw, bias=bias, residual=res, gate=gate)
    assert np.allclose(got, 1.0 + 0.5 * (y + bias), rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------
# golden fixtures (tests/golden/make_golden.py)
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)


def test_golden_rows(golden):
    names = [k[:-2] for k in golden.files if k.endswith("_q") and not k.startswith("fixed")]
    assert {"kat", "allbf16", "allbf16_rows", "act_c1", "act_c5h", "weight_f32"} <= set(names)
    fin = bits(all_finite_bf16())
    for n in names:
        x = golden[f"{n}_x"] if f"{n}_x" in golden.files else (fin.reshape(1, -1) if n == "allbf16"
                                                               else fin.reshape(255, 256))
        q, s = oracle.quant_rows(x)
        assert np.array_equal(q, golden[f"{n}_q"]), n
        assert np.array_equal(s.view(np.uint32), golden[f"{n}_s"].view(np.uint32)), n
    assert golden["kat_s"].view(np.uint32)[0] == 0x38A92493


def test_golden_fixed_scales(golden):
    fin = bits(all_finite_bf16())
    for i in range(len(FIXED_SCALES)):
        assert np.array_equal(oracle.pack_fixed(fin, float(golden[f"fixed{i}_scale"][0])), golden[f"fixed{i}_q"])


def test_golden_gemm(golden):
    G = golden
    common = (G["gemm_qa"], G["gemm_sa"], G["gemm_qw"], G["gemm_sw"])
    res = oracle.bf16_to_f32(G["gemm_res"])
    gate = oracle.bf16_to_f32(G["gemm_gate"])
    assert np.array_equal(oracle.ref_linear(*common, bias=G["gemm_bias"]), G["gemm_plain"])
    assert np.array_equal(oracle.ref_linear(*common, bias=G["gemm_bias"], act="gelu_tanh"), G["gemm_gelu"])
    assert np.array_equal(oracle.ref_linear(*common, act="geglu"), G["gemm_geglu"])
    assert np.array_equal(oracle.ref_linear(*common, act="swiglu"), G["gemm_swiglu"])
    assert np.array_equal(oracle.ref_linear(*common, bias=G["gemm_bias"], residual=res, gate=gate),
                          G["gemm_gated_res"])


def test_f32_to_bf16_rounding_matches_torch():
    x = np.random.default_rng(3).standard_normal(100000).astype(np.float32) * 1000
    assert np.array_equal(oracle.f32_to_bf16(x), bits(torch.from_numpy(x).to(torch.bfloat16)))


# ---------------------------------------------------------------------------
# residual_norm (kernels/norm.py:25-94)
# ---------------------------------------------------------------------------

def _rnq_inputs(M=33, D=1152, seed=3):
    # the reference's own test case (tests/test_gi_kernels.py:93-112), on the CPU
    g = torch.Generator().manual_seed(seed)
    res = torch.randn(M, D, generator=g)
    delta = torch.randn(M, D, generator=g).to(torch.bfloat16)
    dr, dc, b, gate = torch.rand(M, generator=g), torch.rand(D, generator=g), torch.randn(D, generator=g), \
        torch.rand(D, generator=g)
    w, beta = torch.rand(D, generator=g), torch.randn(D, generator=g)
    ms, mh = torch.randn(D, generator=g) * 0.1, torch.randn(D, generator=g) * 0.1
    return res, delta, dr, dc, b, gate, w, beta, ms, mh


@pytest.mark.parametrize("layernorm", [False, True])
def test_residual_norm_matches_reference_test_expectation(oracle_mod, layernorm):
    res, delta, dr, dc, b, gate, w, beta, ms, mh = _rnq_inputs()
    x, y = oracle_mod.residual_norm(res.numpy(), delta.float().numpy(), dr.numpy(), dc.numpy(), b.numpy(),
                                    gate.numpy(), layernorm=layernorm, weight=w.numpy(), beta=beta.numpy(),
                                    mod_scale=ms.numpy(), mod_shift=mh.numpy())
    # the reference test's expectation, evaluated by torch in float32, op by op
    expect = res + (delta.float() * dr[:, None] * dc + b) * gate
    assert np.array_equal(x, expect.numpy())
    xc = expect - expect.mean(-1, keepdim=True) if layernorm else expect
    ty = xc * torch.rsqrt(xc.pow(2).mean(-1, keepdim=True) + 1e-6)
    ty = (ty * w + beta) * (1 + ms) + mh
    assert np.abs(y - ty.double().numpy()).max() < 2e-5 * np.abs(y).max()


def test_residual_norm_against_torch_norms(oracle_mod):
    g = torch.Generator().manual_seed(9)
    x = torch.randn(7, 640, generator=g) * 3 + 0.5
    w, b = torch.rand(640, generator=g), torch.randn(640, generator=g)
    _, y = oracle_mod.residual_norm(x.numpy(), layernorm=True, weight=w.numpy(), beta=b.numpy(), eps=1e-5)
    ref = torch.nn.functional.layer_norm(x.double(), (640,), w.double(), b.double(), eps=float(np.float32(1e-5)))
    assert np.abs(y - ref.numpy()).max() < 1e-12
    _, y = oracle_mod.residual_norm(x.numpy(), weight=w.numpy(), eps=1e-6)
    ref = torch.nn.functional.rms_norm(x.double(), (640,), w.double(), eps=float(np.float32(1e-6)))
    assert np.abs(y - ref.numpy()).max() < 1e-12


def test_residual_norm_closed_forms(oracle_mod):
    D = 256
    c = np.array([[2.0], [-0.5], [0.0]], dtype=np.float32) * np.ones((3, D), np.float32)
    with np.errstate(invalid="ignore"):
        _, y = oracle_mod.residual_norm(c, eps=0.0)
    assert np.allclose(y[0], 1.0) and np.allclose(y[1], -1.0) and np.isnan(y[2]).all()  # 0/sqrt(0)
    _, y = oracle_mod.residual_norm(c, layernorm=True, eps=1e-6)
    assert np.abs(y).max() == 0.0  # constant rows centre to zero
    # unit-RMS rows are fixed points of RMS norm (eps 0)
    g = np.random.default_rng(0).standard_normal((4, D)).astype(np.float32)
    g /= np.sqrt((g.astype(np.float64) ** 2).mean(axis=1, keepdims=True)).astype(np.float32)
    _, y = oracle_mod.residual_norm(g, eps=0.0)
    assert np.abs(y - g).max() < 1e-6


def test_residual_norm_tables_and_bf16_store(oracle_mod):
    rng = np.random.default_rng(1)
    M, D, n = 6, 64, 3
    res = rng.standard_normal((M, D)).astype(np.float32)
    delta = rng.standard_normal((M, D)).astype(np.float32)
    gate = rng.random((n, D)).astype(np.float32)
    ms, mh = rng.standard_normal((n, D)).astype(np.float32), rng.standard_normal((n, D)).astype(np.float32)
    idx = np.array([2, 0, 1, 1, 2, 0], dtype=np.int32)
    x, y = oracle_mod.residual_norm(res, delta, gate=gate, mod_scale=ms, mod_shift=mh, mod_index=idx)
    for m in range(M):  # row m uses table row idx[m]
        xm, ym = oracle_mod.residual_norm(res[m:m + 1], delta[m:m + 1], gate=gate[idx[m]], mod_scale=ms[idx[m]],
                                          mod_shift=mh[idx[m]])
        assert np.array_equal(x[m], xm[0]) and np.array_equal(y[m], ym[0])
    # bf16 residual: the stored (rounded) sum is what gets normalized
    xb, _ = oracle_mod.residual_norm(res, delta, res_bf16=True)
    assert np.array_equal(xb, oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16((res + delta).astype(np.float32))))


# ---------------------------------------------------------------------------
# qkv_split (kernels/rope.py:21-80)
# ---------------------------------------------------------------------------

def _qkv_case(T=7, HQ=4, HKV=2, HD=128, seed=2):
    # the reference test's case (tests/test_gi_kernels.py:58-70), on the CPU
    from instinctflash_amd.kernels.rope import rope_inv_freq
    g = torch.Generator().manual_seed(seed)
    raw = torch.randn(T, (HQ + 2 * HKV) * HD, generator=g).to(torch.bfloat16)
    row = torch.rand(T, generator=g) + 0.5
    col = torch.rand(raw.shape[1], generator=g) + 0.5
    bias = torch.randn(raw.shape[1], generator=g)
    qn, kn = torch.rand(HD, generator=g) + 0.5, torch.rand(HD, generator=g) + 0.5
    inv = rope_inv_freq(HD, 1e6, "cpu")
    pos = torch.stack([torch.arange(T), torch.arange(T) * 2, torch.arange(T) * 3], 1).float()
    sec = (torch.arange(HD // 2) % 3).int()
    return raw, row, col, bias, qn, kn, inv, pos, sec


def test_qkv_split_matches_reference_test_expectation(oracle_mod):
    T, HQ, HKV, HD = 7, 4, 2, 128
    raw, row, col, bias, qn, kn, inv, pos, sec = _qkv_case()
    q, k, v = oracle_mod.qkv_split(raw.float().numpy(), HQ, HKV, HD, row.numpy(), col.numpy(), bias.numpy(),
                                   inv.numpy(), pos.numpy(), sec.numpy(), qn.numpy(), kn.numpy())
    # the reference test's own formula (tests/test_gi_kernels.py:74-88), in torch float32
    x = raw.float() * row[:, None] * col + bias
    xq, xk, xv = x[:, :HQ * HD].view(T, HQ, HD), x[:, HQ * HD:(HQ + HKV) * HD].view(T, HKV, HD), \
        x[:, (HQ + HKV) * HD:].view(T, HKV, HD)
    rms = lambda t, w: t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + 1e-6) * w  # noqa: E731
    ang = pos.gather(1, sec.long()[None].expand(T, -1)) * inv

    def rope(t):
        c, s = ang.cos()[:, None], ang.sin()[:, None]
        lo, hi = t[..., :HD // 2], t[..., HD // 2:]
        return torch.cat([lo * c - hi * s, hi * c + lo * s], -1)
    assert np.abs(q - rope(rms(xq, qn)).double().numpy()).max() < 1e-4
    assert np.abs(k - rope(rms(xk, kn)).double().numpy()).max() < 1e-4
    assert np.array_equal(v, xv.double().numpy())


def test_qkv_split_invariants(oracle_mod):
    from instinctflash_amd.kernels.rope import rope_inv_freq
    T, HQ, HKV, HD = 5, 2, 1, 64
    rng = np.random.default_rng(4)
    raw = rng.standard_normal((T, (HQ + 2 * HKV) * HD)).astype(np.float32)
    inv = rope_inv_freq(HD, 1e4, "cpu").numpy()
    assert inv[0] == 1.0 and np.allclose(inv[1:] / inv[:-1], 1e4 ** (-2 / HD))
    pos = (np.arange(T, dtype=np.float32) * 37)[:, None]
    q0, k0, v0 = oracle_mod.qkv_split(raw, HQ, HKV, HD)
    q, k, v = oracle_mod.qkv_split(raw, HQ, HKV, HD, inv_freq=inv, pos=pos)
    half = HD // 2
    pair = lambda t: t[..., :half] ** 2 + t[..., half:] ** 2  # noqa: E731
    assert np.allclose(pair(q), pair(q0)) and np.allclose(pair(k), pair(k0))  # rotations keep pair norms
    assert np.array_equal(q[0], q0[0]) and np.array_equal(v, v0)              # position 0: identity
    # rotating by a then b equals rotating by a + b (float32 angles exact for these integers)
    q2, _, _ = oracle_mod.qkv_split(np.concatenate([q[:, :, :].reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)], 1)
                                    .astype(np.float32), HQ, HKV, HD, inv_freq=inv, pos=pos)
    qa, _, _ = oracle_mod.qkv_split(raw, HQ, HKV, HD, inv_freq=inv, pos=2 * pos)
    assert np.abs(q2 - qa).max() < 1e-5
    # normalized heads have unit RMS (unit weights)
    qn, kn, _ = oracle_mod.qkv_split(raw, HQ, HKV, HD, q_norm=np.ones(HD), k_norm=np.ones(HD), eps=0.0)
    assert np.allclose(np.sqrt((qn ** 2).mean(-1)), 1.0) and np.allclose(np.sqrt((kn ** 2).mean(-1)), 1.0)


# ---------------------------------------------------------------------------
# wan_qkv (kernels/wan.py:19-81)
# ---------------------------------------------------------------------------

def test_wan_qkv_against_qkv_split_and_rms_norm(oracle_mod):
    from instinctflash_amd.kernels.rope import rope_inv_freq
    H, HD, T, B = 3, 16, 4, 2
    D, half = H * HD, HD // 2
    rng = np.random.default_rng(5)
    raw = rng.standard_normal((B * T, 3 * D)).astype(np.float32)
    inv = rope_inv_freq(HD, 1e4, "cpu").numpy()
    pos = rng.integers(0, 50, (T, 3)).astype(np.float32)
    sec = (np.arange(half) % 3).astype(np.int32)
    q, k, v = oracle_mod.wan_qkv(raw, H, HD, T, inv_freq=inv, pos=pos, sections=sec)
    # interleaved pairs (2j, 2j+1) == split halves (j, j + HD/2) after a per-head permutation
    perm = np.concatenate([np.arange(0, HD, 2), np.arange(1, HD, 2)])
    cols = np.concatenate([h * HD + perm for h in range(H)])
    raw_split = np.concatenate([raw[:, p * D:(p + 1) * D][:, cols] for p in range(3)], axis=1)
    pos_rows = pos[np.arange(B * T) % T]
    qs, ks, vs = oracle_mod.qkv_split(raw_split, H, H, HD, inv_freq=inv, pos=pos_rows, sections=sec)
    assert np.abs(q[:, cols] - qs.reshape(B * T, D)).max() < 1e-12
    assert np.abs(k[:, cols] - ks.reshape(B * T, D)).max() < 1e-12
    assert np.array_equal(v, raw[:, 2 * D:].astype(np.float64))
    # full-width RMS norm == torch rms_norm over D
    w = rng.random(D) + 0.5
    qn, _ = oracle_mod.wan_qkv(raw, H, HD, T, parts=2, q_norm=w, k_norm=w)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(raw[:, :D]).double(), (D,), torch.from_numpy(w),
                                       eps=float(np.float32(1e-6)))
    assert np.abs(qn - ref.numpy()).max() < 1e-12


def test_wan_qkv_rotation_invariants(oracle_mod):
    from instinctflash_amd.kernels.rope import rope_inv_freq
    H, HD, T = 2, 32, 3
    D = H * HD
    rng = np.random.default_rng(6)
    raw = rng.standard_normal((T, 2 * D)).astype(np.float32)
    inv = rope_inv_freq(HD, 1e4, "cpu").numpy()
    pos = np.array([[0.0], [5.0], [900.0]], np.float32)
    q0, _ = oracle_mod.wan_qkv(raw, H, HD, T, parts=2)
    q, _ = oracle_mod.wan_qkv(raw, H, HD, T, parts=2, inv_freq=inv, pos=pos)
    pair = lambda a: (a.reshape(T, -1, 2) ** 2).sum(-1)  # noqa: E731
    assert np.allclose(pair(q), pair(q0)) and np.array_equal(q[0], q0[0])


def test_moe_router_matches_reference_test_construction(oracle_mod):
    # tests/test_gi_kernels.py:179-192: topk of sigmoid + bias, scatter the
    # unbiased sigmoid, renormalize to `scale`.
    g = torch.Generator().manual_seed(7)
    M, D, E = 51, 768, 32
    x = torch.randn(M, D, generator=g, dtype=torch.float64)
    gw = torch.randn(E, D, generator=g, dtype=torch.float64) * 0.05
    eb = torch.rand(E, generator=g, dtype=torch.float64) * 0.01
    got, _ = oracle_mod.moe_router(x.numpy(), gw.numpy(), eb.numpy(), 4, 4.0)
    s = torch.sigmoid(x @ gw.t())
    idx = torch.topk(s + eb, 4, -1).indices
    ref = torch.zeros(M, E, dtype=torch.float64).scatter(1, idx, s.gather(1, idx))
    ref = ref / (ref.sum(-1, keepdim=True) + 1e-20) * 4.0
    assert np.abs(got - ref.numpy()).max() < 1e-12


def test_moe_router_brute_force_and_invariants(oracle_mod):
    import itertools
    rng = np.random.default_rng(3)
    M, D, E, K = 20, 16, 7, 3
    x = rng.standard_normal((M, D))
    gw = rng.standard_normal((E, D)) * 0.3
    eb = rng.standard_normal(E) * 0.2
    got, sel = oracle_mod.moe_router(x, gw, eb, K, 2.5)
    sg = 1.0 / (1.0 + np.exp(-(x @ gw.T)))
    for m in range(M):
        # the chosen set maximizes the summed selection score over all K-subsets
        best = max(itertools.combinations(range(E), K), key=lambda c: sum(sel[m, list(c)]))
        assert set(np.nonzero(got[m])[0]) == set(best)
        w = sg[m, list(best)]
        assert np.allclose(got[m, list(best)], w / w.sum() * 2.5, rtol=1e-14)
    assert np.allclose(got.sum(1), 2.5) and ((got == 0).sum(1) == E - K).all()
    # the bias moves selection only: a huge bias on expert 0 forces it in with its unbiased weight
    eb2 = eb.copy()
    eb2[0] = 100.0
    got2, _ = oracle_mod.moe_router(x, gw, eb2, K, 2.5)
    chosen_sum = np.where(got2 > 0, sg, 0.0).sum(1)
    assert (got2[:, 0] > 0).all() and np.allclose(got2[:, 0], 2.5 * sg[:, 0] / chosen_sum, rtol=1e-14)
    # equal scores pick the lowest index (repeated argmax)
    tie, _ = oracle_mod.moe_router(np.zeros((1, D)), gw, np.zeros(E), K, 1.0)
    assert np.array_equal(np.nonzero(tie[0])[0], np.arange(K)) and np.allclose(tie[0, :K], 1.0 / K)


def test_moe_act_matches_reference_test_construction(oracle_mod):
    # tests/test_gi_kernels.py:193-203: column weights by repeat_interleave of
    # the routing weights over each expert's group, ones for the shared expert.
    g = torch.Generator().manual_seed(5)
    M, E, G, S = 6, 4, 16, 24
    F = E * G + S
    gu = torch.randn(M, 2 * F, generator=g)
    row, col = torch.rand(M, generator=g) + 0.5, torch.rand(2 * F, generator=g) + 0.5
    rw = torch.rand(M, E, generator=g)
    h = oracle_mod.moe_act(gu.numpy(), row.numpy(), col.numpy(), rw.numpy(), E, G, E * G)
    xg = gu.double() * row.double()[:, None] * col.double()
    wcol = torch.cat([rw.double().repeat_interleave(G, 1), torch.ones(M, S, dtype=torch.float64)], 1)
    ref = torch.nn.functional.silu(xg[:, :F]) * xg[:, F:] * wcol
    assert np.abs(h - ref.numpy()).max() <= 1e-5 * np.abs(ref.numpy()).max()
    # unit routing weights reduce it to the plain SwiGLU of gated_act_quant
    plain = oracle_mod.moe_act(gu.numpy(), row.numpy(), col.numpy(), np.ones((M, E), np.float32), E, G, E * G)
    sw = torch.nn.functional.silu(xg[:, :F]) * xg[:, F:]
    assert np.abs(plain - sw.numpy()).max() <= 1e-5 * np.abs(sw.numpy()).max()
    # n_routed beyond E*G clamps to the last expert's weight
    cl = oracle_mod.moe_act(gu.numpy(), row.numpy(), col.numpy(), rw.numpy(), E, G, F)
    ratio = cl[:, E * G:] / np.where(plain[:, E * G:] == 0, 1, plain[:, E * G:])
    nz = plain[:, E * G:] != 0
    assert np.allclose(ratio[nz], np.broadcast_to(rw.numpy()[:, E - 1:E], ratio.shape)[nz], rtol=1e-6)


def _ref_attention_torch(q, k, v, limits, scale):
    # tests/test_gi_kernels.py:22-30, evaluated in float64
    g = q.shape[2] // k.shape[2]
    kk = k.double().repeat_interleave(g, 2)
    vv = v.double().repeat_interleave(g, 2)
    s = torch.einsum("bqhd,bkhd->bhqk", q.double(), kk) * scale
    n = torch.arange(k.shape[1])
    s = s.masked_fill(~(n[None, :] < limits[:, None])[None, None], float("-inf"))
    return torch.einsum("bhqk,bkhd->bqhd", s.softmax(-1), vv)


@pytest.mark.parametrize("hd,hq,hkv", [(256, 8, 1), (72, 16, 16), (128, 16, 2)])
def test_attention_matches_reference_formulation_and_sdpa(oracle_mod, hd, hq, hkv):
    g = torch.Generator().manual_seed(hd)
    q = torch.randn(2, 9, hq, hd, generator=g)
    k = torch.randn(2, 21, hkv, hd, generator=g)
    v = torch.randn(2, 21, hkv, hd, generator=g)
    lim = torch.tensor([1, 5, 21, 13, 7, 21, 2, 3, 20])
    got = oracle_mod.attention(q.numpy(), k.numpy(), v.numpy(), lim.numpy(), hd ** -0.5)
    ref = _ref_attention_torch(q, k, v, lim, hd ** -0.5)
    assert np.abs(got - ref.numpy()).max() < 1e-12
    # torch's fused attention with the same boolean mask, per KV-head group
    grp = hq // hkv
    mask = torch.arange(21)[None, :] < lim[:, None]
    sd = torch.nn.functional.scaled_dot_product_attention(
        q.double().transpose(1, 2), k.double().repeat_interleave(grp, 2).transpose(1, 2),
        v.double().repeat_interleave(grp, 2).transpose(1, 2), attn_mask=mask[None, None], scale=hd ** -0.5)
    assert np.abs(got - sd.transpose(1, 2).numpy()).max() < 1e-10


def test_attention_closed_forms_and_index(oracle_mod):
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 4, 2, 16))
    k = rng.standard_normal((1, 9, 1, 16))
    v = rng.standard_normal((1, 9, 1, 16))
    one = oracle_mod.attention(q, k, v, np.array([1, 1, 1, 1]), 0.25)
    assert np.allclose(one, np.broadcast_to(v[:, :1], one.shape))  # one visible key: its value row
    flat = oracle_mod.attention(np.zeros_like(q), k, v, np.array([3, 9, 5, 2]), 0.25)
    for t, n in enumerate((3, 9, 5, 2)):  # equal scores: the mean of the visible rows
        assert np.allclose(flat[0, t], v[0, :n, 0].mean(0)[None, :])
    idx = np.array([8, 0, 4, 4, 2])  # pooled cache: key n is row idx[n]
    got = oracle_mod.attention(q, k, v, np.array([5, 3, 1, 5]), 0.25, kv_index=idx)
    assert np.allclose(got, oracle_mod.attention(q, k[:, idx], v[:, idx], np.array([5, 3, 1, 5]), 0.25))
