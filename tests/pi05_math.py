"""Float32 restatement of the pi05 model math (test checker, not product code).

The computation the reference engine performs (instinctflash/engines/pi05/
engine.py:142-245), written directly in torch: every projection input is
quantized per token to E4M3 with this package's recipe (max(amax, 1e-12) *
fl32(1/448), IEEE division, RNE cast), weights are the dequantized per-channel
E4M3 weights, and everything else is float32 (attention in float32 softmax),
rounded to fp16 / bf16 where instinctflash_amd.pi05_forward stores a tensor in
that type (q/k/v and attention outputs fp16; MLP activations, the prefix
q|k|v and the expert's projection outputs bf16), so that both sides quantize
the same values. Used by tests/test_gpu_pi05_forward.py to check
instinctflash_amd.pi05_forward end to end."""
import torch
import torch.nn.functional as Fn

INV448 = torch.tensor(1.0 / 448.0, dtype=torch.float32).item()


def quant(x):
    x = x.float()
    s = x.abs().amax(dim=1).clamp_min(1e-12) * INV448
    q = (x / s[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn).float()
    return q * s[:, None]


def bf16(x):
    return x.bfloat16().float()


def lin(x, w, act=None):
    """quantize x per token, project with the dequantized FP8 weight (+ bias)."""
    W = w.w.float() * w.scale.float()[:, None]
    y = quant(x) @ W.t()
    if w.bias is not None:
        y = y + w.bias.float()
    if act == "gelu_tanh":
        y = Fn.gelu(y, approximate="tanh")
    elif act == "geglu":
        F = y.shape[1] // 2
        y = Fn.gelu(y[:, :F], approximate="tanh") * y[:, F:]
    return y


def rms(x, eps=1e-6):
    return x * torch.rsqrt(x.pow(2).mean(dim=1, keepdim=True) + eps)


def layer_norm(x, w, b, eps=1e-6):
    return Fn.layer_norm(x, (x.shape[1],), w, b, eps)


def rope(x, pos, inv_freq):
    """split-half rotary of [T, H, HD] at float32 angles pos[t] * inv_freq[i]."""
    ang = (pos.float()[:, None] * inv_freq.float()[None, :]).double()
    c, s = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
    half = x.shape[-1] // 2
    lo, hi = x[..., :half].double(), x[..., half:].double()
    return torch.cat([lo * c - hi * s, hi * c + lo * s], dim=-1).float()


def attend(q, k, v, scale):
    """q [Tq, H, D], k/v [Tk, Hkv, D] (Hkv divides H), float32 softmax."""
    H, Hkv = q.shape[1], k.shape[1]
    k = k.float().repeat_interleave(H // Hkv, dim=1)
    v = v.float().repeat_interleave(H // Hkv, dim=1)
    a = torch.einsum("qhd,khd->hqk", q.float(), k) * scale
    return torch.einsum("hqk,khd->qhd", a.softmax(dim=-1), v)


def forward(p, images, prompt_rows, noise, inv_freq, trace=None):
    """Actions [chunk, action] and the last prefix layer's keys [n_prefix, HD];
    ``trace`` (a dict), if given, receives intermediate streams."""
    d = p.dims
    pl = p.plain
    T, n = d.image_rows, prompt_rows.shape[0]
    half = torch.float16
    # vision
    pix = images.view(d.views, 3, 16, 14, 16, 14).permute(0, 2, 4, 3, 5, 1).reshape(T, 588)
    x = (pix.half().float() @ p.patch_w.float()).half().float() + p.patch_b
    x = (x.view(d.views, d.patches, d.vis_d) + p.pos_emb).view(T, d.vis_d)
    for i, blk in enumerate(p.vision):
        qkv = lin(layer_norm(x, *blk.ln1), pl[f"v{i}.qkv"]).half()
        qkv = qkv.view(d.views, d.patches, 3, d.vis_heads, d.vis_hd)
        ctx = torch.cat([attend(qkv[b, :, 0], qkv[b, :, 1], qkv[b, :, 2], d.vis_hd ** -0.5)
                         for b in range(d.views)]).half().view(T, d.vis_d)
        x = x + lin(ctx, pl[f"v{i}.o"])
        h = bf16(lin(layer_norm(x, *blk.ln2), pl[f"v{i}.fc1"], "gelu_tanh"))
        x = x + lin(h, pl[f"v{i}.fc2"])
    if trace is not None:
        trace["vision"] = x
    px = torch.cat([lin(layer_norm(x, *p.post_ln), pl["projector"]), prompt_rows.float()])
    # prefix (valid rows only: the engine's padding rows never reach them)
    S = T + n
    pos = torch.arange(S, device=x.device, dtype=torch.float32)
    keys, values = [], []
    HD = d.head_dim
    for i in range(d.prefix_layers):
        qkv = bf16(lin(rms(px), pl[f"p{i}.qkv"])).view(S, d.heads + 2, HD)
        q = rope(qkv[:, :d.heads], pos, inv_freq).half()
        k = rope(qkv[:, d.heads:d.heads + 1], pos, inv_freq).half()
        keys.append(k)
        values.append(qkv[:, d.heads + 1:].half())
        if i == d.prefix_layers - 1:
            if trace is not None:
                trace["prefix"] = px
            break
        ctx = attend(q, k, values[-1], HD ** -0.5).half().reshape(S, d.heads * HD)
        px = px + lin(ctx, pl[f"p{i}.o"])
        px = px + lin(bf16(lin(rms(px), pl[f"p{i}.gate_up"], "geglu")), pl[f"p{i}.down"])
    # expert
    A = d.chunk
    cpos = torch.arange(S, S + A, device=x.device, dtype=torch.float32)
    act = noise.float().clone()
    L = d.expert_layers
    for t in range(d.steps):
        ma, mf = p.mod_attn[t], p.mod_ffn[t]
        dx = act @ p.action_in[0] + p.action_in[1]
        for i in range(L):
            h = rms(dx) * (1 + ma[i, 0]) + ma[i, 1]
            qkv = lin(h, pl[f"e{i}.qkv"]).view(A, d.heads + 2, HD)
            q = rope(qkv[:, :d.heads], cpos, inv_freq).half()
            k = torch.cat([keys[i], rope(qkv[:, d.heads:d.heads + 1], cpos, inv_freq).half()])
            v = torch.cat([values[i], qkv[:, d.heads + 1:].half()])
            ctx = attend(q, k, v, HD ** -0.5).half().reshape(A, d.heads * HD)
            dx = dx + bf16(lin(ctx, pl[f"e{i}.o"])) * ma[i, 2]
            h = rms(dx) * (1 + mf[i, 0]) + mf[i, 1]
            dx = dx + bf16(lin(bf16(lin(h, pl[f"e{i}.gate_up"], "geglu")), pl[f"e{i}.down"])) * mf[i, 2]
        y = rms(dx) * (1 + p.mod_final[t, 0]) + p.mod_final[t, 1]
        act = act + (y @ p.action_out[0] + p.action_out[1]) * (-1.0 / d.steps)
    return act, keys[-1][:, 0]
