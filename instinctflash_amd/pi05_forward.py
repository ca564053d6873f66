"""pi05 (SigLIP + Gemma-2B prefix + Gemma-300M flow-matching expert) forward
on the gfx950 kernels, as one launch schedule captured into one HIP graph.

The model is the one the reference engine serves (instinctflash/engines/pi05/
engine.py:1-12; dimensions :27-31; math of its three stages :142-245). This
module is not that engine: it plans its own schedule for MI355X from the
fused entry points of this package.

* Every projection dequantizes in its own epilogue (``linear``): no raw bf16
  accumulator goes to HBM. The residual updates of the vision tower and of
  the prefix are the projections' residual epilogues on the float32 residual
  stream; the next pre-norm then only normalizes (``residual_norm_quant``
  without a delta).
* Because each projection has consumed its token scales before the next
  producer runs, one E4M3 operand buffer and one scale vector serve the whole
  forward.
* GLU weights are packed once (``pack_glu``): GeGLU runs in the gate|up
  projection's epilogue and writes the half-width activation, which
  ``quant_rows`` requantizes.
* The 50-row expert uses the M <= 64 weight tile layout (``pack_skinny``);
  its q|k|v projection applies the rotary embedding and writes the K/V cache
  rows in its epilogue (``linear_qkv_rope``), and its attention writes the
  output projection's E4M3 operand directly (``attention(q8=...)``).
* Sequence lengths (valid prefix rows, key count of the expert) live in
  device memory, so a captured graph serves any prompt length up to the
  physical row count it was captured for.

Weights are random with the published architecture's shapes (no checkpoint
is available here): ``random_pi05``. ``Pi05Forward.run()`` executes the
schedule eagerly; ``capture()`` returns a replayable ``torch.cuda.CUDAGraph``.
The schedule is built once, at construction, as a list of ``Launch``
records (``Pi05Forward.schedule``); running it is iterating over the list.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .kernels import E4M3, Fp8Weight, attention, linear, pack_glu, quant_rows, quantize_weight, \
    residual_norm_quant, row_quant
from .kernels.attention import SplitWorkspace, split_count
from .kernels.fp8 import pack_skinny
from .kernels.rope import linear_qkv_rope, permute_rope_rows, qkv_split, rope_inv_freq


@dataclass(frozen=True)
class Pi05Dims:
    """Architecture constants (reference engines/pi05/engine.py:27-31) and the
    serving geometry. Layer counts are parameters so tests can run short
    stacks of the same blocks."""
    views: int = 3
    max_prompt: int = 48
    chunk: int = 50
    steps: int = 10
    vision_layers: int = 27
    prefix_layers: int = 18
    expert_layers: int = 18
    patches: int = 256          # 224 / 14 squared
    vis_d: int = 1152
    vis_heads: int = 16
    vis_hd: int = 72
    vis_ff: int = 4304
    lm_d: int = 2048
    lm_ff: int = 16384
    ex_d: int = 1024
    ex_ff: int = 4096
    heads: int = 8              # query heads of prefix and expert (one KV head)
    head_dim: int = 256
    action: int = 32
    bucket: int = 16

    @property
    def image_rows(self) -> int:
        return self.views * self.patches

    @property
    def prefix_rows(self) -> int:  # physical rows of the prefix stage
        return self.image_rows + -(-self.max_prompt // self.bucket) * self.bucket

    @property
    def qkv_n(self) -> int:
        return (self.heads + 2) * self.head_dim


@dataclass
class VisionBlock:
    ln1: tuple
    qkv: Fp8Weight      # + bias
    o: Fp8Weight        # + bias
    ln2: tuple
    fc1: Fp8Weight      # + bias (GELU-tanh epilogue)
    fc2: Fp8Weight      # + bias


@dataclass
class DecoderBlock:
    qkv: Fp8Weight
    o: Fp8Weight | None
    gate_up: Fp8Weight | None   # GLU-packed
    down: Fp8Weight | None


@dataclass
class Pi05Params:
    dims: Pi05Dims
    patch_w: torch.Tensor       # [588, vis_d] fp16, pixel (row, col, channel) order
    patch_b: torch.Tensor
    pos_emb: torch.Tensor       # [patches, vis_d]
    vision: list
    post_ln: tuple
    projector: Fp8Weight
    prefix: list
    expert: list                # skinny-tiled weights, rope-ordered q|k|v
    action_in: tuple            # (w^T [action, ex_d], b)
    action_out: tuple           # (w^T [ex_d, action], b)
    mod_attn: torch.Tensor      # [steps, L, 3, ex_d]: scale, shift, gate
    mod_ffn: torch.Tensor
    mod_final: torch.Tensor     # [steps, 2, ex_d]
    plain: dict = field(default_factory=dict)  # unpacked copies for checkers (keep_plain=True)


def random_pi05(dims: Pi05Dims, device, seed=0, keep_plain=False) -> Pi05Params:
    """Random weights of the architecture: projections N(0, 0.02) quantized per
    output channel, norm affines near identity, small adaptive-norm tables.
    With ``keep_plain`` the unpacked FP8 weights are kept for parity checks."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    d = dims
    plain = {}

    def rnd(*shape, std=1.0):
        return torch.randn(*shape, generator=g, device=dev) * std

    def proj(name, n, k, bias=False):
        w = quantize_weight(rnd(n, k, std=0.02), rnd(n, std=0.01) if bias else None, dev)
        if keep_plain:
            plain[name] = w
        return w

    def affine(n):
        return (1.0 + rnd(n, std=0.05), rnd(n, std=0.02))

    vision = [VisionBlock(affine(d.vis_d), proj(f"v{i}.qkv", 3 * d.vis_d, d.vis_d, True),
                          proj(f"v{i}.o", d.vis_d, d.vis_d, True), affine(d.vis_d),
                          proj(f"v{i}.fc1", d.vis_ff, d.vis_d, True), proj(f"v{i}.fc2", d.vis_d, d.vis_ff, True))
              for i in range(d.vision_layers)]
    prefix = []
    for i in range(d.prefix_layers):
        qkv = proj(f"p{i}.qkv", d.qkv_n, d.lm_d)
        if i == d.prefix_layers - 1:  # only this layer's K/V reach the expert
            prefix.append(DecoderBlock(qkv, None, None, None))
            continue
        prefix.append(DecoderBlock(qkv, proj(f"p{i}.o", d.lm_d, d.heads * d.head_dim),
                                   pack_glu(proj(f"p{i}.gate_up", 2 * d.lm_ff, d.lm_d)),
                                   proj(f"p{i}.down", d.lm_d, d.lm_ff)))
    expert = []
    for i in range(d.expert_layers):
        expert.append(DecoderBlock(
            pack_skinny(permute_rope_rows(proj(f"e{i}.qkv", d.qkv_n, d.ex_d), d.heads, 1, d.head_dim)),
            pack_skinny(proj(f"e{i}.o", d.ex_d, d.heads * d.head_dim)),
            pack_skinny(pack_glu(proj(f"e{i}.gate_up", 2 * d.ex_ff, d.ex_d))),
            pack_skinny(proj(f"e{i}.down", d.ex_d, d.ex_ff))))
    L = d.expert_layers
    return Pi05Params(
        dims=d,
        patch_w=rnd(3 * 14 * 14, d.vis_d, std=0.02).half(), patch_b=rnd(d.vis_d, std=0.01),
        pos_emb=rnd(d.patches, d.vis_d, std=0.02), vision=vision, post_ln=affine(d.vis_d),
        projector=proj("projector", d.lm_d, d.vis_d, True), prefix=prefix, expert=expert,
        action_in=(rnd(d.action, d.ex_d, std=0.1), rnd(d.ex_d, std=0.01)),
        action_out=(rnd(d.ex_d, d.action, std=0.02), rnd(d.action, std=0.01)),
        mod_attn=rnd(d.steps, L, 3, d.ex_d, std=0.1), mod_ffn=rnd(d.steps, L, 3, d.ex_d, std=0.1),
        mod_final=rnd(d.steps, 2, d.ex_d, std=0.1), plain=plain)


@dataclass
class Launch:
    """One entry of the schedule: ``fn()`` enqueues it on the current stream;
    ``io`` names what it reads and writes (used by parity checks)."""
    name: str
    kind: str       # linear | qkv_rope | norm | quant | attention | split | torch
    fn: object
    io: dict


class Pi05Forward:
    """The three stages of a pi05 prediction as one schedule of launches.

    Inputs (device tensors, written by ``set_inputs``): images [V, 3, 224, 224]
    in [-1, 1], prompt rows [n, lm_d] (the scaled token embeddings), noise
    [chunk, action]. Output: ``actions`` [chunk, action] after the Euler steps."""

    def __init__(self, params: Pi05Params, device):
        self.p = params
        d = self.d = params.dims
        dev = self.dev = torch.device(device)
        f32, f16, bf16 = torch.float32, torch.float16, torch.bfloat16
        T, S, A = d.image_rows, d.prefix_rows, d.chunk
        widest = max(d.vis_ff, d.lm_ff, d.ex_ff, d.heads * d.head_dim)
        # one E4M3 operand and one token-scale vector for every projection
        self.op8 = torch.zeros(S * widest, dtype=E4M3, device=dev)
        self.op_scale = torch.zeros(S, dtype=f32, device=dev)
        # inputs
        self.images = torch.zeros(d.views, 3, 224, 224, dtype=f32, device=dev)
        self.prompt = torch.zeros(S - T, d.lm_d, dtype=f32, device=dev)
        self.noise = torch.zeros(A, d.action, dtype=f32, device=dev)
        self.n_prefix = torch.zeros(1, dtype=torch.int32, device=dev)   # image rows + prompt tokens
        self.n_keys = torch.zeros(1, dtype=torch.int32, device=dev)     # n_prefix + chunk
        # vision stage
        self.vis_stream = torch.zeros(T, d.vis_d, dtype=f32, device=dev)
        self.vis_qkv = torch.zeros(T, 3 * d.vis_d, dtype=f16, device=dev)
        self.vis_ctx = torch.zeros(T, d.vis_d, dtype=f16, device=dev)
        self.vis_mlp = torch.zeros(T, d.vis_ff, dtype=bf16, device=dev)
        # prefix stage (float32 residual stream over the physical rows)
        self.lm_stream = torch.zeros(S, d.lm_d, dtype=f32, device=dev)
        self.lm_qkv = torch.zeros(S, d.qkv_n, dtype=bf16, device=dev)
        self.lm_q = torch.zeros(S, d.heads, d.head_dim, dtype=f16, device=dev)
        self.lm_ctx = torch.zeros(S, d.heads * d.head_dim, dtype=f16, device=dev)
        self.lm_mlp = torch.zeros(S, d.lm_ff, dtype=bf16, device=dev)
        # the K/V caches: prefix rows, then the expert's chunk rows after the valid prefix
        self.keys = torch.zeros(d.prefix_layers, S + A, 1, d.head_dim, dtype=f16, device=dev)
        self.values = torch.zeros_like(self.keys)
        self.inv_freq = rope_inv_freq(d.head_dim, 10000.0, dev)
        self.pos_prefix = torch.arange(S, dtype=f32, device=dev)[:, None].contiguous()
        self.pos_chunk = torch.zeros(A, 1, dtype=f32, device=dev)
        # expert stage
        self.actions = torch.zeros(A, d.action, dtype=f32, device=dev)
        self.ex_stream = torch.zeros(A, d.ex_d, dtype=f32, device=dev)
        self.ex_out = torch.zeros(A, d.ex_d, dtype=f32, device=dev)
        self.ex_q = torch.zeros(A, d.heads, d.head_dim, dtype=f16, device=dev)
        self.ex_proj = torch.zeros(A, d.ex_d, dtype=bf16, device=dev)
        self.ex_mlp = torch.zeros(A, d.ex_ff, dtype=bf16, device=dev)
        self.ex_split = SplitWorkspace(1, A, d.heads, 1, d.head_dim, max(2, split_count(1, A, d.heads, 1, S + A)),
                                       dev)
        dt = -1.0 / d.steps  # Euler step of the flow from t = 1 to 0
        self.out_w = (params.action_out[0] * dt).contiguous()
        self.out_b = (params.action_out[1] * dt).contiguous()
        self.rows = S
        # the whole prediction as one ordered list of launches
        self.schedule: list[Launch] = []
        self._plan_vision()
        self._plan_prefix()
        self._plan_expert()

    # ------------------------------------------------------------------ inputs
    def set_inputs(self, images, prompt_rows, noise):
        """images [V, 3, 224, 224]; prompt_rows [n, lm_d] (n <= max_prompt, the
        scaled token embeddings); noise [chunk, action]."""
        d = self.d
        n = int(prompt_rows.shape[0])
        if not 1 <= n <= d.max_prompt:
            raise ValueError(f"prompt rows must be 1..{d.max_prompt}, got {n}")
        self.images.copy_(images)
        self.prompt.zero_()
        self.prompt[:n].copy_(prompt_rows)
        self.noise.copy_(noise)
        valid = d.image_rows + n
        self.n_prefix.fill_(valid)
        self.n_keys.fill_(valid + d.chunk)
        torch.arange(valid, valid + d.chunk, out=self.pos_chunk[:, 0])

    # ---------------------------------------------------------------- schedule
    def _op(self, rows, cols):
        return self.op8[: rows * cols].view(rows, cols)

    def _add(self, name, kind, fn, **io):
        self.schedule.append(Launch(name, kind, fn, io))

    def _linear(self, name, rows, cols, w, out, *, act=None, residual=False, ref=None):
        a, s = self._op(rows, cols), self.op_scale[:rows]
        res = out if residual else None
        self._add(name, "linear", lambda: linear(a, s, w, out=out, act=act, residual=res),
                  a=a, s=s, w=ref, out=out, act=act, residual=residual)

    def _norm(self, name, res, **kw):
        self._add(name, "norm", lambda: residual_norm_quant(res, **kw), res=res, **kw)

    def _quant(self, name, x, rows, cols):
        q, s = self._op(rows, cols), self.op_scale[:rows]
        if x.dtype == torch.float16:
            self._add(name, "quant", lambda: row_quant(x, q, s), x=x, q=q, s=s)
        else:
            self._add(name, "quant", lambda: quant_rows(x, q, s), x=x, q=q, s=s)

    def _attention(self, name, q, k, v, *, scale, out=None, kv_len=None, q8=None, split=None):
        s = self.op_scale[: q.shape[1]] if q8 is not None else None
        self._add(name, "attention",
                  lambda: attention(q, k, v, out=out, kv_len=kv_len, scale=scale, split=split, q8=q8, q8_scale=s),
                  q=q, k=k, v=v, out=out, kv_len=kv_len, scale=scale, q8=q8, q8_scale=s)

    def _plan_vision(self):
        p, d = self.p, self.d
        T, D, FF = d.image_rows, d.vis_d, d.vis_ff
        s = self.op_scale[:T]

        def embed():
            # 14 x 14 patches: pixel (row, col, channel) vectors times the patch weight
            pix = self.images.view(d.views, 3, 16, 14, 16, 14).permute(0, 2, 4, 3, 5, 1).reshape(T, 588)
            torch.mm(pix.half(), p.patch_w, out=self.vis_ctx)
            torch.add(self.vis_ctx, p.patch_b, out=self.vis_stream)
            self.vis_stream.view(d.views, d.patches, D).add_(p.pos_emb)
        self._add("vision.embed", "torch", embed)
        heads = self.vis_qkv.view(d.views, d.patches, 3, d.vis_heads, d.vis_hd)
        ctx = self.vis_ctx.view(d.views, d.patches, d.vis_heads, d.vis_hd)
        for i, blk in enumerate(p.vision):
            tag = f"vision{i}"
            self._norm(f"{tag}.ln1", self.vis_stream, layernorm=True, weight=blk.ln1[0], beta=blk.ln1[1],
                       q=self._op(T, D), q_scale=s)
            self._linear(f"{tag}.qkv", T, D, blk.qkv, self.vis_qkv, ref=f"v{i}.qkv")
            self._attention(f"{tag}.attention", heads[:, :, 0], heads[:, :, 1], heads[:, :, 2], out=ctx,
                            scale=d.vis_hd ** -0.5)
            self._quant(f"{tag}.quant_ctx", self.vis_ctx, T, D)
            self._linear(f"{tag}.o", T, D, blk.o, self.vis_stream, residual=True, ref=f"v{i}.o")
            self._norm(f"{tag}.ln2", self.vis_stream, layernorm=True, weight=blk.ln2[0], beta=blk.ln2[1],
                       q=self._op(T, D), q_scale=s)
            self._linear(f"{tag}.fc1", T, D, blk.fc1, self.vis_mlp, act="gelu_tanh", ref=f"v{i}.fc1")
            self._quant(f"{tag}.quant_mlp", self.vis_mlp, T, FF)
            self._linear(f"{tag}.fc2", T, FF, blk.fc2, self.vis_stream, residual=True, ref=f"v{i}.fc2")
        self._norm("vision.post_ln", self.vis_stream, layernorm=True, weight=p.post_ln[0], beta=p.post_ln[1],
                   q=self._op(T, D), q_scale=s)
        self._linear("vision.projector", T, D, p.projector, self.lm_stream[:T], ref="projector")

    def _plan_prefix(self):
        p, d = self.p, self.d
        S, D, HD, T = self.rows, d.lm_d, d.head_dim, d.image_rows
        s = self.op_scale[:S]
        self._add("prefix.prompt", "torch", lambda: self.lm_stream[T:].copy_(self.prompt))
        for i, blk in enumerate(p.prefix):
            tag = f"prefix{i}"
            self._norm(f"{tag}.norm_attn", self.lm_stream, q=self._op(S, D), q_scale=s)
            self._linear(f"{tag}.qkv", S, D, blk.qkv, self.lm_qkv, ref=f"p{i}.qkv")
            kv = (self.keys[i], self.values[i])
            self._add(f"{tag}.rope_split", "split",
                      lambda kv=kv: qkv_split(self.lm_qkv, self.lm_q, kv[0], kv[1], heads_q=d.heads, heads_kv=1,
                                              head_dim=HD, inv_freq=self.inv_freq, pos=self.pos_prefix),
                      qkv=self.lm_qkv, q=self.lm_q, k=kv[0], v=kv[1], pos=self.pos_prefix, kv_base=0)
            if blk.o is None:  # the last layer only feeds the expert's K/V
                break
            self._attention(f"{tag}.attention", self.lm_q[None], self.keys[i][None], self.values[i][None],
                            out=self.lm_ctx.view(1, S, d.heads, HD), kv_len=self.n_prefix, scale=HD ** -0.5)
            self._quant(f"{tag}.quant_ctx", self.lm_ctx, S, d.heads * HD)
            self._linear(f"{tag}.o", S, d.heads * HD, blk.o, self.lm_stream, residual=True, ref=f"p{i}.o")
            self._norm(f"{tag}.norm_mlp", self.lm_stream, q=self._op(S, D), q_scale=s)
            self._linear(f"{tag}.gate_up", S, D, blk.gate_up, self.lm_mlp, act="geglu", ref=f"p{i}.gate_up")
            self._quant(f"{tag}.quant_mlp", self.lm_mlp, S, d.lm_ff)
            self._linear(f"{tag}.down", S, d.lm_ff, blk.down, self.lm_stream, residual=True, ref=f"p{i}.down")

    def _plan_expert(self):
        p, d = self.p, self.d
        A, D, HD = d.chunk, d.ex_d, d.head_dim
        s = self.op_scale[:A]
        last = len(p.expert) - 1
        self._add("expert.noise", "torch", lambda: self.actions.copy_(self.noise))
        for t in range(d.steps):
            ma, mf = p.mod_attn[t], p.mod_ffn[t]
            self._add(f"step{t}.action_in", "torch",
                      lambda: torch.addmm(p.action_in[1], self.actions, p.action_in[0], out=self.ex_stream))
            self._norm(f"step{t}.norm0", self.ex_stream, mod_scale=ma[0, 0], mod_shift=ma[0, 1],
                       q=self._op(A, D), q_scale=s)
            for i, blk in enumerate(p.expert):
                tag = f"step{t}.layer{i}"
                a, kv = self._op(A, D), (self.keys[i], self.values[i])
                self._add(f"{tag}.qkv_rope", "qkv_rope",
                          lambda blk=blk, a=a, kv=kv: linear_qkv_rope(
                              a, s, blk.qkv, self.ex_q, kv[0], kv[1], inv_freq=self.inv_freq, pos=self.pos_chunk,
                              kv_base=self.n_prefix),
                          a=a, s=s, w=f"e{i}.qkv", q=self.ex_q, k=kv[0], v=kv[1], pos=self.pos_chunk,
                          kv_base=self.n_prefix)
                self._attention(f"{tag}.attention", self.ex_q[None], self.keys[i][None], self.values[i][None],
                                kv_len=self.n_keys, scale=HD ** -0.5, q8=self._op(A, d.heads * HD),
                                split=self.ex_split)
                self._linear(f"{tag}.o", A, d.heads * HD, blk.o, self.ex_proj, ref=f"e{i}.o")
                self._norm(f"{tag}.norm_mlp", self.ex_stream, delta=self.ex_proj, gate=ma[i, 2],
                           mod_scale=mf[i, 0], mod_shift=mf[i, 1], q=self._op(A, D), q_scale=s)
                self._linear(f"{tag}.gate_up", A, D, blk.gate_up, self.ex_mlp, act="geglu", ref=f"e{i}.gate_up")
                self._quant(f"{tag}.quant_mlp", self.ex_mlp, A, d.ex_ff)
                self._linear(f"{tag}.down", A, d.ex_ff, blk.down, self.ex_proj, ref=f"e{i}.down")
                if i < last:
                    self._norm(f"{tag}.norm_attn", self.ex_stream, delta=self.ex_proj, gate=mf[i, 2],
                               mod_scale=ma[i + 1, 0], mod_shift=ma[i + 1, 1], q=self._op(A, D), q_scale=s)
                else:
                    self._norm(f"{tag}.norm_out", self.ex_stream, delta=self.ex_proj, gate=mf[i, 2],
                               mod_scale=p.mod_final[t, 0], mod_shift=p.mod_final[t, 1], y=self.ex_out)
            self._add(f"step{t}.euler", "torch",
                      lambda: self.actions.addmm_(self.ex_out, self.out_w).add_(self.out_b))

    # --------------------------------------------------------------- execution
    def run(self):
        for launch in self.schedule:
            launch.fn()
        return self.actions

    def capture(self):
        """Warm on a side stream, then capture the whole schedule into one graph."""
        side = torch.cuda.Stream(self.dev)
        side.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(side):
            self.run()
        torch.cuda.current_stream(self.dev).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            self.run()
        return graph
