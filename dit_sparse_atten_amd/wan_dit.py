"""A Wan2.1-shaped video DiT and its denoising loop, for end-to-end timing of
the attention backends (random initialisation; no checkpoints are loaded).

The reference times its backends inside Wan's own model through Diffusers
(wan_diffusers.py:75-191, infer.py:180-223).  This module rebuilds that
model's shape so the same loop runs here:
  * patch embedding (1 x 2 x 2 patches of 16 latent channels), text MLP
    (4096 -> dim, GELU-tanh, dim -> dim), sinusoidal time MLP and the six
    per-block modulation vectors;
  * per block: LayerNorm + modulation, self-attention with RMSNorm-ed Q/K and
    3D RoPE through the selected backend, gated residual; LayerNorm (affine) and
    cross-attention over the text tokens; LayerNorm + modulation, GELU-tanh FFN,
    gated residual;
  * output LayerNorm + modulation, projection and unpatchify;
  * 5-step flow-matching loop on Wan's shifted schedule (shift 5:
    t = 999, 952, 882, 768, 555, as the reference's runs record them) with a
    classifier-free-guidance pair per step (branch 0 conditional, branch 1
    unconditional); the update is a plain Euler step, where Wan uses a
    multistep solver: the model calls, which are what is timed, are the same.
GEMMs go through torch (hipBLASLt, the FFN's GELU-tanh in the GEMM epilogue);
the norms, modulation, RoPE and residuals are libdsa HIP kernels; self-attention is whatever backend the caller passes,
cross-attention is the dense libdsa kernel.  The routing context (layer,
step, branch, grid) is set before every self-attention call, as the
reference's context hooks do (context.py:43-49).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import ops
from .attention_backends.context import set_routing_context


@dataclass(frozen=True)
class WanDiTConfig:
    """Wan2.1-T2V-1.3B shape."""

    layers: int = 30
    dim: int = 1536
    heads: int = 12
    ffn_dim: int = 8960
    text_dim: int = 4096
    freq_dim: int = 256
    in_channels: int = 16
    out_channels: int = 16
    patch: tuple = (1, 2, 2)
    eps: float = 1e-6
    # > 0: every block's q and k projections share one random bias vector of
    # this scale.  After RMSNorm and 3D RoPE its self-product depends only on
    # the relative (frame, y, x) offset and peaks at zero, so attention gains
    # the spatial locality of a trained video DiT.  0: plain random init.
    qk_position_bias: float = 0.0
    # Scale of the self-attention q/k RMSNorm weights (a softmax temperature:
    # scores scale with its square).  1: the plain random init.
    qk_norm_scale: float = 1.0

    @property
    def head_dim(self):
        return self.dim // self.heads


def rope_cos_sin(grid, head_dim=128, theta=10000.0, device=None):
    """fp32 [tokens, head_dim / 2, 2] (cos, sin) of Wan's 3D RoPE over the
    (F, H, W) patch grid, flattened frame-major: the head dims split into a
    time part of head_dim - 4 * (head_dim // 6) and two spatial parts of
    2 * (head_dim // 6), each rotating consecutive pairs by
    position * theta^(-2j / part)."""
    frames, height, width = grid
    spatial = 2 * (head_dim // 6)
    parts = (head_dim - 2 * spatial, spatial, spatial)
    axes = [torch.arange(n, dtype=torch.float64) for n in (frames, height, width)]
    positions = torch.stack(torch.meshgrid(*axes, indexing="ij"), dim=-1).reshape(-1, 3)
    angles = torch.cat([
        positions[:, a:a + 1] * theta ** (-torch.arange(0, part, 2, dtype=torch.float64) / part)
        for a, part in enumerate(parts)], dim=-1)
    table = torch.stack([torch.cos(angles), torch.sin(angles)], dim=-1).to(torch.float32)
    return table.contiguous().to(device) if device is not None else table.contiguous()


def flow_timesteps(steps=5, shift=5.0, train_steps=1000):
    """Wan's shifted flow-matching schedule: sigmas from 1 - 1/train_steps down
    to 0, shifted as shift * s / (1 + (shift - 1) * s), and the integer
    timesteps floor(sigma * train_steps) of every step (999, 952, 882, 768,
    555 for 5 steps at shift 5, as the reference's runs record them)."""
    sigmas = torch.linspace(1.0 - 1.0 / train_steps, 0.0, steps + 1, dtype=torch.float64)
    shifted = shift * sigmas / (1 + (shift - 1) * sigmas)
    return shifted, torch.floor(shifted[:-1] * train_steps)


def _sinusoidal(t, dim):
    half = dim // 2
    freqs = torch.exp(-math.log(10000.0) * torch.arange(half, dtype=torch.float64) / half)
    args = float(t) * freqs
    return torch.cat([torch.cos(args), torch.sin(args)]).to(torch.float32)


class WanDiT:
    """Random-initialised Wan2.1-shaped DiT on one HIP device (bf16 weights)."""

    def __init__(self, config=None, device="cuda", seed=0):
        self.config = c = config or WanDiTConfig()
        self.device = torch.device(device)
        # Weights are drawn on the device (1.3B values would take seconds on the host).
        gen = torch.Generator(device=self.device).manual_seed(seed)

        def randn(*shape):
            return torch.randn(*shape, generator=gen, device=self.device)

        def linear(out_features, in_features):
            w = randn(out_features, in_features) / math.sqrt(in_features)
            return w.to(torch.bfloat16), (randn(out_features) * 0.02).to(torch.bfloat16)

        def vector(n, scale=0.02, offset=0.0):
            return offset + randn(n) * scale

        patch_in = c.in_channels * math.prod(c.patch)
        self.patch = linear(c.dim, patch_in)
        self.text1, self.text2 = linear(c.dim, c.text_dim), linear(c.dim, c.dim)
        self.time1, self.time2 = linear(c.dim, c.freq_dim), linear(c.dim, c.dim)
        self.time_proj = linear(6 * c.dim, c.dim)
        self.blocks = []
        for _ in range(c.layers):
            q_proj, k_proj = linear(c.dim, c.dim), linear(c.dim, c.dim)
            if c.qk_position_bias > 0:
                shared = (randn(c.dim) * c.qk_position_bias).to(torch.bfloat16)
                q_proj, k_proj = (q_proj[0], shared), (k_proj[0], shared)
            self.blocks.append({
                "table": randn(6, c.dim) / math.sqrt(c.dim),
                "q": q_proj, "k": k_proj,
                "v": linear(c.dim, c.dim), "o": linear(c.dim, c.dim),
                "norm_q": vector(c.dim, offset=1.0) * c.qk_norm_scale,
                "norm_k": vector(c.dim, offset=1.0) * c.qk_norm_scale,
                "cq": linear(c.dim, c.dim), "ck": linear(c.dim, c.dim),
                "cv": linear(c.dim, c.dim), "co": linear(c.dim, c.dim),
                "cnorm_q": vector(c.dim, offset=1.0), "cnorm_k": vector(c.dim, offset=1.0),
                "norm2_w": vector(c.dim, offset=1.0), "norm2_b": vector(c.dim),
                "ffn1": linear(c.ffn_dim, c.dim), "ffn2": linear(c.dim, c.ffn_dim),
            })
        self.head_table = randn(2, c.dim) / math.sqrt(c.dim)
        self.head = linear(c.out_channels * math.prod(c.patch), c.dim)
        self._rope = {}

    def _cos_sin(self, grid):
        if grid not in self._rope:
            self._rope[grid] = rope_cos_sin(grid, self.config.head_dim, device=self.device)
        return self._rope[grid]

    def embed_text(self, context):
        """[1, L, text_dim] bf16 -> [1, L, dim] (Linear, GELU-tanh, Linear)."""
        h = F.gelu(F.linear(context, *self.text1), approximate="tanh")
        return F.linear(h, *self.text2)

    def _block(self, x, blk, ctx, temb6, cos_sin, backend):
        c = self.config
        batch, tokens, _ = x.shape
        heads, head_dim = c.heads, c.head_dim
        mod = blk["table"] + temb6  # [6, dim] fp32
        h = ops.layernorm_modulate(x, shift=mod[0:1], scale=mod[1:2], eps=c.eps)
        q = ops.rmsnorm_rope(F.linear(h, *blk["q"]), blk["norm_q"], head_dim, cos_sin, c.eps)
        k = ops.rmsnorm_rope(F.linear(h, *blk["k"]), blk["norm_k"], head_dim, cos_sin, c.eps)
        v = F.linear(h, *blk["v"])
        shape = (batch, tokens, heads, head_dim)
        attn = backend(q.view(shape), k.view(shape), v.view(shape), dtype=torch.bfloat16)
        o = F.linear(attn.reshape(batch, tokens, c.dim), *blk["o"])
        x = ops.gated_residual(x, o, gate=mod[2:3], out=x)
        # Cross-attention over the text tokens (dense kernel, no RoPE).
        h = ops.layernorm_modulate(x, weight=blk["norm2_w"], bias=blk["norm2_b"], eps=c.eps)
        q = ops.rmsnorm_rope(F.linear(h, *blk["cq"]), blk["cnorm_q"], head_dim, None, c.eps)
        k = ops.rmsnorm_rope(F.linear(ctx, *blk["ck"]), blk["cnorm_k"], head_dim, None, c.eps)
        v = F.linear(ctx, *blk["cv"])
        ctx_shape = (batch, ctx.shape[1], heads, head_dim)
        attn = ops.bsa_fwd(q.view(shape), k.view(ctx_shape), v.view(ctx_shape))
        x = ops.gated_residual(x, F.linear(attn.reshape(batch, tokens, c.dim), *blk["co"]),
                               out=x)
        # Feed-forward; the GELU-tanh runs in the GEMM's epilogue (hipBLASLt).
        h = ops.layernorm_modulate(x, shift=mod[3:4], scale=mod[4:5], eps=c.eps)
        w1, b1 = blk["ffn1"]
        f = torch._addmm_activation(b1, h.view(-1, c.dim), w1.t(), use_gelu=True)
        f = F.linear(f, *blk["ffn2"]).view(batch, tokens, c.dim)
        return ops.gated_residual(x, f, gate=mod[5:6], out=x)

    def forward(self, latents, timestep, ctx, backend, step=0, branch=0):
        """latents [1, C, F, H, W] bf16; ctx = embed_text(text) -> noise prediction."""
        c = self.config
        _, channels, frames, height, width = latents.shape
        pf, ph, pw = c.patch
        grid = (frames // pf, height // ph, width // pw)
        tokens = math.prod(grid)
        patches = latents.reshape(1, channels, grid[0], pf, grid[1], ph, grid[2], pw)
        patches = patches.permute(0, 2, 4, 6, 1, 3, 5, 7).reshape(1, tokens, -1)
        x = F.linear(patches, *self.patch).contiguous()
        t = _sinusoidal(timestep, c.freq_dim).to(self.device)
        temb = F.linear(F.silu(F.linear(t.to(torch.bfloat16), *self.time1)), *self.time2)
        temb6 = F.linear(F.silu(temb), *self.time_proj).float().view(6, c.dim)
        cos_sin = self._cos_sin(grid)
        for layer, blk in enumerate(self.blocks):
            set_routing_context(attention_id=layer, step=step, branch=branch, grid=grid)
            x = self._block(x, blk, ctx, temb6, cos_sin, backend)
        shift_scale = self.head_table + temb.float().view(1, c.dim)
        h = ops.layernorm_modulate(x, shift=shift_scale[0:1], scale=shift_scale[1:2], eps=c.eps)
        out = F.linear(h, *self.head)
        out = out.reshape(1, grid[0], grid[1], grid[2], c.out_channels, pf, ph, pw)
        return out.permute(0, 4, 1, 5, 2, 6, 3, 7).reshape(latents.shape)

    __call__ = forward


def denoise(model, backend, latents, text_cond, text_uncond, steps=5, guidance=5.0,
            shift=5.0, on_call=None):
    """Flow-matching Euler loop with classifier-free guidance: per step the
    conditional (branch 0) then the unconditional (branch 1) forward.
    ``on_call(step, branch, phase)`` is invoked with phase "start" right
    before and "end" right after every model call (the reference times each
    call the same way, infer.py:180-223)."""
    sigmas, timesteps = flow_timesteps(steps, shift)
    contexts = (model.embed_text(text_cond), model.embed_text(text_uncond))
    x = latents
    for step in range(steps):
        preds = []
        for branch, ctx in enumerate(contexts):
            if on_call:
                on_call(step, branch, "start")
            preds.append(model(x, float(timesteps[step]), ctx, backend, step=step, branch=branch))
            if on_call:
                on_call(step, branch, "end")
        cond, uncond = preds
        noise = uncond.float() + guidance * (cond.float() - uncond.float())
        x = (x.float() + float(sigmas[step + 1] - sigmas[step]) * noise).to(latents.dtype)
    return x
