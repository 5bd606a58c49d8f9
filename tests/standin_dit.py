"""Stand-in for the un-vendored comfy.ldm.minimax.model pieces the hooks touch.

Restates the stock DiT attention forward exactly as the reference does at
custom_nodes/h3_profiler/__init__.py:92-111 (and harness/sp_runtime.py:89-102):
qkv_proj -> split -> rms_rope_split_half_ on [1,S,H,D] views (rope path) or
per-head RMSNorm (no-rope path) -> [1,H,S,D] -> optimized_attention(...,
skip_reshape=True) -> [S,H*D] -> out_proj.  The prologue and attention here are
plain torch (fp32 math), i.e. the "stock" math the patched forward must match.
"""
from __future__ import annotations

import copy
import types

import torch
import torch.nn as nn


def rms_rope_split_half_(q, k, rope_freqs, qw, kw, epsilon=1e-6, rot_dim=None):
    """Torch restatement of the prologue contract, in place on [B,S,H,D] views."""
    B, S, H, D = q.shape
    rot = rope_freqs.shape[-3] * 2 if rot_dim is None else rot_dim
    for t, w in ((q, qw), (k, kw)):
        x = t.float()
        y = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + epsilon) * w.float()
        if rot:
            half = rot // 2
            R = rope_freqs.float().reshape(rope_freqs.shape[0], S, 1, half, 2, 2)
            a, c = y[..., :half], y[..., half:rot]
            y = torch.cat([R[..., 0, 0] * a + R[..., 0, 1] * c, R[..., 1, 0] * a + R[..., 1, 1] * c,
                           y[..., rot:]], dim=-1)
        t.copy_(y.to(t.dtype))


def _attention_impl(q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                    skip_output_reshape=False, transformer_options=None):
    if not skip_reshape:
        B, S, HD = q.shape
        q, k, v = (t.view(B, -1, heads, HD // heads).transpose(1, 2) for t in (q, k, v))
    o = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(),
                                                         attn_mask=mask).to(q.dtype)
    if skip_output_reshape:
        return o
    B, H, S, D = o.shape
    return o.transpose(1, 2).reshape(B, S, H * D)


def optimized_attention(q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                        skip_output_reshape=False, transformer_options={}):
    """ComfyUI entry: honours transformer_options['optimized_attention_override']."""
    kw = dict(mask=mask, attn_precision=attn_precision, skip_reshape=skip_reshape,
              skip_output_reshape=skip_output_reshape, transformer_options=transformer_options)
    ov = (transformer_options or {}).get("optimized_attention_override")
    if ov is not None:
        return ov(_attention_impl, q, k, v, heads, **kw)
    return _attention_impl(q, k, v, heads, **kw)


class RMSNorm(nn.Module):
    def __init__(self, dim, eps=1e-6, dtype=None, device=None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, dtype=dtype, device=device))

    def forward(self, x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps) * self.weight.float()).to(x.dtype)


class Attention(nn.Module):
    def __init__(self, dim, heads, head_dim=128, eps=1e-6, dtype=None, device=None):
        super().__init__()
        self.heads, self.head_dim = heads, head_dim
        self.qkv_proj = nn.Linear(dim, 3 * heads * head_dim, bias=False, dtype=dtype, device=device)
        self.out_proj = nn.Linear(heads * head_dim, dim, bias=False, dtype=dtype, device=device)
        self.q_norm = RMSNorm(head_dim, eps, dtype=dtype, device=device)
        self.k_norm = RMSNorm(head_dim, eps, dtype=dtype, device=device)

    def forward(self, x, rope_freqs=None, transformer_options={}):
        s = x.shape[0]
        q, k, v = self.qkv_proj(x).split(self.heads * self.head_dim, dim=-1)
        v = v.view(s, self.heads, self.head_dim)
        if rope_freqs is not None:
            q = q.view(1, s, self.heads, self.head_dim)
            k = k.view(1, s, self.heads, self.head_dim)
            rot = rope_freqs.shape[-3] * 2
            rms_rope_split_half_(q, k, rope_freqs, self.q_norm.weight, self.k_norm.weight,
                                 epsilon=self.q_norm.eps, rot_dim=rot)
            q, k = q[0], k[0]
        else:
            q = self.q_norm(q.view(s, self.heads, self.head_dim))
            k = self.k_norm(k.view(s, self.heads, self.head_dim))
        q, k, v = (t.transpose(0, 1).unsqueeze(0) for t in (q, k, v))
        out = optimized_attention(q, k, v, self.heads, mask=None, skip_reshape=True,
                                  transformer_options=transformer_options)
        return self.out_proj(out.squeeze(0))


class DiTBlock(nn.Module):
    """A DiT block reduced to what the hooks touch: its self-attention at `.attn`."""

    def __init__(self, dim, heads, attention_cls=Attention, dtype=None, device=None):
        super().__init__()
        self.attn = attention_cls(dim, heads, dtype=dtype, device=device)

    def forward(self, x, rope_freqs=None, transformer_options={}):
        return x + self.attn(x, rope_freqs=rope_freqs, transformer_options=transformer_options)


class MiniMaxH3Model(nn.Module):
    """`depth` DiT blocks run in order (the diffusion model's block loop, without the MLPs)."""

    def __init__(self, dim, heads, depth=50, attention_cls=Attention, dtype=None, device=None):
        super().__init__()
        self.blocks = nn.ModuleList(DiTBlock(dim, heads, attention_cls, dtype, device) for _ in range(depth))

    def forward(self, x, rope_freqs=None, transformer_options={}):
        for block in self.blocks:
            x = block(x, rope_freqs=rope_freqs, transformer_options=transformer_options)
        return x


class ModelPatcher:
    """The parts of ComfyUI's ModelPatcher a model-patching node uses: .model.diffusion_model,
    .model_options (with "transformer_options") and clone(), which shares the weights."""

    def __init__(self, diffusion_model, model_options=None):
        self.model = types.SimpleNamespace(diffusion_model=diffusion_model)
        self.model_options = {"transformer_options": {}} if model_options is None else model_options

    def clone(self):
        return ModelPatcher(self.model.diffusion_model, copy.deepcopy(self.model_options))

    def __call__(self, x, rope_freqs, sigma=None, sample_sigmas=None):
        """One sampling step: the diffusion model under this patcher's transformer_options, with the
        step's sigma and the run's sigma schedule added as the sampler adds them."""
        opts = dict(self.model_options.get("transformer_options", {}))
        if sigma is not None:
            opts["sigmas"] = torch.tensor([float(sigma)])
        if sample_sigmas is not None:
            opts["sample_sigmas"] = torch.tensor([float(s) for s in sample_sigmas])
        return self.model.diffusion_model(x, rope_freqs=rope_freqs, transformer_options=opts)
