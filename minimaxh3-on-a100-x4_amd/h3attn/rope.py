"""RoPE rotation tables in ComfyUI's rope_freqs layout.

ComfyUI DiTs hand the attention a float32 tensor [B, S, 1, rot/2, 2, 2] of
2x2 rotation matrices [[cos, -sin], [sin, cos]] (rot_dim = shape[-3] * 2,
harness/sp_runtime.py:97; token axis = dim 1, harness/sp_runtime.py:233-238).
"""
from __future__ import annotations

import torch


def rope_freqs(S: int, rot_dim: int, theta: float = 10000.0, positions: torch.Tensor | None = None,
               device=None) -> torch.Tensor:
    """1-D RoPE table: angle(s, i) = pos[s] * theta^(-2i/rot_dim), i < rot_dim/2.

    Returns float32 [1, S, 1, rot_dim/2, 2, 2].
    """
    if rot_dim <= 0 or rot_dim % 2:
        raise ValueError("rot_dim must be a positive even number")
    pos = (torch.arange(S, dtype=torch.float64) if positions is None
           else positions.to(torch.float64).reshape(-1).cpu())
    i = torch.arange(rot_dim // 2, dtype=torch.float64)
    omega = theta ** (-2.0 * i / rot_dim)
    ang = pos[:, None] * omega[None, :]
    c, s = torch.cos(ang), torch.sin(ang)
    table = torch.stack([c, -s, s, c], dim=-1).reshape(len(pos), rot_dim // 2, 2, 2)
    return table.to(torch.float32).reshape(1, len(pos), 1, rot_dim // 2, 2, 2).to(device)
