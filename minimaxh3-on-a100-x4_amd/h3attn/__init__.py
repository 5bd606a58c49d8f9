"""h3attn - MI355X (gfx950) exact attention path of the MiniMax-H3 video DiT.

Python side of libh3attn: tensor entry points (ops), the block-sparse h3_sla
path (sla), the ComfyUI drop-in hooks (hooks), RoPE tables (rope), HIP-graph
capture of layer sequences (graphs) and per-component timing (profiling).  All
arithmetic happens in the HIP kernels of libh3attn.so; nothing here computes
attention on the CPU.
"""
from ._lib import H3AError, LIB_PATH, version
from .ops import (attn_fwd, attn_fwd_blocksparse, block_map_to_lut, kernel_attrs,
                  qk_rmsnorm_rope_, rms_rope_split_half_, test_pv, test_qk)
from .rope import rope_freqs

__all__ = [
    "H3AError", "LIB_PATH", "version", "attn_fwd", "attn_fwd_blocksparse", "block_map_to_lut",
    "kernel_attrs", "qk_rmsnorm_rope_", "rms_rope_split_half_", "test_qk", "test_pv", "rope_freqs",
]
