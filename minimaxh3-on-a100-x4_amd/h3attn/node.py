"""ComfyUI node "H3SLAPatch" on libh3attn: the h3_sla node's inputs and output
(custom_nodes/h3_sla/__init__.py:308-349), so that a workflow saved with that
node loads and runs here.  A custom node's __init__.py re-exports
NODE_CLASS_MAPPINGS / NODE_DISPLAY_NAME_MAPPINGS from this module.

The work is hooks.patch_model: clone the model, install the DiT scope patch,
tag the layers and set the block-sparse override with its per-layer schedule.
"""
from __future__ import annotations

from . import hooks, sla


class H3SLAPatch:
    @classmethod
    def INPUT_TYPES(cls):
        # Input names, types and defaults are the node's; blk offers the sizes the kernels run.
        lo, hi = min(sla.SUPPORTED_BLOCKS), max(sla.SUPPORTED_BLOCKS)
        return {
            "required": {
                "model": ("MODEL",),
                "topk": ("FLOAT", {"default": 0.35, "min": 0.02, "max": 1.0, "step": 0.01,
                                   "tooltip": "fraction of key blocks each query block keeps (1 - sparsity)"}),
                "blk": ("INT", {"default": 64, "min": lo, "max": hi, "step": sla.BLOCK_STEP,
                                "tooltip": "query and key block size (64, 128, 192 and 256 run the "
                                           "native kernels, the other sizes 32-key columns with sub-block masks)"}),
                "enabled": ("BOOLEAN", {"default": True}),
            },
            "optional": {
                "preset": (sla.PRESET_CHOICES, {"default": "off",
                                                "tooltip": "off: topk on every layer; quality / balanced / speed: "
                                                           "per-layer presets; custom: layer_keep"}),
                "layer_keep": ("STRING", {"default": "",
                                          "tooltip": "custom only, e.g. '25:31-42,46-49;20:43' "
                                                     "(percent or ratio : layer ranges); other layers keep topk"}),
            },
        }

    RETURN_TYPES = ("MODEL",)
    FUNCTION = "patch"
    CATEGORY = "MiniMaxH3"

    def patch(self, model, topk, blk, enabled, preset="off", layer_keep=""):
        return (hooks.patch_model(model, topk=topk, blk=blk, enabled=enabled, preset=preset,
                                  layer_keep=layer_keep),)


NODE_CLASS_MAPPINGS = {"H3SLAPatch": H3SLAPatch}
NODE_DISPLAY_NAME_MAPPINGS = {"H3SLAPatch": "H3 SLA Sparse Attention (MI355X)"}
