"""Block-sparse attention for the h3_sla path (custom_nodes/h3_sla/__init__.py).

The reference runs thu-ml/SLA's `get_block_map` (mean-pooled q.k^T scores,
top-k key blocks per query block) and SLA's Triton `_attention` over the kept
blocks (custom_nodes/h3_sla/__init__.py:226-235).  Here libh3attn pools q and k
per block, selects the kept key blocks straight into the LUT form, and runs the
gfx950 block-sparse kernel, which never touches a skipped key block.

Also mirrors the node's per-layer keep schedule (PRESETS, parse_ranges,
parse_layer_keep, resolve_schedule; custom_nodes/h3_sla/__init__.py:44-96),
whose table of presets must stay identical to the reference's.
"""
from __future__ import annotations

import math

import torch

from . import ops

# Per-layer keep presets; the table is the reference's
# (custom_nodes/h3_sla/__init__.py:44-49): every layer not listed keeps default_keep.
PRESETS = {
    "quality": {"default_keep": 0.15, "layers": {0.25: "31-42,46-49"}, "research_name": "E8"},
    "balanced": {"default_keep": 0.15, "layers": {0.25: "31-42,48-49"}, "research_name": "T2"},
    "speed": {"default_keep": 0.15, "layers": {0.25: "34-42"}, "research_name": "E3"},
}
PRESET_CHOICES = ["off", "quality", "balanced", "speed", "custom"]


def parse_ranges(spec) -> list[int]:
    """'31-42,46,48-49' -> [31, ..., 42, 46, 48, 49] (custom_nodes/h3_sla/__init__.py:57-63)."""
    layers: list[int] = []
    for item in str(spec).split(","):
        item = item.strip()
        if not item:
            continue
        lo, sep, hi = item.partition("-")
        first = int(lo)
        last = int(hi) if sep and hi else first
        layers.extend(range(first, last + 1))
    return layers


def parse_layer_keep(spec) -> dict[int, float]:
    """'25:31-42,46-49;20:43' -> {layer: keep}; values > 1 are percentages (h3_sla:66-74)."""
    out: dict[int, float] = {}
    for part in str(spec).split(";"):
        part = part.strip()
        if not part:
            continue
        val, _, ranges = part.partition(":")
        keep = float(val)
        if keep > 1.0:
            keep /= 100.0
        for layer in parse_ranges(ranges):
            out[layer] = keep
    return out


def resolve_schedule(preset="off", topk=0.35, layer_keep="", n_layers=50):
    """-> (name, [keep per layer]) (custom_nodes/h3_sla/__init__.py:77-96)."""
    name = (preset or "off").lower()
    if name == "off":
        return "off", [float(topk)] * n_layers
    keeps = [float(topk)] * n_layers
    if name == "custom":
        for layer, keep in parse_layer_keep(layer_keep).items():
            if 0 <= layer < n_layers:
                keeps[layer] = keep
        return "custom", keeps
    if name not in PRESETS:
        raise ValueError(f"unknown SLA preset {name!r}; choose one of {PRESET_CHOICES}")
    spec = PRESETS[name]
    keeps = [float(spec["default_keep"])] * n_layers
    for keep, ranges in spec["layers"].items():
        for layer in parse_ranges(ranges):
            if 0 <= layer < n_layers:
                keeps[layer] = float(keep)
    return name, keeps


def _ranges_str(layers) -> str:
    """[31, 32, 33, 46] -> '31-33,46' (the inverse of parse_ranges)."""
    ls = sorted(layers)
    out = []
    i = 0
    while i < len(ls):
        j = i
        while j + 1 < len(ls) and ls[j + 1] == ls[j] + 1:
            j += 1
        out.append(f"{ls[i]}-{ls[j]}" if j > i else f"{ls[i]}")
        i = j + 1
    return ",".join(out)


def schedule_summary(name: str, keeps, blk: int = 64) -> dict:
    """Summary of a per-layer schedule (custom_nodes/h3_sla/__init__.py:110-124).

    Same keys as the node's, except its latency predictions, which are fits of
    A100 SP-2 measurements and do not describe this hardware.
    """
    keeps = [float(x) for x in keeps]
    counts: dict[str, int] = {}
    for kv in keeps:
        key = f"{round(kv * 100)}"
        counts[key] = counts.get(key, 0) + 1
    default = max(set(keeps), key=keeps.count)
    by = {f"SLA{round(kv * 100)}": _ranges_str([i for i, x in enumerate(keeps) if x == kv])
          for kv in sorted(set(keeps)) if kv != default}
    return {"preset": name, "research_name": PRESETS.get(name, {}).get("research_name"),
            "default_keep": default, "layers_by_keep": by, "counts": counts,
            "keeps": [round(x, 4) for x in keeps], "blk": int(blk)}


def format_summary(sm: dict) -> str:
    """Log lines of a schedule summary (custom_nodes/h3_sla/__init__.py:127-136), '[h3_sla] '-prefixed."""
    head = f"SLA preset: {sm['preset']}"
    if sm.get("research_name"):
        head += f" (research {sm['research_name']})"
    lines = [head, f"default keep: {round(sm['default_keep'] * 100)}%"]
    for name, ranges in sm["layers_by_keep"].items():
        lines.append(f"{name} layers: {ranges}")
    lines.append("layer counts: " + ", ".join(f"SLA{k}={v}" for k, v in sorted(sm["counts"].items())))
    return "\n".join("[h3_sla] " + x for x in lines)


# ---------------------------------------------------------------------------
# Block sizes (query and key blocks alike): those the h3_sla node offers, 16 to
# 256 in steps of 16 (custom_nodes/h3_sla/__init__.py:315).  The multiples of
# the kernels' 64-key stage (ops.NATIVE_BLOCKS) run the native block-sparse
# kernels; the others run over 32-key columns with 16x16 sub-block masks
# (ops.attn_fwd_blocksparse_tiles).  Anything else is refused up front.
BLOCK_STEP = 16
SUPPORTED_BLOCKS = tuple(range(16, 257, BLOCK_STEP))


def check_block(blk) -> int:
    """Return blk as an int, or raise ValueError if the kernels cannot run it."""
    b = int(blk)
    if b not in SUPPORTED_BLOCKS:
        raise ValueError(f"SLA block size {blk} unsupported by libh3attn; use a multiple of 16 from 16 to 256")
    return b


def keep_count(topk_ratio: float, nk: int) -> int:
    """Key blocks kept by score per query block: floor(ratio * nk), at least 1, at most nk."""
    return max(1, min(nk, int(math.floor(topk_ratio * nk + 1e-9))))


def get_block_map(q: torch.Tensor, k: torch.Tensor, topk_ratio: float, BLKQ: int = 64, BLKK: int = 64,
                  force_diag: bool = False, smooth_k: bool = True, want_map: bool = True, pooled=None):
    """Block map from mean-pooled scores -> (block_map uint8 [B,H,nq,nk] or None, lut int32, counts int32).

    Defaults follow SLA's get_block_map as the h3_sla node calls it
    (custom_nodes/h3_sla/__init__.py:232): top floor(ratio*nk) key blocks by
    pooled score, no forced diagonal.  SLA centres k by its sequence mean
    first (smooth_k); that shifts every score of a query block by the same
    amount and cannot change which key blocks are kept, so the selection is
    computed without it.  The H3 block-sparse workload (128x128 tiles, top 25 %) uses
    force_diag=True.  Pooling and selection run in libh3attn; ties are broken
    towards the lower key-block index.  `pooled`: the block means (pq, pk)
    already taken, by the prologue that wrote q and k
    (ops.qk_rmsnorm_rope_(..., pool_blk=...)); then q and k are not read again.
    """
    del smooth_k  # selection-invariant, see above
    BLKQ, BLKK = check_block(BLKQ), check_block(BLKK)
    if pooled is not None:
        pq, pk = pooled
        want_q = (q.shape[0], q.shape[1], -(-q.shape[2] // BLKQ), q.shape[3])
        want_k = (k.shape[0], k.shape[1], -(-k.shape[2] // BLKK), k.shape[3])
        if tuple(pq.shape) != want_q or tuple(pk.shape) != want_k:
            raise ValueError(f"pooled means {tuple(pq.shape)}, {tuple(pk.shape)} do not match q/k at "
                             f"blocks {BLKQ}, {BLKK}")
    else:
        pq = ops.block_pool(q, BLKQ)
        pk = ops.block_pool(k, BLKK)
    kc = keep_count(topk_ratio, pk.shape[2])
    return ops.block_select(pq, pk, kc, BLKQ, BLKK, force_diag=force_diag, want_map=want_map)


def sparse_attention(q, k, v, topk_ratio: float, blk: int = 64, force_diag: bool = False,
                     smooth_k: bool = True, pooled=None):
    """[1,H,S,D] -> [1,H,S,D] block-sparse attention (SLA sparse branch only; h3_sla:226-235).

    Native block sizes run on the block LUT; the others on the tile LUT
    built from the block map.  `pooled`: block means from the prologue (see
    get_block_map).
    """
    blk = check_block(blk)
    out_dtype = q.dtype
    q16, k16, v16 = (t.to(torch.bfloat16) for t in (q, k, v))
    native = blk in ops.NATIVE_BLOCKS
    bmap, lut, counts = get_block_map(q16, k16, topk_ratio, blk, blk, force_diag=force_diag,
                                      smooth_k=smooth_k, want_map=not native, pooled=pooled)
    if native:
        o = ops.attn_fwd_blocksparse(q16, k16, v16, lut, counts, blk, blk)
    else:
        tlut, tcnt = ops.block_map_to_tile_lut(bmap, blk, blk, q16.shape[2], k16.shape[2])
        o = ops.attn_fwd_blocksparse_tiles(q16, k16, v16, tlut, tcnt)
    return o.to(out_dtype)
