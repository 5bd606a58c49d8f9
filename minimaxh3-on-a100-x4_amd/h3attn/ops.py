"""Tensor-level entry points over the libh3attn C ABI.

PyTorch supplies device memory and the current HIP stream; all arithmetic runs
in the gfx950 kernels of libh3attn.  Every function validates shapes/dtypes on
the host, passes raw pointers + element strides + torch's current stream, and
raises (ValueError for bad arguments, H3AError for HIP failures).  There is no
CPU fallback.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from ._lib import check, lib, strides3

HEAD_DIM = 128


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _norm_stride(t: torch.Tensor, dim: int) -> int:
    # A size-1 dimension is never stepped along; its stride is irrelevant.
    return 0 if t.shape[dim] == 1 else t.stride(dim)


def _kernel_ready(t: torch.Tensor, outer_dims) -> bool:
    """Last dim unit-stride, base 16-byte aligned, outer strides multiples of 8."""
    if t.stride(-1) != 1 or t.data_ptr() % 16 != 0:
        return False
    return all(_norm_stride(t, d) % 8 == 0 and _norm_stride(t, d) >= 0 for d in outer_dims)


def _as_kernel_input(name: str, t: torch.Tensor) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if t.dim() != 4:
        raise ValueError(f"{name} must be 4-D [B,H,S,D], got shape {tuple(t.shape)}")
    if t.shape[-1] != HEAD_DIM:
        raise ValueError(f"{name}: head_dim {t.shape[-1]} unsupported (only {HEAD_DIM})")
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (libh3attn has no CPU path)")
    # Layouts the kernel cannot stream directly are made contiguous (same HIP path).
    return t if _kernel_ready(t, (0, 1, 2)) else t.contiguous()


def _bhs(t: torch.Tensor):
    return strides3(_norm_stride(t, 0), _norm_stride(t, 1), _norm_stride(t, 2))


def _prepare_attn(q, k, v, out):
    q = _as_kernel_input("q", q)
    k = _as_kernel_input("k", k)
    v = _as_kernel_input("v", v)
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    if tuple(k.shape) != (B, H, Skv, D) or tuple(v.shape) != (B, H, Skv, D):
        raise ValueError(f"shape mismatch: q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    if Sq == 0 or Skv == 0 or B == 0 or H == 0:
        raise ValueError("empty attention input")
    if not (q.device == k.device == v.device):
        raise ValueError("q, k, v must be on the same device")
    if out is None:
        out = torch.empty((B, H, Sq, D), dtype=torch.bfloat16, device=q.device)
    else:
        if tuple(out.shape) != (B, H, Sq, D) or out.dtype != torch.bfloat16 or out.device != q.device:
            raise ValueError("out must be a bf16 [B,H,Sq,128] tensor on q's device")
        if not _kernel_ready(out, (0, 1, 2)):
            raise ValueError("out must have unit last stride, 16-byte alignment and strides multiple of 8")
    return q, k, v, out, (B, H, Sq, Skv, D)


def attn_workspace_bytes(B: int, H: int, Sq: int, Skv: int, D: int = HEAD_DIM) -> int:
    """Workspace bytes h3a_attn_fwd_ws needs on the current device (0: no split)."""
    n = ctypes.c_size_t(0)
    check("h3a_attn_fwd_workspace_size", lib().h3a_attn_fwd_workspace_size(B, H, Sq, Skv, D, ctypes.byref(n)))
    return int(n.value)


def attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float | None = None,
             out: torch.Tensor | None = None, split_tail: bool = True) -> torch.Tensor:
    """Dense non-causal attention, q [B,H,Sq,128], k/v [B,H,Skv,128] bf16 -> [B,H,Sq,128].

    Any strides with a unit last dimension are read in place (e.g. the
    [1,H,S,D] transposed views of a fused QKV projection); `out` may also be a
    strided view (e.g. [1,S,H,D] memory seen as [1,H,S,D]).

    split_tail: run through h3a_attn_fwd_ws with a workspace from torch's
    allocator on q's stream, so the last partly filled round of workgroups is
    split along the keys (equal results up to rounding); False runs
    h3a_attn_fwd, which never splits.
    """
    q, k, v, out, (B, H, Sq, Skv, D) = _prepare_attn(q, k, v, out)
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            B, H, Sq, Skv, D, _bhs(q), _bhs(k), _bhs(v), _bhs(out), sc)
    with torch.cuda.device(q.device):
        nbytes = attn_workspace_bytes(B, H, Sq, Skv, D) if split_tail else 0
        if nbytes:
            ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
            rc = lib().h3a_attn_fwd_ws(*args, ws.data_ptr(), nbytes, _stream(q))
            check("h3a_attn_fwd_ws", rc)
        else:
            rc = lib().h3a_attn_fwd(*args, _stream(q))
            check("h3a_attn_fwd", rc)
    return out


PROF_WAVES = 8
PROF_SLOTS = 12


def attn_fwd_profiled(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float | None = None,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """attn_fwd through the phase-profile build (libh3attn_prof.so), unsplit (h3a_attn_fwd).

    Workgroup 0 of the launch records its per-wave phase ticks; read them with
    prof_read().  The profile build stamps the shader clock inside the stage
    loop, so it runs a little slower than the product build.
    """
    q, k, v, out, (B, H, Sq, Skv, D) = _prepare_attn(q, k, v, out)
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    L = lib(profile=True)
    with torch.cuda.device(q.device):
        rc = L.h3a_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, H, Sq, Skv, D,
                            _bhs(q), _bhs(k), _bhs(v), _bhs(out), sc, _stream(q))
    check("h3a_attn_fwd (profile build)", rc, L)
    return out


def attn_fwd_blocksparse_profiled(q, k, v, lut, counts, blk_q: int, blk_k: int, scale: float | None = None,
                                  out: torch.Tensor | None = None) -> torch.Tensor:
    """attn_fwd_blocksparse through the phase-profile build, unsplit (h3a_attn_fwd_blocksparse).

    The ping-pong sparse kernels (pairs of query blocks) record workgroup 0's
    per-wave phases like the dense kernel; read them with prof_read().
    """
    q, k, v, out, (B, H, Sq, Skv, D) = _prepare_attn(q, k, v, out)
    lut, counts = lut.contiguous(), counts.contiguous()
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    L = lib(profile=True)
    with torch.cuda.device(q.device):
        rc = L.h3a_attn_fwd_blocksparse(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, H, Sq, Skv,
                                        D, _bhs(q), _bhs(k), _bhs(v), _bhs(out), lut.data_ptr(), counts.data_ptr(),
                                        int(blk_q), int(blk_k), int(lut.shape[3]), sc, _stream(q))
    check("h3a_attn_fwd_blocksparse (profile build)", rc, L)
    return out


def attn_fwd_blocksparse_tiles_profiled(q, k, v, tile_lut, tile_counts, scale: float | None = None,
                                        out: torch.Tensor | None = None) -> torch.Tensor:
    """attn_fwd_blocksparse_tiles through the phase-profile build (h3a_attn_fwd_blocksparse_tiles)."""
    q, k, v, out, (B, H, Sq, Skv, D) = _prepare_attn(q, k, v, out)
    tile_lut, tile_counts = tile_lut.contiguous(), tile_counts.contiguous()
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    L = lib(profile=True)
    with torch.cuda.device(q.device):
        rc = L.h3a_attn_fwd_blocksparse_tiles(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, H, Sq,
                                              Skv, D, _bhs(q), _bhs(k), _bhs(v), _bhs(out), tile_lut.data_ptr(),
                                              tile_counts.data_ptr(), int(tile_lut.shape[3]), sc, _stream(q))
    check("h3a_attn_fwd_blocksparse_tiles (profile build)", rc, L)
    return out


def prof_enabled(profile: bool = True) -> bool:
    """Whether the library (profile=True: the profile build) records phases."""
    return bool(lib(profile=profile).h3a_prof_enabled())


def prof_read(profile: bool = True) -> list[list[int]]:
    """[8 waves][12 slots] phase ticks of the last dense launch's workgroup 0 (h3a_prof_read)."""
    L = lib(profile=profile)
    buf = (ctypes.c_uint64 * (PROF_WAVES * PROF_SLOTS))()
    check("h3a_prof_read", L.h3a_prof_read(buf), L)
    return [[int(buf[w * PROF_SLOTS + i]) for i in range(PROF_SLOTS)] for w in range(PROF_WAVES)]


def prof_reset(profile: bool = True) -> None:
    L = lib(profile=profile)
    check("h3a_prof_reset", L.h3a_prof_reset(), L)


def sparse_workspace_bytes(B: int, H: int, Sq: int, Skv: int, blk_q: int, blk_k: int, max_k_blocks: int,
                           D: int = HEAD_DIM) -> int:
    """Workspace bytes h3a_attn_fwd_blocksparse_ws needs on the current device (0: no split)."""
    n = ctypes.c_size_t(0)
    check("h3a_attn_fwd_blocksparse_workspace_size",
          lib().h3a_attn_fwd_blocksparse_workspace_size(B, H, Sq, Skv, D, int(blk_q), int(blk_k),
                                                        int(max_k_blocks), ctypes.byref(n)))
    return int(n.value)


# Block sizes h3a_attn_fwd_blocksparse runs natively (multiples of its 64-key
# stage); every other multiple of 16 runs over tile LUTs with sub-block masks.
NATIVE_BLOCKS = (64, 128, 192, 256)


def _check_block_size(blk) -> int:
    b = int(blk)
    if b <= 0 or b % 16 != 0:
        raise ValueError(f"block size {blk} unsupported: a positive multiple of 16")
    return b


def attn_fwd_blocksparse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, lut: torch.Tensor,
                         counts: torch.Tensor, blk_q: int, blk_k: int, scale: float | None = None,
                         out: torch.Tensor | None = None, split_tail: bool = True) -> torch.Tensor:
    """Block-sparse attention over the kept key blocks listed in `lut`.

    lut: int32 [B,H,ceil(Sq/blk_q),max_k_blocks] ascending key-block indices;
    counts: int32 [B,H,ceil(Sq/blk_q)] number of valid entries per row.
    blk_q, blk_k: multiples of 16.  Sizes in NATIVE_BLOCKS run
    h3a_attn_fwd_blocksparse; with any other size the LUT becomes a block map
    (h3a_lut_to_block_map), then a tile LUT (h3a_block_map_to_tile_lut), run
    by h3a_attn_fwd_blocksparse_tiles.
    split_tail: as for attn_fwd (h3a_attn_fwd_blocksparse_ws with a workspace
    from torch's allocator); False runs h3a_attn_fwd_blocksparse, which never
    splits.
    """
    blk_q, blk_k = _check_block_size(blk_q), _check_block_size(blk_k)
    if blk_q not in NATIVE_BLOCKS or blk_k not in NATIVE_BLOCKS:
        Sq, Skv = q.shape[2], k.shape[2]
        bmap = lut_to_block_map(lut, counts, -(-Skv // blk_k))
        tlut, tcnt = block_map_to_tile_lut(bmap, blk_q, blk_k, Sq, Skv)
        return attn_fwd_blocksparse_tiles(q, k, v, tlut, tcnt, scale=scale, out=out, queues=split_tail)
    q, k, v, out, (B, H, Sq, Skv, D) = _prepare_attn(q, k, v, out)
    nqb = -(-Sq // blk_q)
    if lut.dtype != torch.int32 or counts.dtype != torch.int32:
        raise ValueError("lut and counts must be int32")
    if lut.dim() != 4 or tuple(lut.shape[:3]) != (B, H, nqb):
        raise ValueError(f"lut must be [B,H,{nqb},max_k], got {tuple(lut.shape)}")
    if tuple(counts.shape) != (B, H, nqb):
        raise ValueError(f"counts must be [B,H,{nqb}], got {tuple(counts.shape)}")
    if lut.device != q.device or counts.device != q.device:
        raise ValueError("lut/counts must be on q's device")
    lut = lut.contiguous()
    counts = counts.contiguous()
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, H, Sq, Skv, D,
            _bhs(q), _bhs(k), _bhs(v), _bhs(out), lut.data_ptr(), counts.data_ptr(),
            int(blk_q), int(blk_k), int(lut.shape[3]), sc)
    with torch.cuda.device(q.device):
        nbytes = (sparse_workspace_bytes(B, H, Sq, Skv, blk_q, blk_k, int(lut.shape[3]), D)
                  if split_tail else 0)
        if nbytes:
            ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
            rc = lib().h3a_attn_fwd_blocksparse_ws(*args, ws.data_ptr(), nbytes, _stream(q))
            check("h3a_attn_fwd_blocksparse_ws", rc)
        else:
            rc = lib().h3a_attn_fwd_blocksparse(*args, _stream(q))
            check("h3a_attn_fwd_blocksparse", rc)
    return out


def tiles_workspace_bytes(B: int, H: int, Sq: int, Skv: int, max_tiles: int, D: int = HEAD_DIM) -> int:
    """Workspace bytes h3a_attn_fwd_blocksparse_tiles_ws needs on the current device: the pair map
    (8 bytes per pair of 64-row sub-blocks, up to 16384 sub-blocks per (b,h)) and the work-queue
    counters of a persistent launch (0: neither)."""
    n = ctypes.c_size_t(0)
    check("h3a_attn_fwd_blocksparse_tiles_workspace_size",
          lib().h3a_attn_fwd_blocksparse_tiles_workspace_size(B, H, Sq, Skv, D, int(max_tiles), ctypes.byref(n)))
    return int(n.value)


def attn_fwd_blocksparse_tiles(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tile_lut: torch.Tensor,
                               tile_counts: torch.Tensor, scale: float | None = None,
                               out: torch.Tensor | None = None, queues: bool = True) -> torch.Tensor:
    """Block-sparse attention over 32-key columns with 16x16 sub-block masks (block_map_to_tile_lut).

    tile_lut: int32 [B,H,ceil(Sq/64),max_tiles], entries column << 8 | mask;
    tile_counts: int32 [B,H,ceil(Sq/64)].  queues: run through
    h3a_attn_fwd_blocksparse_tiles_ws (64-row sub-blocks paired by stage count,
    per-XCD work queues, workspace from torch's allocator); False runs
    h3a_attn_fwd_blocksparse_tiles (sub-blocks 2p and 2p+1 paired).  Both give
    the same output bit for bit.
    """
    q, k, v, out, (B, H, Sq, Skv, D) = _prepare_attn(q, k, v, out)
    nsub = -(-Sq // 64)
    if tile_lut.dtype != torch.int32 or tile_counts.dtype != torch.int32:
        raise ValueError("tile_lut and tile_counts must be int32")
    if tile_lut.dim() != 4 or tuple(tile_lut.shape[:3]) != (B, H, nsub):
        raise ValueError(f"tile_lut must be [B,H,{nsub},max_tiles], got {tuple(tile_lut.shape)}")
    if tuple(tile_counts.shape) != (B, H, nsub):
        raise ValueError(f"tile_counts must be [B,H,{nsub}], got {tuple(tile_counts.shape)}")
    if tile_lut.device != q.device or tile_counts.device != q.device:
        raise ValueError("tile_lut/tile_counts must be on q's device")
    tile_lut, tile_counts = tile_lut.contiguous(), tile_counts.contiguous()
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    max_tiles = int(tile_lut.shape[3])
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, H, Sq, Skv, D,
            _bhs(q), _bhs(k), _bhs(v), _bhs(out), tile_lut.data_ptr(), tile_counts.data_ptr(), max_tiles, sc)
    with torch.cuda.device(q.device):
        nbytes = tiles_workspace_bytes(B, H, Sq, Skv, max_tiles, D) if queues else 0
        if nbytes:
            ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
            rc = lib().h3a_attn_fwd_blocksparse_tiles_ws(*args, ws.data_ptr(), nbytes, _stream(q))
            check("h3a_attn_fwd_blocksparse_tiles_ws", rc)
        else:
            rc = lib().h3a_attn_fwd_blocksparse_tiles(*args, _stream(q))
            check("h3a_attn_fwd_blocksparse_tiles", rc)
    return out


def block_map_to_tile_lut(block_map: torch.Tensor, blk_q: int, blk_k: int, Sq: int, Skv: int,
                          max_tiles: int | None = None):
    """0/1 block map [B,H,ceil(Sq/blk_q),ceil(Skv/blk_k)] at block sizes that are multiples of 16
    -> (tile_lut int32 [B,H,ceil(Sq/64),max_tiles], tile_counts int32 [B,H,ceil(Sq/64)]) for
    attn_fwd_blocksparse_tiles.  max_tiles defaults to ceil(Skv/32), which always suffices."""
    blk_q, blk_k = _check_block_size(blk_q), _check_block_size(blk_k)
    if block_map.dim() != 4 or not block_map.is_cuda:
        raise ValueError("block_map must be a 4-D GPU tensor [B,H,nq,nk]")
    B, H, nq, nk = block_map.shape
    if (nq, nk) != (-(-Sq // blk_q), -(-Skv // blk_k)):
        raise ValueError(f"block_map [.., {nq}, {nk}] does not match Sq={Sq}/blk_q={blk_q}, Skv={Skv}/blk_k={blk_k}")
    m = block_map.to(torch.uint8).contiguous()
    ncols = -(-Skv // 32)
    max_tiles = ncols if max_tiles is None else int(max_tiles)
    nsub = -(-Sq // 64)
    lut = torch.empty((B, H, nsub, max_tiles), dtype=torch.int32, device=m.device)
    counts = torch.empty((B, H, nsub), dtype=torch.int32, device=m.device)
    rc = lib().h3a_block_map_to_tile_lut(m.data_ptr(), B, H, int(Sq), int(Skv), blk_q, blk_k, lut.data_ptr(),
                                         counts.data_ptr(), max_tiles, _stream(m))
    check("h3a_block_map_to_tile_lut", rc)
    return lut, counts


def lut_to_block_map(lut: torch.Tensor, counts: torch.Tensor, nk: int) -> torch.Tensor:
    """Block LUT [B,H,nq,max_k] + counts [B,H,nq] -> 0/1 uint8 block map [B,H,nq,nk]."""
    if lut.dtype != torch.int32 or counts.dtype != torch.int32 or not lut.is_cuda or lut.dim() != 4:
        raise ValueError("lut must be an int32 GPU tensor [B,H,nq,max_k] with int32 counts")
    B, H, nq, max_k = lut.shape
    if tuple(counts.shape) != (B, H, nq) or counts.device != lut.device:
        raise ValueError(f"counts must be [B,H,{nq}] on lut's device")
    lut, counts = lut.contiguous(), counts.contiguous()
    bmap = torch.empty((B, H, nq, int(nk)), dtype=torch.uint8, device=lut.device)
    rc = lib().h3a_lut_to_block_map(lut.data_ptr(), counts.data_ptr(), B, H, nq, int(nk), int(max_k),
                                    bmap.data_ptr(), _stream(lut))
    check("h3a_lut_to_block_map", rc)
    return bmap


def block_map_to_lut(block_map: torch.Tensor, max_k_blocks: int | None = None):
    """Boolean/uint8 block map [B,H,nq,nk] -> (lut int32 [B,H,nq,max_k], counts int32 [B,H,nq])."""
    if block_map.dim() != 4 or not block_map.is_cuda:
        raise ValueError("block_map must be a 4-D GPU tensor [B,H,nq,nk]")
    m = block_map.to(torch.uint8).contiguous()
    B, H, nq, nk = m.shape
    if max_k_blocks is None:
        max_k_blocks = max(1, int(m.sum(dim=-1, dtype=torch.int32).max().item()))
    lut = torch.empty((B, H, nq, max_k_blocks), dtype=torch.int32, device=m.device)
    counts = torch.empty((B, H, nq), dtype=torch.int32, device=m.device)
    rc = lib().h3a_block_map_to_lut(m.data_ptr(), B, H, nq, nk, lut.data_ptr(), counts.data_ptr(),
                                    int(max_k_blocks), _stream(m))
    check("h3a_block_map_to_lut", rc)
    return lut, counts


def block_pool(x: torch.Tensor, blk: int) -> torch.Tensor:
    """Block means over the valid rows of each block: bf16 [B,H,S,128] -> fp32 [B,H,ceil(S/blk),128]."""
    x = _as_kernel_input("x", x)
    B, H, S, D = x.shape
    out = torch.empty((B, H, -(-S // blk), D), dtype=torch.float32, device=x.device)
    rc = lib().h3a_block_pool(x.data_ptr(), B, H, S, D, _bhs(x), int(blk), out.data_ptr(), _stream(x))
    check("h3a_block_pool", rc)
    return out


def block_select(pq: torch.Tensor, pk: torch.Tensor, keep: int, blk_q: int, blk_k: int,
                 force_diag: bool = True, max_k_blocks: int | None = None, want_map: bool = True):
    """Top-`keep` key blocks per query block by pooled score (+ diagonal) -> (map|None, lut, counts)."""
    for name, t in (("pq", pq), ("pk", pk)):
        if t.dtype != torch.float32 or not t.is_cuda or t.dim() != 4 or t.shape[-1] != HEAD_DIM:
            raise ValueError(f"{name} must be an fp32 GPU tensor [B,H,n,128]")
    pq, pk = pq.contiguous(), pk.contiguous()
    B, H, nq, _ = pq.shape
    nk = pk.shape[2]
    if tuple(pk.shape[:2]) != (B, H):
        raise ValueError("pq and pk must share [B,H]")
    if max_k_blocks is None:
        max_k_blocks = min(nk, int(keep) + (1 if force_diag else 0))
    lut = torch.empty((B, H, nq, max_k_blocks), dtype=torch.int32, device=pq.device)
    counts = torch.empty((B, H, nq), dtype=torch.int32, device=pq.device)
    bmap = torch.empty((B, H, nq, nk), dtype=torch.uint8, device=pq.device) if want_map else None
    rc = lib().h3a_block_select(pq.data_ptr(), pk.data_ptr(), B, H, nq, nk, int(keep),
                                1 if force_diag else 0, int(blk_q), int(blk_k), lut.data_ptr(),
                                counts.data_ptr(), int(max_k_blocks),
                                None if bmap is None else bmap.data_ptr(), _stream(pq))
    check("h3a_block_select", rc)
    return bmap, lut, counts


def _rope_table(rope: torch.Tensor, B: int, S: int, rot_dim: int):
    """Validate a ComfyUI-style rope_freqs tensor; return (tensor, batch stride, seq stride)."""
    if rope.dtype != torch.float32:
        raise ValueError(f"rope table must be float32, got {rope.dtype}")
    if rope.dim() < 4 or tuple(rope.shape[-2:]) != (2, 2):
        raise ValueError(f"rope table must end in [rot/2, 2, 2], got {tuple(rope.shape)}")
    if rope.shape[-3] != rot_dim // 2:
        raise ValueError(f"rope table has {rope.shape[-3]} frequencies, rot_dim {rot_dim} needs {rot_dim // 2}")
    # Accepted leading layouts: [S,...], [Bt,S,...], [Bt,S,1,...] (head axis broadcast).
    lead = list(rope.shape[:-3])
    lead_strides = list(rope.stride()[:-3])
    if len(lead) == 3:
        if lead[2] != 1:
            raise ValueError("rope table head axis must have size 1")
        lead, lead_strides = lead[:2], lead_strides[:2]
    if len(lead) == 1:
        lead, lead_strides = [1] + lead, [0] + lead_strides
    if len(lead) != 2 or lead[1] != S or lead[0] not in (1, B):
        raise ValueError(f"rope table leading dims {tuple(rope.shape[:-3])} do not match B={B}, S={S}")
    inner = rope.stride()[-3:]
    if tuple(inner) != (4, 2, 1):
        rope = rope.contiguous()
        return _rope_table(rope, B, S, rot_dim)
    sb = 0 if lead[0] == 1 else lead_strides[0]
    ss = lead_strides[1]
    if rope.data_ptr() % 16 or sb % 4 or ss % 4:
        rope = rope.contiguous()
        return _rope_table(rope, B, S, rot_dim)
    return rope, sb, ss


def qk_rmsnorm_rope_(q: torch.Tensor, k: torch.Tensor, rope: torch.Tensor | None, qw: torch.Tensor,
                     kw: torch.Tensor, eps: float = 1e-6, rot_dim: int | None = None,
                     pool_blk: int | None = None):
    """In-place per-head RMSNorm (weights qw/kw over head_dim) + split-half RoPE on q, k [B,S,H,128].

    q and k are typically strided views of the fused QKV projection output.
    The rotation for frequency i < rot_dim/2 is rope[..., s, i, :, :] applied to
    the pair (x[i], x[i + rot_dim/2]).  Returns None; with pool_blk, also pools
    the result in the same pass (h3a_qk_rmsnorm_rope_pool) and returns the fp32
    block means (q_means, k_means) [B,H,ceil(S/pool_blk),128], equal to
    block_pool of the updated q and k (as [B,H,S,128]).
    """
    for name, t in (("q", q), ("k", k)):
        if t.dtype != torch.bfloat16 or not t.is_cuda or t.dim() != 4 or t.shape[-1] != HEAD_DIM:
            raise ValueError(f"{name} must be a bf16 GPU tensor [B,S,H,128], got {t.dtype} {tuple(t.shape)}")
        if not _kernel_ready(t, (0, 1, 2)):
            raise ValueError(f"{name}: in-place update needs unit last stride, 16-byte alignment and "
                             "outer strides that are multiples of 8 elements")
    if tuple(q.shape) != tuple(k.shape):
        raise ValueError("q and k must have the same shape")
    B, S, H, D = q.shape
    if rot_dim is None:
        rot_dim = 0 if rope is None else int(rope.shape[-3]) * 2
    rot_dim = int(rot_dim)
    ws = []
    for name, w in (("qw", qw), ("kw", kw)):
        if w.numel() != D:
            raise ValueError(f"{name} must have {D} elements")
        w = w.reshape(D).to(device=q.device, dtype=torch.bfloat16).contiguous()
        ws.append(w)
    if rot_dim > 0:
        if rope is None:
            raise ValueError("rope table required when rot_dim > 0")
        rope, rsb, rss = _rope_table(rope.to(q.device), B, S, rot_dim)
        rptr = rope.data_ptr()
    else:
        rptr, rsb, rss = None, 0, 0
    args = (q.data_ptr(), k.data_ptr(), B, S, H, D,
            strides3(_norm_stride(q, 0), _norm_stride(q, 1), _norm_stride(q, 2)),
            strides3(_norm_stride(k, 0), _norm_stride(k, 1), _norm_stride(k, 2)),
            rptr, int(rsb), int(rss), rot_dim, ws[0].data_ptr(), ws[1].data_ptr(), float(eps))
    if pool_blk is None:
        check("h3a_qk_rmsnorm_rope", lib().h3a_qk_rmsnorm_rope(*args, _stream(q)))
        return None
    blk = int(pool_blk)
    if blk <= 0:
        raise ValueError(f"pool_blk {pool_blk} must be positive")
    means = torch.empty((2, B, H, -(-S // blk), D), dtype=torch.float32, device=q.device)
    check("h3a_qk_rmsnorm_rope_pool",
          lib().h3a_qk_rmsnorm_rope_pool(*args, blk, means[0].data_ptr(), means[1].data_ptr(), _stream(q)))
    return means[0], means[1]


def rms_rope_split_half_(q, k, rope_freqs, qw, kw, epsilon: float = 1e-6, rot_dim: int | None = None):
    """Signature-compatible stand-in for comfy.quant_ops.ck.rms_rope_split_half_ (in place).

    Called at harness/sp_runtime.py:98 and custom_nodes/h3_profiler/__init__.py:104-105
    as rms_rope_split_half_(q, k, rope_freqs, qw, kw, epsilon=eps, rot_dim=rot).
    """
    qk_rmsnorm_rope_(q, k, rope_freqs, qw, kw, eps=epsilon, rot_dim=rot_dim)


def test_qk(Q: torch.Tensor, K: torch.Tensor) -> torch.Tensor:
    """S[32,64] fp32 = Q[32,128] @ K[64,128]^T on one wavefront through the attention fragment code."""
    if tuple(Q.shape) != (32, 128) or tuple(K.shape) != (64, 128):
        raise ValueError("test_qk expects Q[32,128], K[64,128]")
    Q = Q.to(torch.bfloat16).contiguous()
    K = K.to(torch.bfloat16).contiguous()
    S = torch.empty((32, 64), dtype=torch.float32, device=Q.device)
    check("h3a_test_qk", lib().h3a_test_qk(Q.data_ptr(), K.data_ptr(), S.data_ptr(), _stream(Q)))
    return S


def test_pv(P: torch.Tensor, V: torch.Tensor) -> torch.Tensor:
    """O[32,128] fp32 = P[32,64] @ V[64,128] on one wavefront through the attention fragment code."""
    if tuple(P.shape) != (32, 64) or tuple(V.shape) != (64, 128):
        raise ValueError("test_pv expects P[32,64], V[64,128]")
    P = P.to(torch.bfloat16).contiguous()
    V = V.to(torch.bfloat16).contiguous()
    O = torch.empty((32, 128), dtype=torch.float32, device=P.device)
    check("h3a_test_pv", lib().h3a_test_pv(P.data_ptr(), V.data_ptr(), O.data_ptr(), _stream(P)))
    return O


def kernel_attrs(which: int = _lib.KERNEL_ATTN_DENSE):
    """[VGPRs, LDS bytes, max WGs/CU, clock kHz, occupancy, threads] for a kernel (current device)."""
    out = (ctypes.c_double * 6)()
    check("h3a_kernel_attrs", lib().h3a_kernel_attrs(int(which), out))
    return [float(x) for x in out]
