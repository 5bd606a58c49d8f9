"""numpy front end of the CPU oracle (oracle/h3_oracle.c -> oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product never imports it.

bf16 tensors are numpy uint16 arrays of bf16 bit patterns; helpers convert.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE, "-B"], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i, d = ctypes.c_int, ctypes.c_double
        i64 = ctypes.c_int64
        L.oracle_attn_fwd.restype = i
        L.oracle_attn_fwd.argtypes = [P, P, P, P, i, i, i, i, i, P, P, P, P, d, i, P, i, i]
        L.oracle_qk_rmsnorm_rope.restype = i
        L.oracle_qk_rmsnorm_rope.argtypes = [P, P, i, i, i, i, P, P, P, i64, i64, i, P, P, d]
        L.oracle_block_map.restype = i
        L.oracle_block_map.argtypes = [P, P, i, i, i, i, i, P, P, i, i, i, i, i, P, P]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        _lib = L
    return _lib


# ---------------------------------------------------------------------------
# bf16 helpers (numpy)
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bits (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _strides_elems(a: np.ndarray, dims):
    return np.array([a.strides[d] // a.itemsize for d in dims], dtype=np.int64)


# ---------------------------------------------------------------------------
def attn_fwd(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None,
             round_p: bool = True, block_map: np.ndarray | None = None, blk_q: int = 128,
             blk_k: int = 128) -> np.ndarray:
    """q [B,H,Sq,D], k/v [B,H,Skv,D] bf16 bits (uint16) -> O [B,H,Sq,D] float32."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    assert k.shape == (B, H, Skv, D) and v.shape == (B, H, Skv, D)
    o = np.zeros((B, H, Sq, D), dtype=np.float32)
    sc = 1.0 / np.sqrt(D) if scale is None else float(scale)
    bm = None
    if block_map is not None:
        bm = np.ascontiguousarray(block_map, dtype=np.uint8)
        assert bm.shape == (B, H, -(-Sq // blk_q), -(-Skv // blk_k)), bm.shape
    st = [_strides_elems(t, (0, 1, 2)) for t in (q, k, v, o)]
    rc = _load().oracle_attn_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(o), B, H, Sq, Skv, D,
                                 _ptr(st[0]), _ptr(st[1]), _ptr(st[2]), _ptr(st[3]), sc,
                                 1 if round_p else 0, None if bm is None else _ptr(bm),
                                 int(blk_q), int(blk_k))
    if rc != 0:
        raise RuntimeError(f"oracle_attn_fwd failed ({rc})")
    return o


def qk_rmsnorm_rope(q: np.ndarray, k: np.ndarray, rope: np.ndarray | None, qw: np.ndarray,
                    kw: np.ndarray, eps: float = 1e-6, rot_dim: int | None = None):
    """q, k [B,S,H,D] bf16 bits; rope fp32 [S, rot/2, 2, 2] or [B, S, rot/2, 2, 2].

    Returns new (q_out, k_out) bf16 bit arrays (inputs untouched).
    """
    q = np.array(q, dtype=np.uint16, copy=True, order="C")
    k = np.array(k, dtype=np.uint16, copy=True, order="C")
    B, S, H, D = q.shape
    if rot_dim is None:
        rot_dim = 0 if rope is None else rope.shape[-3] * 2
    if rot_dim > 0:
        r = np.ascontiguousarray(rope, dtype=np.float32)
        if r.ndim == 4:
            rsb, rss = 0, r.strides[0] // 4
        else:
            rsb = r.strides[0] // 4 if r.shape[0] > 1 else 0
            rss = r.strides[1] // 4
        rptr = _ptr(r)
    else:
        r, rptr, rsb, rss = None, None, 0, 0
    qw = np.ascontiguousarray(qw, dtype=np.uint16)
    kw = np.ascontiguousarray(kw, dtype=np.uint16)
    qs = _strides_elems(q, (0, 1, 2))
    ks = _strides_elems(k, (0, 1, 2))
    rc = _load().oracle_qk_rmsnorm_rope(_ptr(q), _ptr(k), B, S, H, D, _ptr(qs), _ptr(ks), rptr,
                                        int(rsb), int(rss), int(rot_dim), _ptr(qw), _ptr(kw), float(eps))
    if rc != 0:
        raise RuntimeError(f"oracle_qk_rmsnorm_rope failed ({rc})")
    return q, k


def block_map(q: np.ndarray, k: np.ndarray, blk_q: int, blk_k: int, keep: int,
              force_diag: bool = True, smooth_k: bool = False, return_scores: bool = False):
    """Mean-pooled top-`keep` block map [B,H,nq,nk] (uint8) from q [B,H,Sq,D], k [B,H,Skv,D] bf16 bits."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    nq, nk = -(-Sq // blk_q), -(-Skv // blk_k)
    m = np.zeros((B, H, nq, nk), dtype=np.uint8)
    sc = np.zeros((B, H, nq, nk), dtype=np.float64) if return_scores else None
    qs = _strides_elems(q, (0, 1, 2))
    ks = _strides_elems(k, (0, 1, 2))
    rc = _load().oracle_block_map(_ptr(q), _ptr(k), B, H, Sq, Skv, D, _ptr(qs), _ptr(ks),
                                  int(blk_q), int(blk_k), int(keep), 1 if force_diag else 0,
                                  1 if smooth_k else 0, _ptr(m), None if sc is None else _ptr(sc))
    if rc != 0:
        raise RuntimeError(f"oracle_block_map failed ({rc})")
    return (m, sc) if return_scores else m


def rope_table(S: int, rot_dim: int, theta: float = 10000.0, positions=None) -> np.ndarray:
    """fp32 [S, rot/2, 2, 2] rotation matrices [[cos,-sin],[sin,cos]], angle = pos * theta^(-2i/rot)."""
    pos = np.arange(S, dtype=np.float64) if positions is None else np.asarray(positions, np.float64)
    i = np.arange(rot_dim // 2, dtype=np.float64)
    omega = theta ** (-2.0 * i / rot_dim)
    ang = pos[:, None] * omega[None, :]
    c, s = np.cos(ang), np.sin(ang)
    return np.stack([c, -s, s, c], axis=-1).reshape(len(pos), rot_dim // 2, 2, 2).astype(np.float32)
