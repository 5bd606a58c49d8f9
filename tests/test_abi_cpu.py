"""The C ABI on the CPU: the library loads, exports every symbol include/h3attn.h
declares, and rejects bad arguments with error codes before any HIP call (no
compute calls here: this container has no GPU)."""
from __future__ import annotations

import ctypes
import os
import re
import threading

import pytest

from conftest import ROOT
from h3attn import _lib

HEADER = os.path.join(ROOT, "include", "h3attn.h")
S3 = _lib.strides3
ROW = S3(0, 0, 128)  # output strides with one row per step (o rows must not overlap)


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(h3a_\w+)\s*\(", text, re.M)))


def test_header_symbols_exported_and_bound():
    L = _lib.lib()
    syms = header_symbols()
    assert len(syms) >= 9
    for s in syms:
        assert hasattr(L, s), f"{s} not exported by libh3attn.so"
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(syms)


def test_version():
    assert _lib.version().startswith("h3attn ")
    assert "gfx950" in _lib.version()


def _attn(L, q=16, k=16, v=16, o=16, B=1, H=1, Sq=4, Skv=4, D=128, qs=(0, 0, 0), scale=0.1):
    z = S3(0, 0, 0)
    return L.h3a_attn_fwd(q, k, v, o, B, H, Sq, Skv, D, S3(*qs), z, z, z, scale, None)


def test_attn_argument_errors():
    L = _lib.lib()
    assert _attn(L, q=None) == _lib.H3A_ERR_INVALID_ARG
    assert b"null" in L.h3a_last_error()
    assert _attn(L, Sq=0) == _lib.H3A_ERR_INVALID_ARG
    assert _attn(L, B=-1) == _lib.H3A_ERR_INVALID_ARG
    assert _attn(L, D=64) == _lib.H3A_ERR_UNSUPPORTED
    assert b"head_dim 64" in L.h3a_last_error()
    assert _attn(L, scale=0.0) == _lib.H3A_ERR_INVALID_ARG
    assert _attn(L, scale=float("nan")) == _lib.H3A_ERR_INVALID_ARG
    assert _attn(L, q=24) == _lib.H3A_ERR_ALIGNMENT        # 8-byte aligned only
    assert _attn(L, qs=(0, 0, 12)) == _lib.H3A_ERR_ALIGNMENT  # row stride not a multiple of 8
    assert _attn(L, qs=(0, -8, 8)) == _lib.H3A_ERR_ALIGNMENT
    z = S3(0, 0, 0)
    big = S3(0, 0, 1 << 24)  # a 64-row K/V stage would not fit 32-bit byte offsets
    assert L.h3a_attn_fwd(16, 16, 16, 16, 1, 1, 4, 4, 128, z, big, z, z, 0.1, None) == _lib.H3A_ERR_UNSUPPORTED
    assert b"sequence stride" in L.h3a_last_error()
    assert L.h3a_attn_fwd(16, 16, 16, 16, 1, 1, 4, 4, 128, z, z, big, z, 0.1, None) == _lib.H3A_ERR_UNSUPPORTED
    # Output rows less than one row apart overlap (a length-1 sequence's stride is free).
    for oss in (0, 64, 120):
        assert L.h3a_attn_fwd(16, 16, 16, 16, 1, 1, 4, 4, 128, z, z, z, S3(0, 0, oss), 0.1, None) == \
            _lib.H3A_ERR_INVALID_ARG
        assert b"rows overlap" in L.h3a_last_error()


def test_blocksparse_argument_errors():
    L = _lib.lib()
    z = S3(0, 0, 0)

    def call(lut=16, counts=16, bq=128, bk=128, maxk=1, Skv=300):
        return L.h3a_attn_fwd_blocksparse(16, 16, 16, 16, 1, 1, 300, Skv, 128, z, z, z, ROW, lut, counts,
                                          bq, bk, maxk, 0.1, None)

    assert call(lut=None) == _lib.H3A_ERR_INVALID_ARG
    for bq, bk in ((32, 128), (48, 128), (320, 128), (128, 96), (128, 16), (128, 512)):
        assert call(bq=bq, bk=bk) == _lib.H3A_ERR_UNSUPPORTED
        assert b"unsupported" in L.h3a_last_error()
    assert call(maxk=0) == _lib.H3A_ERR_INVALID_ARG
    assert call(maxk=4) == _lib.H3A_ERR_INVALID_ARG  # 300 keys = 3 blocks of 128
    assert b"max_k_blocks" in L.h3a_last_error()
    assert call(bk=256, maxk=3) == _lib.H3A_ERR_INVALID_ARG  # 2 blocks of 256
    assert call(bk=192, maxk=3) == _lib.H3A_ERR_INVALID_ARG  # 2 blocks of 192


def test_tile_entry_argument_errors():
    """The tile-LUT path (block sizes outside the native kernels'): argument errors before any HIP call."""
    L = _lib.lib()
    z = S3(0, 0, 0)

    def tiles(lut=16, counts=16, maxt=1, Skv=300, D=128):
        return L.h3a_attn_fwd_blocksparse_tiles(16, 16, 16, 16, 1, 1, 300, Skv, D, z, z, z, ROW, lut, counts,
                                                maxt, 0.1, None)

    assert tiles(lut=None) == _lib.H3A_ERR_INVALID_ARG
    assert tiles(D=64) == _lib.H3A_ERR_UNSUPPORTED
    assert tiles(maxt=0) == _lib.H3A_ERR_INVALID_ARG
    assert tiles(maxt=11) == _lib.H3A_ERR_INVALID_ARG  # 300 keys = 10 columns of 32
    assert b"max_tiles" in L.h3a_last_error()
    assert tiles(Skv=65535 * 32, maxt=1) == _lib.H3A_ERR_UNSUPPORTED  # past the columns an entry names
    ws = L.h3a_attn_fwd_blocksparse_tiles_ws
    assert ws(16, 16, 16, 16, 1, 1, 300, 300, 128, z, z, z, ROW, None, 16, 1, 0.1, None, 0, None) == \
        _lib.H3A_ERR_INVALID_ARG
    n = ctypes.c_size_t(7)
    assert L.h3a_attn_fwd_blocksparse_tiles_workspace_size(1, 1, 300, 300, 64, 1, ctypes.byref(n)) == \
        _lib.H3A_ERR_UNSUPPORTED
    assert L.h3a_attn_fwd_blocksparse_tiles_workspace_size(1, 1, 300, 300, 128, 11, ctypes.byref(n)) == \
        _lib.H3A_ERR_INVALID_ARG

    def conv(m=16, bq=32, bk=48, maxt=5, Sq=300, Skv=300):
        return L.h3a_block_map_to_tile_lut(m, 1, 1, Sq, Skv, bq, bk, 16, 16, maxt, None)

    assert conv(m=None) == _lib.H3A_ERR_INVALID_ARG
    for bq, bk in ((40, 48), (32, 8), (0, 64), (-16, 64)):
        assert conv(bq=bq, bk=bk) == _lib.H3A_ERR_UNSUPPORTED
    assert conv(maxt=11) == _lib.H3A_ERR_INVALID_ARG
    assert conv(Skv=65535 * 32, maxt=1) == _lib.H3A_ERR_UNSUPPORTED
    assert conv(Sq=0) == _lib.H3A_ERR_INVALID_ARG
    assert L.h3a_lut_to_block_map(None, 16, 1, 1, 2, 2, 1, 16, None) == _lib.H3A_ERR_INVALID_ARG
    assert L.h3a_lut_to_block_map(16, 16, 1, 1, 2, 0, 1, 16, None) == _lib.H3A_ERR_INVALID_ARG


def test_lut_and_prologue_argument_errors():
    L = _lib.lib()
    assert L.h3a_block_map_to_lut(None, 1, 1, 2, 2, 16, 16, 1, None) == _lib.H3A_ERR_INVALID_ARG
    assert L.h3a_block_map_to_lut(16, 1, 1, 2, 2, 16, 16, 3, None) == _lib.H3A_ERR_INVALID_ARG
    z = S3(0, 0, 0)

    def rope(rot=128, ropep=16, D=128, eps=1e-6, qs=(0, 0, 0), rss=64):
        return L.h3a_qk_rmsnorm_rope(16, 16, 1, 4, 2, D, S3(*qs), z, ropep, 0, rss, rot, 16, 16, eps, None)

    assert rope(D=64) == _lib.H3A_ERR_UNSUPPORTED
    assert rope(rot=24) == _lib.H3A_ERR_UNSUPPORTED
    assert rope(rot=144) == _lib.H3A_ERR_UNSUPPORTED
    assert rope(ropep=None) == _lib.H3A_ERR_INVALID_ARG
    assert rope(eps=-1.0) == _lib.H3A_ERR_INVALID_ARG
    assert rope(qs=(0, 3, 0)) == _lib.H3A_ERR_ALIGNMENT
    assert rope(rss=6) == _lib.H3A_ERR_ALIGNMENT
    pool = L.h3a_qk_rmsnorm_rope_pool
    assert pool(16, 16, 1, 4, 2, 128, z, z, 16, 0, 64, 128, 16, 16, 1e-6, 64, None, 16, None) == \
        _lib.H3A_ERR_INVALID_ARG
    assert pool(16, 16, 1, 4, 2, 128, z, z, 16, 0, 64, 128, 16, 16, 1e-6, 0, 16, 16, None) == \
        _lib.H3A_ERR_INVALID_ARG
    assert pool(16, 16, 1, 4, 2, 128, z, z, 16, 0, 64, 128, 16, 16, 1e-6, 64, 16, 20, None) == \
        _lib.H3A_ERR_ALIGNMENT
    assert pool(16, 16, 1, 4, 2, 64, z, z, 16, 0, 64, 128, 16, 16, 1e-6, 64, 16, 16, None) == \
        _lib.H3A_ERR_UNSUPPORTED
    assert L.h3a_block_pool(None, 1, 1, 10, 128, z, 64, 16, None) == _lib.H3A_ERR_INVALID_ARG
    assert L.h3a_block_pool(16, 1, 1, 10, 64, z, 64, 16, None) == _lib.H3A_ERR_UNSUPPORTED
    assert L.h3a_block_pool(16, 1, 1, 10, 128, z, 0, 16, None) == _lib.H3A_ERR_INVALID_ARG
    assert L.h3a_block_pool(24, 1, 1, 10, 128, z, 64, 16, None) == _lib.H3A_ERR_ALIGNMENT
    sel = L.h3a_block_select
    assert sel(None, 16, 1, 1, 4, 4, 2, 1, 64, 64, 16, 16, 3, None, None) == _lib.H3A_ERR_INVALID_ARG
    assert sel(16, 16, 1, 1, 4, 4, 5, 1, 64, 64, 16, 16, 3, None, None) == _lib.H3A_ERR_INVALID_ARG  # keep > nk
    assert sel(16, 16, 1, 1, 4, 4, 2, 1, 64, 64, 16, 16, 5, None, None) == _lib.H3A_ERR_INVALID_ARG  # max_k > nk
    assert sel(16, 16, 1, 1, 4, 9000, 2, 1, 64, 64, 16, 16, 3, None, None) == _lib.H3A_ERR_UNSUPPORTED
    assert L.h3a_kernel_attrs(0, None) == _lib.H3A_ERR_INVALID_ARG
    out = (ctypes.c_double * 6)()
    assert L.h3a_kernel_attrs(99, out) == _lib.H3A_ERR_INVALID_ARG
    assert L.h3a_test_qk(None, 16, 16, None) == _lib.H3A_ERR_INVALID_ARG
    assert L.h3a_test_pv(16, 24, 16, None) == _lib.H3A_ERR_ALIGNMENT


def test_last_error_is_thread_local_and_cleared():
    L = _lib.lib()
    assert _attn(L, D=64) == _lib.H3A_ERR_UNSUPPORTED
    seen = {}

    def other():
        seen["before"] = L.h3a_last_error()
        _attn(L, q=None)
        seen["after"] = L.h3a_last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["before"] == b""
    assert b"null" in seen["after"]
    assert b"head_dim" in L.h3a_last_error()  # this thread's message is untouched
    L.h3a_block_map_to_lut(None, 1, 1, 1, 1, 16, 16, 1, None)
    assert b"null" in L.h3a_last_error()


def test_python_check_raises_typed_errors():
    L = _lib.lib()
    rc = _attn(L, D=64)
    with pytest.raises(ValueError):
        _lib.check("h3a_attn_fwd", rc)
    with pytest.raises(_lib.H3AError):
        _lib.check("h3a_attn_fwd", _lib.H3A_ERR_HIP)


def test_workspace_entry_points_argument_errors():
    """h3a_attn_fwd_ws / h3a_attn_fwd_workspace_size reject bad arguments before any HIP call."""
    L = _lib.lib()
    n = ctypes.c_size_t(123)
    assert L.h3a_attn_fwd_workspace_size(1, 1, 4, 4, 128, None) == _lib.H3A_ERR_INVALID_ARG
    assert L.h3a_attn_fwd_workspace_size(1, 0, 4, 4, 128, ctypes.byref(n)) == _lib.H3A_ERR_INVALID_ARG
    assert L.h3a_attn_fwd_workspace_size(1, 1, 4, 4, 64, ctypes.byref(n)) == _lib.H3A_ERR_UNSUPPORTED
    assert n.value == 123  # untouched on error
    z = S3(0, 0, 0)
    ws = L.h3a_attn_fwd_ws
    assert ws(None, 16, 16, 16, 1, 1, 4, 4, 128, z, z, z, z, 0.1, None, 0, None) == _lib.H3A_ERR_INVALID_ARG
    assert ws(16, 16, 16, 16, 1, 1, 4, 4, 64, z, z, z, z, 0.1, None, 0, None) == _lib.H3A_ERR_UNSUPPORTED
    assert ws(16, 16, 16, 16, 1, 1, 4, 4, 128, S3(0, 0, 12), z, z, z, 0.1, None, 0, None) == _lib.H3A_ERR_ALIGNMENT
