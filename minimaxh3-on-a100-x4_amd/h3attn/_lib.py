"""ctypes binding of libh3attn.so (the C ABI in include/h3attn.h).

The library is prebuilt in-tree (build_lib.py / __graft_entry__.build()).
There is no fallback: if the library is missing or cannot be loaded, every
entry point raises, so a HIP code path can never silently become something
else.  This module never initialises the GPU by itself; loading the library
only maps it.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("H3ATTN_LIB", os.path.join(_HERE, "libh3attn.so"))
# The phase-profile build of the same sources (H3A_PROFILE=1): its dense kernel
# stamps the shader clock at cluster boundaries (h3a_prof_read).
PROF_LIB_PATH = os.environ.get("H3ATTN_PROF_LIB", os.path.join(_HERE, "libh3attn_prof.so"))

H3A_OK = 0
H3A_ERR_INVALID_ARG = 1
H3A_ERR_UNSUPPORTED = 2
H3A_ERR_ALIGNMENT = 3
H3A_ERR_HIP = 4

KERNEL_ATTN_DENSE = 0
KERNEL_ATTN_SPARSE_128 = 1
KERNEL_ATTN_SPARSE_64 = 2
KERNEL_QK_ROPE = 3
KERNEL_ATTN_SPARSE_TILES = 4

_c_i64_3 = ctypes.c_int64 * 3
_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float

# Every symbol of include/h3attn.h with its (restype, argtypes).
SIGNATURES = {
    "h3a_version": (ctypes.c_char_p, []),
    "h3a_last_error": (ctypes.c_char_p, []),
    "h3a_attn_fwd": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                          _c_i64_3, _c_i64_3, _c_i64_3, _c_i64_3, _f, _vp]),
    "h3a_attn_fwd_workspace_size": (_i, [_i, _i, _i, _i, _i, ctypes.POINTER(ctypes.c_size_t)]),
    "h3a_attn_fwd_ws": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                             _c_i64_3, _c_i64_3, _c_i64_3, _c_i64_3, _f, _vp, ctypes.c_size_t, _vp]),
    "h3a_attn_fwd_noalloc": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                  _c_i64_3, _c_i64_3, _c_i64_3, _c_i64_3, _f, _vp]),
    "h3a_attn_fwd_blocksparse": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                      _c_i64_3, _c_i64_3, _c_i64_3, _c_i64_3,
                                      _vp, _vp, _i, _i, _i, _f, _vp]),
    "h3a_attn_fwd_blocksparse_workspace_size": (_i, [_i, _i, _i, _i, _i, _i, _i, _i,
                                                     ctypes.POINTER(ctypes.c_size_t)]),
    "h3a_attn_fwd_blocksparse_ws": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                         _c_i64_3, _c_i64_3, _c_i64_3, _c_i64_3,
                                         _vp, _vp, _i, _i, _i, _f, _vp, ctypes.c_size_t, _vp]),
    "h3a_attn_fwd_blocksparse_tiles": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                            _c_i64_3, _c_i64_3, _c_i64_3, _c_i64_3, _vp, _vp, _i, _f, _vp]),
    "h3a_attn_fwd_blocksparse_tiles_workspace_size": (_i, [_i, _i, _i, _i, _i, _i,
                                                           ctypes.POINTER(ctypes.c_size_t)]),
    "h3a_attn_fwd_blocksparse_tiles_ws": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                               _c_i64_3, _c_i64_3, _c_i64_3, _c_i64_3, _vp, _vp, _i, _f,
                                               _vp, ctypes.c_size_t, _vp]),
    "h3a_block_map_to_tile_lut": (_i, [_vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _i, _vp]),
    "h3a_lut_to_block_map": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _vp, _vp]),
    "h3a_block_map_to_lut": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _i, _vp]),
    "h3a_qk_rmsnorm_rope": (_i, [_vp, _vp, _i, _i, _i, _i, _c_i64_3, _c_i64_3,
                                 _vp, _i64, _i64, _i, _vp, _vp, _f, _vp]),
    "h3a_qk_rmsnorm_rope_pool": (_i, [_vp, _vp, _i, _i, _i, _i, _c_i64_3, _c_i64_3,
                                      _vp, _i64, _i64, _i, _vp, _vp, _f, _i, _vp, _vp, _vp]),
    "h3a_block_pool": (_i, [_vp, _i, _i, _i, _i, _c_i64_3, _i, _vp, _vp]),
    "h3a_block_select": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _i, _vp, _vp]),
    "h3a_kernel_attrs": (_i, [_i, ctypes.POINTER(ctypes.c_double)]),
    "h3a_prof_enabled": (_i, []),
    "h3a_prof_read": (_i, [ctypes.POINTER(ctypes.c_uint64)]),
    "h3a_prof_reset": (_i, []),
    "h3a_test_qk": (_i, [_vp, _vp, _vp, _vp]),
    "h3a_test_pv": (_i, [_vp, _vp, _vp, _vp]),
}

_lock = threading.Lock()
_handles: dict = {}


class H3AError(RuntimeError):
    """A libh3attn call returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with code {code}: {msg}")
        self.code = code


def lib(profile: bool = False) -> ctypes.CDLL:
    """Load (once) and return the library (profile=True: its phase-profile build); raise if not built."""
    path = PROF_LIB_PATH if profile else LIB_PATH
    handle = _handles.get(path)
    if handle is not None:
        return handle
    with _lock:
        if path not in _handles:
            if not os.path.exists(path):
                raise RuntimeError(
                    f"{os.path.basename(path)} not found at {path}; build it first "
                    "(python __graft_entry__.py build, or build_lib.py)")
            h = ctypes.CDLL(path)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(h, name)
                fn.restype = res
                fn.argtypes = args
            _handles[path] = h
    return _handles[path]


def check(fn: str, rc: int, handle: ctypes.CDLL | None = None) -> None:
    if rc != H3A_OK:
        msg = (handle or lib()).h3a_last_error().decode(errors="replace")
        if rc in (H3A_ERR_INVALID_ARG, H3A_ERR_UNSUPPORTED, H3A_ERR_ALIGNMENT):
            raise ValueError(f"{fn}: {msg} (code {rc})")
        raise H3AError(fn, rc, msg)


def strides3(a, b, c) -> ctypes.Array:
    return _c_i64_3(int(a), int(b), int(c))


def version() -> str:
    return lib().h3a_version().decode()
