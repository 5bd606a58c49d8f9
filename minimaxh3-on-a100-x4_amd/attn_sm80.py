"""Drop-in replacement for the reference's attn_sm80/attn_sm80.py on MI355X.

Same surface as attn_sm80/attn_sm80.py:10-42:
    _build()            -> extension object (fa3, fa3_pp, kernel_attrs, pp_attrs,
                           get_prof, reset_prof, test_qk, test_pv), cached
    _build(profile=True)-> the same over the phase-profile build (the reference
                           built a second extension with -DPROFILE for this,
                           attn_sm80/report_metrics.py:77-80)
    fa3_sm80_h3(q,k,v)  -> O via the hand-written kernel
    sdpa_flash(q,k,v)   -> O via torch SDPA forced to the FLASH backend
    attn(q,k,v,backend) -> dispatch; unknown backend raises ValueError(backend)

Differences (all in the caller's favour): the kernel is the gfx950 HIP kernel
of libh3attn (prebuilt, no JIT); B > 1 is honoured (the reference ignored B,
fa3_sm80_h3.cu:461); strided inputs are read in place instead of being copied
with .contiguous() (attn_sm80.py:28); launches go on torch's current stream.
The default backend name is "hip"; the reference's "fa3_sm80_h3" is accepted
as an alias, so existing callers keep working.
"""
from __future__ import annotations

import threading

import torch
from torch.nn.attention import SDPBackend, sdpa_kernel

import h3attn
from h3attn import ops as _ops
from h3attn import _lib

BACKENDS = ("hip", "fa3_sm80_h3", "fa3_pp", "sdpa_flash", "sdpa")
_ext = None
_ext_lock = threading.Lock()


class _Ext:
    """Object with the reference extension's method names (fa3_sm80_h3.cu:584-593)."""

    profile = False

    def fa3(self, Q, K, V, O):
        _ops.attn_fwd(Q, K, V, out=O)

    def fa3_pp(self, Q, K, V, O):  # the reference's pipelined variant; pipelining is internal here
        self.fa3(Q, K, V, O)

    @staticmethod
    def kernel_attrs():
        return torch.tensor(_ops.kernel_attrs(_lib.KERNEL_ATTN_DENSE), dtype=torch.float64)

    pp_attrs = kernel_attrs

    def get_prof(self):
        """float64[5]: wait, qk, softmax, pv, epilogue (fa3_sm80_h3.cu:96, 572-577).

        The phase ticks of wave 0 (group A) of workgroup 0 in the last dense
        launch, in shader-clock ticks summed over its stages: wait = DMA issue,
        DMA wait and both barriers; qk = the matrix cluster, where the QK^T
        and PV MFMAs are interleaved (so pv is 0: it is inside qk); softmax =
        the softmax cluster; epilogue = normalise and store.  Only the profile
        build records them; the product build returns zeros, as the
        reference's non-PROFILE build does.
        """
        if not self.profile:
            return torch.zeros(5, dtype=torch.float64)
        w0 = _ops.prof_read(profile=True)[0]
        return torch.tensor([w0[0] + w0[2] + w0[4] + w0[5], w0[1], w0[3], 0, w0[9]], dtype=torch.float64)

    def reset_prof(self):
        if self.profile:
            _ops.prof_reset(profile=True)

    @staticmethod
    def test_qk(Q, K, S):
        """S[r,64] = Q[r,128] @ K[64,128]^T, r <= 32 (reference: r = 16)."""
        r = Q.shape[0]
        Qp = torch.zeros((32, 128), dtype=torch.bfloat16, device=Q.device)
        Qp[:r] = Q
        S.copy_(_ops.test_qk(Qp, K)[:r])

    @staticmethod
    def test_pv(P, V, O):
        """O[r,128] = P[r,64] @ V[64,128], r <= 32 (reference: r = 16)."""
        r = P.shape[0]
        Pp = torch.zeros((32, 64), dtype=torch.bfloat16, device=P.device)
        Pp[:r] = P
        O.copy_(_ops.test_pv(Pp, V)[:r])


class _ProfExt(_Ext):
    """The extension over libh3attn_prof.so: fa3 runs the unsplit dense kernel of the
    profile build, and get_prof / reset_prof read and clear its phase ticks."""

    profile = True

    def fa3(self, Q, K, V, O):
        _ops.attn_fwd_profiled(Q, K, V, out=O)


_prof_ext = None


def _build(profile: bool = False):
    """Return the (prebuilt) kernel extension; raises if its library is missing.

    profile=True returns the phase-profile build's extension instead.
    """
    global _ext, _prof_ext
    with _ext_lock:
        if profile:
            if _prof_ext is None:
                _lib.lib(profile=True)  # loads or raises: no silent fallback
                _prof_ext = _ProfExt()
            return _prof_ext
        if _ext is None:
            _lib.lib()
            _ext = _Ext()
        return _ext


def fa3_sm80_h3(q, k, v):
    _build()
    return h3attn.attn_fwd(q, k, v)


def sdpa_flash(q, k, v):
    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            return torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=False)
    except RuntimeError as e:
        raise RuntimeError(f"sdpa_flash: torch's FLASH_ATTENTION SDPA backend cannot run these inputs "
                           f"on this build/device ({e})") from e


def sdpa(q, k, v):
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=False)


def attn(q, k, v, backend="hip"):
    if backend in ("hip", "fa3_sm80_h3", "fa3_pp"):
        return fa3_sm80_h3(q, k, v)
    if backend == "sdpa_flash":
        return sdpa_flash(q, k, v)
    if backend == "sdpa":
        return sdpa(q, k, v)
    raise ValueError(backend)
