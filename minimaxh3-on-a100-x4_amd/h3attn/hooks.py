"""Drop-in hooks that route the MiniMax-H3 DiT attention through libh3attn.

Surfaces mirrored (paths relative to the reference checkout):

* Attention.forward(self, x, rope_freqs=None, transformer_options={}) as a
  class-attribute monkeypatch that keeps the original for chaining
  (harness/sp_runtime.py:85-126, 257-267; the stock math is restated at
  custom_nodes/h3_profiler/__init__.py:92-111):
      qkv_proj -> split -> rms_rope_split_half_ (rope path) -> [1,H,S,D] views
      -> optimized_attention(q,k,v,heads,mask=None,skip_reshape=True,...)
      -> [1,S,H*D] -> out_proj
  Calls with rope_freqs=None (the TokenRefiner, harness/sp_runtime.py:20-26)
  fall through to the original forward.
* ComfyUI's optimized_attention signature, and the
  transformer_options["optimized_attention_override"] callable contract
  override(func, q, k, v, heads, mask=None, skip_reshape=True, ...) -> [1,S,H*D]
  with fall-back to `func` on any exception (custom_nodes/h3_sla/__init__.py:265-284).
* The h3_sla scope patch (thread-local "inside a DiT block" flag + layer index,
  custom_nodes/h3_sla/__init__.py:244-262) and its per-layer sparse override.

In the patched forward, q/k are normalised in place inside the fused QKV
output, q/k/v are read by the kernel through strided views (no copies), and O
is written directly in the [S, H*D] layout out_proj consumes.
"""
from __future__ import annotations

import os
import threading
from typing import Callable

import torch

from . import ops, profiling, sla

_state = threading.local()


# ---------------------------------------------------------------------------
# attention callables with ComfyUI's optimized_attention signature
def hip_optimized_attention(q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                            skip_output_reshape=False, transformer_options=None, **_):
    """ComfyUI optimized_attention on libh3attn (dense, non-causal, no mask).

    skip_reshape: q/k/v are [B,H,S,D]; otherwise [B,S,H*D].  Returns [B,S,H*D]
    (or [B,H,S,D] with skip_output_reshape).  A mask raises ValueError: the
    kernel is mask-free, as is every DiT call site (mask=None).
    """
    if mask is not None:
        raise ValueError("libh3attn attention takes no mask")
    if not skip_reshape:
        B, S, HD = q.shape
        D = HD // heads
        q, k, v = (t.view(t.shape[0], t.shape[1], heads, D).transpose(1, 2) for t in (q, k, v))
    B, H, S, D = q.shape
    if skip_output_reshape:
        return ops.attn_fwd(q, k, v)
    out = torch.empty((B, S, H, D), dtype=torch.bfloat16, device=q.device)
    ops.attn_fwd(q, k, v, out=out.transpose(1, 2))
    return out.view(B, S, H * D)


def _gate(args, kwargs) -> bool:
    """The h3_sla gate: no mask, 4-D q with head_dim 128 (custom_nodes/h3_sla/__init__.py:271-273)."""
    if kwargs.get("mask") is not None or len(args) < 3:
        return False
    q = args[0]
    return hasattr(q, "shape") and q.dim() == 4 and q.shape[-1] == 128


def make_override(attention: Callable = hip_optimized_attention, log=print):
    """transformer_options['optimized_attention_override'] running the HIP dense kernel.

    Expects skip_reshape=True calls ([1,H,S,D] inputs) as the DiT makes; any
    other call, or any exception, goes to the wrapped `func`.
    """
    def override(func, *args, **kwargs):
        try:
            if _gate(args, kwargs) and kwargs.get("skip_reshape", False):
                q, k, v, heads = args[0], args[1], args[2], args[3] if len(args) > 3 else kwargs.get("heads")
                return attention(q, k, v, heads, mask=None, skip_reshape=True)
        except Exception as e:  # never break a render on the fast path
            log(f"[h3attn] override fell back to the original attention: {e}")
        return func(*args, **kwargs)

    override.h3sla = None
    return override


# ---------------------------------------------------------------------------
# h3_sla-compatible scope flag, schedule and sparse override
def install_scope_patch(attention_cls) -> None:
    """Mark DiT-block attention calls (rope_freqs is not None) in a thread-local flag (idempotent)."""
    fwd = attention_cls.forward
    if getattr(fwd, "_h3attn_scope", False):
        return

    def scoped(self, x, rope_freqs=None, transformer_options={}):
        prev = getattr(_state, "on", False), getattr(_state, "layer", None)
        _state.on = rope_freqs is not None
        _state.layer = getattr(self, "_h3sla_layer", None)
        try:
            return fwd(self, x, rope_freqs=rope_freqs, transformer_options=transformer_options)
        finally:
            _state.on, _state.layer = prev

    scoped._h3attn_scope = True
    scoped._h3attn_orig = fwd
    attention_cls.forward = scoped


def in_dit_scope() -> bool:
    return bool(getattr(_state, "on", False))


class Schedule:
    """Per-layer keep ratios (custom_nodes/h3_sla/__init__.py:139-212, without the status file).

    blk is checked here, when the schedule is built, as the node checks its
    kernel when it patches the model (h3_sla:331): an unsupported size raises
    ValueError instead of turning every sparse layer into a dense one later.
    timing (default: env H3_SLA_TIMING == "1", as at h3_sla:147) records HIP
    events around each sparse layer; they are resolved at the last layer of a
    step (h3_sla:199-212) into attn_ms / attn_n per layer.
    """

    def __init__(self, name: str, keeps, blk: int = 64, force_diag: bool = False, smooth_k: bool = True,
                 timing: bool | None = None):
        self.name, self.keeps, self.blk = name, [float(x) for x in keeps], sla.check_block(blk)
        self.force_diag, self.smooth_k = force_diag, smooth_k
        self.default_keep = max(set(self.keeps), key=self.keeps.count) if self.keeps else 1.0
        self.summary = sla.schedule_summary(name, self.keeps, self.blk) if self.keeps else None
        self.timing = (os.environ.get("H3_SLA_TIMING") == "1") if timing is None else bool(timing)
        self._ev = []
        self.attn_ms = [0.0] * len(self.keeps)
        self.attn_n = [0] * len(self.keeps)

    def keep_for(self, layer):
        if layer is None or not (0 <= layer < len(self.keeps)):
            return self.default_keep
        return self.keeps[layer]

    def flush_timing(self) -> None:
        """Resolve the recorded events into attn_ms / attn_n (synchronises on the last one)."""
        if not self._ev:
            return
        self._ev[-1][2].synchronize()
        for layer, a, b in self._ev:
            self.attn_ms[layer] += a.elapsed_time(b)
            self.attn_n[layer] += 1
        self._ev = []

    def attn_ms_per_layer_call(self):
        """Mean sparse-attention ms per call for each layer (None where it never ran)."""
        return [round(m / n, 3) if n else None for m, n in zip(self.attn_ms, self.attn_n)]

    def _sparse(self, q, k, v, keep):
        return sla.sparse_attention(q, k, v, keep, self.blk, force_diag=self.force_diag, smooth_k=self.smooth_k)

    def run(self, layer, q, k, v, transformer_options=None):
        """[1,H,S,D] sparse output, or None (keep >= 1: caller runs dense)."""
        keep = self.keep_for(layer)
        if keep >= 1.0:
            return None
        if self.timing and layer is not None and 0 <= layer < len(self.keeps):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            o = self._sparse(q, k, v, keep)
            b.record()
            self._ev.append((layer, a, b))
            if layer == len(self.keeps) - 1:  # end of a denoise step
                self.flush_timing()
            return o
        return self._sparse(q, k, v, keep)


def make_sla_override(topk: float = 0.35, blk: int = 64, schedule: Schedule | None = None,
                      log=print):
    """HIP counterpart of h3_sla's _make_override (custom_nodes/h3_sla/__init__.py:265-284).

    Active only inside DiT-block attention (install_scope_patch) with mask=None
    and head_dim 128; returns [1,S,H*D]; any exception falls back to `func`.
    The block size is checked here (ValueError), not at the first call.
    """
    blk = sla.check_block(blk)

    def override(func, *args, **kwargs):
        try:
            if in_dit_scope() and _gate(args, kwargs):
                q, k, v = args[0], args[1], args[2]
                _, H, S, D = q.shape
                if schedule is None:
                    o = sla.sparse_attention(q, k, v, topk, blk)
                else:
                    o = schedule.run(getattr(_state, "layer", None), q, k, v, kwargs.get("transformer_options"))
                if o is not None:
                    return o.transpose(1, 2).reshape(1, S, H * D)
        except Exception as e:  # never break a render on a sparse path
            log(f"[h3attn] sparse override fell back to dense: {e}")
        return func(*args, **kwargs)

    override.h3sla = schedule
    return override


def get_schedule(transformer_options):
    """The active Schedule carried by the override, or None (custom_nodes/h3_sla/__init__.py:287-293)."""
    try:
        return getattr((transformer_options or {}).get("optimized_attention_override"), "h3sla", None)
    except Exception:
        return None


# ---------------------------------------------------------------------------
# Attention.forward patch
def _weight(p, device):
    return p.detach().to(device=device)


def make_attention_forward(orig_forward, prologue: Callable = ops.rms_rope_split_half_,
                           attention: Callable = hip_optimized_attention, timer=None):
    """Build a replacement Attention.forward; `orig_forward` handles rope_freqs=None.

    With a `timer` (h3attn.profiling.OpTimer) the four sub-operations are
    timed under the reference profiler's component names
    (custom_nodes/h3_profiler/__init__.py:98-115) whenever the timer is armed.
    """
    mark = timer.mark if timer is not None else profiling.passthrough

    def forward(self, x, rope_freqs=None, transformer_options={}):
        if rope_freqs is None:
            return orig_forward(self, x, rope_freqs=rope_freqs, transformer_options=transformer_options)
        s = x.shape[0]
        H, D = self.heads, self.head_dim
        qkv = mark("attn.qkv", self.qkv_proj, x)
        q, k, v = qkv.split(H * D, dim=-1)
        q = q.view(1, s, H, D)
        k = k.view(1, s, H, D)
        rot = rope_freqs.shape[-3] * 2
        mark("attn.qknorm_rope", prologue, q, k, rope_freqs, _weight(self.q_norm.weight, x.device),
             _weight(self.k_norm.weight, x.device), epsilon=self.q_norm.eps, rot_dim=rot)
        qh = q.transpose(1, 2)
        kh = k.transpose(1, 2)
        vh = v.view(1, s, H, D).transpose(1, 2)
        override = (transformer_options or {}).get("optimized_attention_override")
        if override is not None:
            out = mark("attn.softmax", override, attention, qh, kh, vh, H, mask=None, skip_reshape=True,
                       transformer_options=transformer_options)
        else:
            out = mark("attn.softmax", attention, qh, kh, vh, H, mask=None, skip_reshape=True,
                       transformer_options=transformer_options)
        return mark("attn.out", self.out_proj, out.reshape(s, H * D))

    forward._h3attn_patched = True
    forward._h3attn_orig = orig_forward
    forward._h3attn_timer = timer
    return forward


def install(attention_cls=None, prologue: Callable = ops.rms_rope_split_half_,
            attention: Callable = hip_optimized_attention, timer=None) -> bool:
    """Patch Attention.forward (comfy.ldm.minimax.model.Attention by default); idempotent.

    `timer`: optional h3attn.profiling.OpTimer that times the sub-operations
    while armed.  Returns True when a patch was installed, False when it
    already was.
    """
    if attention_cls is None:
        import comfy.ldm.minimax.model as mm  # ComfyUI is optional: imported only here
        attention_cls = mm.Attention
    if getattr(attention_cls.forward, "_h3attn_patched", False):
        return False
    attention_cls.forward = make_attention_forward(attention_cls.forward, prologue, attention, timer)
    return True


def uninstall(attention_cls=None) -> bool:
    if attention_cls is None:
        import comfy.ldm.minimax.model as mm
        attention_cls = mm.Attention
    fwd = attention_cls.forward
    if not getattr(fwd, "_h3attn_patched", False):
        return False
    attention_cls.forward = fwd._h3attn_orig
    return True


def install_optimized_attention(module=None) -> bool:
    """Replace module.optimized_attention (as h3_profiler does, custom_nodes/h3_profiler/__init__.py:35,76)
    with a version that runs libh3attn for mask-free head_dim-128 bf16 calls and
    defers to the original otherwise.  A transformer_options override (the
    h3_sla sparse path) still receives every call first.  Idempotent."""
    if module is None:
        import comfy.ldm.minimax.model as module
    orig = module.optimized_attention
    if getattr(orig, "_h3attn_patched", False):
        return False

    def without_override(kw):
        opts = kw.get("transformer_options")
        if isinstance(opts, dict) and "optimized_attention_override" in opts:
            kw = dict(kw)
            kw["transformer_options"] = {n: x for n, x in opts.items() if n != "optimized_attention_override"}
        return kw

    def attention(q, k, v, heads, mask=None, *a, **kw):
        dim_ok = (q.shape[-1] == 128) if kw.get("skip_reshape", False) else (q.shape[-1] == heads * 128)
        if mask is None and not a and q.is_cuda and q.dtype == torch.bfloat16 and dim_ok:
            return hip_optimized_attention(q, k, v, heads, mask=None, **kw)
        # Any override has been applied by now: the original must not apply it again.
        return orig(q, k, v, heads, mask, *a, **without_override(kw))

    def optimized_attention(q, k, v, heads, mask=None, *a, **kw):
        # ComfyUI's optimized_attention hands every call to
        # transformer_options["optimized_attention_override"] when one is set,
        # as override(func, q, k, v, heads, mask=..., ...), func being the
        # attention it would otherwise run; the h3_sla override relies on it
        # (custom_nodes/h3_sla/__init__.py:265-284).
        opts = kw.get("transformer_options")
        override = opts.get("optimized_attention_override") if isinstance(opts, dict) else None
        if override is not None:
            if a:
                return override(attention, q, k, v, heads, mask, *a, **kw)
            return override(attention, q, k, v, heads, mask=mask, **kw)
        return attention(q, k, v, heads, mask, *a, **kw)

    optimized_attention._h3attn_patched = True
    optimized_attention._h3attn_orig = orig
    module.optimized_attention = optimized_attention
    return True
