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

from . import _lib, ops, profiling, sla

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
def _scope_wrap(fwd):
    """`fwd` with the DiT-scope flag and the block's layer tag set around each call."""
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
    return scoped


def install_scope_patch(attention_cls) -> None:
    """Mark DiT-block attention calls (rope_freqs is not None) in a thread-local flag (idempotent).

    The scope wrapper stays outermost: install() / uninstall() place the
    patched forward beneath it whichever of the two is installed first.
    """
    if not getattr(attention_cls.forward, "_h3attn_scope", False):
        attention_cls.forward = _scope_wrap(attention_cls.forward)


def in_dit_scope() -> bool:
    return bool(getattr(_state, "on", False))


def _first_sigma(transformer_options) -> bool:
    """True at the first sampling step of a run: the current sigma is the schedule's first.

    ComfyUI passes the step's sigma as transformer_options["sigmas"] and the
    run's whole schedule as ["sample_sigmas"]; without either (or if they
    cannot be read) every call counts as a first step, as the node treats it
    (custom_nodes/h3_sla/__init__.py:157-162).
    """
    try:
        cur = transformer_options.get("sigmas")
        run = transformer_options.get("sample_sigmas")
        if cur is None or run is None:
            return True
        return float(cur.flatten()[0]) >= float(run.flatten()[0]) - 1e-6
    except Exception:
        return True


class Schedule:
    """Per-layer keep ratios (custom_nodes/h3_sla/__init__.py:139-212, without the status file).

    blk is checked here, when the schedule is built, as the node checks its
    kernel when it patches the model (h3_sla:331): an unsupported size raises
    ValueError instead of turning every sparse layer into a dense one later.

    Layer 0 of every step resolves the timing events still pending from the
    previous step; layer 0 of a run's first step (its first sigma) also counts
    a new generation and logs the schedule summary on rank 0
    (h3_sla:155-170).  timing (default: env H3_SLA_TIMING == "1", as at
    h3_sla:147) records HIP events around each sparse layer; they are also
    resolved at a step's last layer, whatever its keep, into attn_ms / attn_n
    per layer.  A failure while resolving them is logged and drops the
    events: timing never changes what a layer computes.
    """

    def __init__(self, name: str, keeps, blk: int = 64, force_diag: bool = False, smooth_k: bool = True,
                 timing: bool | None = None, log=print):
        self.name, self.keeps, self.blk = name, [float(x) for x in keeps], sla.check_block(blk)
        self.force_diag, self.smooth_k = force_diag, smooth_k
        self.default_keep = max(set(self.keeps), key=self.keeps.count) if self.keeps else 1.0
        self.summary = sla.schedule_summary(name, self.keeps, self.blk) if self.keeps else None
        self.timing = (os.environ.get("H3_SLA_TIMING") == "1") if timing is None else bool(timing)
        self.log = log
        self.generation = 0
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
        pending, self._ev = self._ev, []
        try:
            pending[-1][2].synchronize()
            times = [(layer, a.elapsed_time(b)) for layer, a, b in pending]
        except Exception as e:
            self.log(f"[h3_sla] timing events dropped: {e}")
            return
        for layer, ms in times:
            self.attn_ms[layer] += ms
            self.attn_n[layer] += 1

    def generation_start(self, transformer_options) -> bool:
        """Layer 0 of a step: flush timings; at a run's first sigma, count and report a generation."""
        self.flush_timing()
        if not _first_sigma(transformer_options or {}):
            return False
        self.generation += 1
        if int(os.environ.get("RANK", "0")) == 0 and self.summary is not None:
            self.log(sla.format_summary(self.summary))
        return True

    def attn_ms_per_layer_call(self):
        """Mean sparse-attention ms per call for each layer (None where it never ran)."""
        return [round(m / n, 3) if n else None for m, n in zip(self.attn_ms, self.attn_n)]

    def _sparse(self, q, k, v, keep, pooled=None):
        return sla.sparse_attention(q, k, v, keep, self.blk, force_diag=self.force_diag, smooth_k=self.smooth_k,
                                    pooled=pooled)

    def run(self, layer, q, k, v, transformer_options=None, pooled=None):
        """[1,H,S,D] sparse output, or None (keep >= 1: caller runs dense).

        pooled: the layer's block means from the prologue, if it took them.
        """
        if layer == 0:
            self.generation_start(transformer_options)
        keep = self.keep_for(layer)
        tracked = self.timing and layer is not None and 0 <= layer < len(self.keeps)
        last = layer is not None and layer == len(self.keeps) - 1
        if keep >= 1.0:
            if last:
                self.flush_timing()
            return None
        if not tracked:
            return self._sparse(q, k, v, keep, pooled)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        o = self._sparse(q, k, v, keep, pooled)
        b.record()
        self._ev.append((layer, a, b))
        if last:
            self.flush_timing()
        return o


def make_sla_override(topk: float = 0.35, blk: int = 64, schedule: Schedule | None = None,
                      log=print):
    """HIP counterpart of h3_sla's _make_override (custom_nodes/h3_sla/__init__.py:265-284).

    Active only inside DiT-block attention (install_scope_patch) with mask=None
    and head_dim 128; returns [1,S,H*D].  Without a schedule every such call
    keeps `topk`; with one, the layer index the scope patch recorded picks the
    keep (a keep of 1 or more leaves the layer to `func`, dense).  Any
    exception is logged and the call goes to `func`, so a sparse failure
    costs speed, never the output.  The block size is checked here
    (ValueError), not at the first call.
    """
    blk = sla.check_block(blk)

    def sparse(q, k, v, transformer_options):
        pooled = _take_pooled(q, k, blk)
        if schedule is None:
            return sla.sparse_attention(q, k, v, topk, blk, pooled=pooled)
        return schedule.run(getattr(_state, "layer", None), q, k, v, transformer_options, pooled=pooled)

    def plan(layer):
        """(keep, blk) this override applies to DiT layer `layer`."""
        return (float(topk) if schedule is None else schedule.keep_for(layer)), blk

    def override(func, *args, **kwargs):
        if in_dit_scope() and _gate(args, kwargs):
            q, k, v = args[0], args[1], args[2]
            try:
                o = sparse(q, k, v, kwargs.get("transformer_options"))
            except Exception as e:
                log(f"[h3attn] sparse override fell back to dense: {e}")
                o = None
            if o is not None:
                _, H, S, D = q.shape
                return o.transpose(1, 2).reshape(1, S, H * D)
        return func(*args, **kwargs)

    override.h3sla = schedule
    override.h3attn_plan = plan
    return override


def _pool_blk_for(transformer_options):
    """Block size at which the patched forward's prologue should also pool q and k: the active
    override is an h3attn sparse override that will run this DiT layer block-sparse; else None."""
    if not in_dit_scope():
        return None
    try:
        plan = getattr((transformer_options or {}).get("optimized_attention_override"), "h3attn_plan", None)
        if plan is None:
            return None
        keep, blk = plan(getattr(_state, "layer", None))
        return blk if keep < 1.0 else None
    except Exception:
        return None


def _take_pooled(q, k, blk):
    """The block means the prologue left for this q, k and block size (consumed), or None."""
    p = getattr(_state, "pooled", None)
    _state.pooled = None
    if p is None or p[0] != q.data_ptr() or p[1] != k.data_ptr() or p[2] != blk:
        return None
    return p[3], p[4]


def _dit_blocks(model):
    """The DiT blocks of a ModelPatcher (.model.diffusion_model.blocks), a diffusion model (.blocks)
    or a sequence of blocks."""
    for path in (("model", "diffusion_model", "blocks"), ("diffusion_model", "blocks"), ("blocks",)):
        obj = model
        for name in path:
            obj = getattr(obj, name, None)
            if obj is None:
                break
        if obj is not None:
            return list(obj)
    if isinstance(model, (list, tuple)) or hasattr(model, "__iter__"):
        return list(model)
    raise AttributeError(f"no DiT blocks found on {type(model).__name__}")


def tag_layers(model, log=print):
    """Record each DiT block's index as block.attn._h3sla_layer; returns the block count or None.

    The scope patch reads the tag, so a per-layer schedule knows which layer
    it runs (custom_nodes/h3_sla/__init__.py:296-305).  A model without
    MiniMax-H3 blocks is logged and left untagged (None): every call then
    gets the schedule's default keep.
    """
    try:
        blocks = _dit_blocks(model)
        for i, block in enumerate(blocks):
            block.attn._h3sla_layer = i
        return len(blocks)
    except Exception as e:
        log(f"[h3_sla] could not tag DiT layers ({e}); per-layer presets need MiniMax-H3 blocks")
        return None


def _attention_class(model):
    """The class of the model's DiT-block attention, else comfy.ldm.minimax.model.Attention."""
    try:
        return type(_dit_blocks(model)[0].attn)
    except Exception:
        import comfy.ldm.minimax.model as mm  # ComfyUI is optional: imported only here
        return mm.Attention


def patch_model(model, topk: float = 0.35, blk: int = 64, enabled: bool = True, preset: str = "off",
                layer_keep: str = "", attention_cls=None, log=print):
    """The H3SLAPatch node's patch() on libh3attn (custom_nodes/h3_sla/__init__.py:328-346).

    Returns a clone of the ComfyUI ModelPatcher `model` whose
    transformer_options carry the block-sparse override, or `model` itself
    when not enabled.  preset "off": one keep (`topk`) on every DiT layer.
    Otherwise the blocks are tagged with their layer index, the per-layer
    schedule is resolved (sla.resolve_schedule) and logged.  The scope patch
    goes on `attention_cls` (by default the class of the blocks' attention
    modules, comfy.ldm.minimax.model.Attention in ComfyUI) and the library is loaded here, so that a missing build fails now rather
    than mid-render.  An unsupported `blk` or preset raises ValueError.
    """
    if not enabled:
        return model
    blk = sla.check_block(blk)
    if attention_cls is None:
        attention_cls = _attention_class(model)
    install_scope_patch(attention_cls)
    _lib.lib()
    m = model.clone()
    m.model_options = dict(m.model_options)
    opts = dict(m.model_options.get("transformer_options", {}))
    m.model_options["transformer_options"] = opts
    mode = (preset or "off").lower()
    if mode == "off":
        opts["optimized_attention_override"] = make_sla_override(float(topk), blk, log=log)
        log(f"[h3_sla] H3SLAPatch: topk={float(topk):.3f} (sparsity={100 * (1 - float(topk)):.0f}%) blk={blk}")
        return m
    n = tag_layers(m, log=log) or 50
    name, keeps = sla.resolve_schedule(mode, float(topk), layer_keep, n)
    sched = Schedule(name, keeps, blk, log=log)
    opts["optimized_attention_override"] = make_sla_override(float(topk), blk, schedule=sched, log=log)
    log(f"[h3_sla] H3SLAPatch: per-layer schedule blk={blk}\n" + sla.format_summary(sched.summary))
    return m


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

    When the HIP prologue runs and the transformer_options carry an h3attn
    sparse override that will run this layer block-sparse, the prologue also
    pools q and k at the override's block size (h3a_qk_rmsnorm_rope_pool) and
    leaves the means for the override, so the block map does not read q and
    k again.
    """
    mark = timer.mark if timer is not None else profiling.passthrough
    fuse_pool = prologue is ops.rms_rope_split_half_

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
        qw, kw = _weight(self.q_norm.weight, x.device), _weight(self.k_norm.weight, x.device)
        _state.pooled = None
        pool_blk = _pool_blk_for(transformer_options) if fuse_pool else None
        if pool_blk is None:
            mark("attn.qknorm_rope", prologue, q, k, rope_freqs, qw, kw, epsilon=self.q_norm.eps, rot_dim=rot)
        else:
            pq, pk = mark("attn.qknorm_rope", ops.qk_rmsnorm_rope_, q, k, rope_freqs, qw, kw,
                          eps=self.q_norm.eps, rot_dim=rot, pool_blk=pool_blk)
            _state.pooled = (q.data_ptr(), k.data_ptr(), pool_blk, pq, pk)
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
    fwd = attention_cls.forward
    scoped = getattr(fwd, "_h3attn_scope", False)
    inner = fwd._h3attn_orig if scoped else fwd
    if getattr(inner, "_h3attn_patched", False):
        return False
    patched = make_attention_forward(inner, prologue, attention, timer)
    attention_cls.forward = _scope_wrap(patched) if scoped else patched
    return True


def uninstall(attention_cls=None) -> bool:
    if attention_cls is None:
        import comfy.ldm.minimax.model as mm
        attention_cls = mm.Attention
    fwd = attention_cls.forward
    scoped = getattr(fwd, "_h3attn_scope", False)
    inner = fwd._h3attn_orig if scoped else fwd
    if not getattr(inner, "_h3attn_patched", False):
        return False
    attention_cls.forward = _scope_wrap(inner._h3attn_orig) if scoped else inner._h3attn_orig
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
