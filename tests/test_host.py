"""Host-side logic on the CPU: the attn_sm80 drop-in shim, argument validation of
the tensor ops, the h3_sla schedule mirror, and the hook plumbing on a stand-in
DiT attention module (with torch callables injected in place of the kernels)."""
from __future__ import annotations

import subprocess
import sys

import numpy as np
import pytest
import torch

import attn_sm80
import h3attn
import oracle
import standin_dit
from conftest import ROOT
from h3attn import hooks, sla


# ----------------------------------------------------------------------------- attn_sm80 shim
def test_shim_backends_and_errors():
    """attn(q,k,v,backend) dispatch (attn_sm80/attn_sm80.py:37-42): unknown name -> ValueError(name)."""
    q = k = v = torch.randn(1, 2, 16, 128)
    with pytest.raises(ValueError, match="nope"):
        attn_sm80.attn(q, k, v, backend="nope")
    o = attn_sm80.attn(q, k, v, backend="sdpa")
    assert torch.allclose(o, torch.nn.functional.scaled_dot_product_attention(q, k, v))
    # the HIP backends refuse CPU tensors instead of computing on the CPU
    for name in ("hip", "fa3_sm80_h3", "fa3_pp"):
        with pytest.raises(ValueError, match="GPU"):
            attn_sm80.attn(q.bfloat16(), k.bfloat16(), v.bfloat16(), backend=name)


def test_shim_build_exposes_reference_extension_names():
    ext = attn_sm80._build()
    for name in ("fa3", "fa3_pp", "kernel_attrs", "pp_attrs", "get_prof", "reset_prof", "test_qk", "test_pv"):
        assert callable(getattr(ext, name))
    assert attn_sm80._build() is ext
    assert torch.equal(ext.get_prof(), torch.zeros(5, dtype=torch.float64))


def test_ops_validate_before_any_gpu_call():
    q = torch.zeros(1, 2, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        h3attn.attn_fwd(q, q, q)
    with pytest.raises(ValueError, match="bfloat16"):
        h3attn.attn_fwd(q.float(), q.float(), q.float())
    with pytest.raises(ValueError, match="head_dim"):
        h3attn.attn_fwd(q[..., :64], q[..., :64], q[..., :64])
    with pytest.raises(ValueError, match="4-D"):
        h3attn.attn_fwd(q[0], q[0], q[0])
    with pytest.raises(ValueError):
        h3attn.qk_rmsnorm_rope_(q, q, None, torch.ones(128), torch.ones(128), rot_dim=0)


def test_rope_table_layout():
    t = h3attn.rope_freqs(10, 64)
    assert tuple(t.shape) == (1, 10, 1, 32, 2, 2) and t.dtype == torch.float32
    assert np.allclose(t[0, :, 0].numpy(), oracle.rope_table(10, 64), atol=1e-7)
    assert torch.allclose(t[0, 3, 0, 2], torch.tensor([[t[0, 3, 0, 2, 0, 0], -t[0, 3, 0, 2, 1, 0]],
                                                      [t[0, 3, 0, 2, 1, 0], t[0, 3, 0, 2, 0, 0]]]))


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, f"{ROOT}/bench.py", "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2
    assert "one MI355X" in r.stderr


def test_bench_reads_traffic_from_the_committed_counter_summaries():
    """The roofline "traffic" of the dense, sparse and prologue bench lines comes from the
    profiles/ counter summaries (a "roofline.traffic[.key] = X B" line), not a constant."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench_mod", f"{ROOT}/bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    dense, src = bench.measured_traffic()
    assert src.endswith("attn_dense_h56_s42120_counters.txt") and 2.4e9 < dense < 2e10
    for blk in (128, 64):
        t, src = bench.measured_traffic(bench.SPARSE_TRAFFIC_SUMMARY, f"sparse{blk}")
        assert src.endswith("attn_sparse_h56_s42120_counters.txt") and 1e9 < t < 1e11, (blk, t, src)
    t, why = bench.measured_traffic(bench.SPARSE_TRAFFIC_SUMMARY, "sparse192")
    assert t is None and "no roofline.traffic" in why
    # the prologue moves each byte once: its counters read the algorithmic bytes
    t, src = bench.measured_traffic(bench.PROLOGUE_TRAFFIC_SUMMARY, "prologue")
    alg = bench.prologue_bytes(8192, 56, 128)
    assert src.endswith("prologue_s8192_h56.txt") and 0.99 * alg < t < 1.02 * alg, (t, alg)


# ----------------------------------------------------------------------------- h3_sla schedule
def test_schedule_parsing():
    assert sla.parse_ranges("31-42,46,48-49") == list(range(31, 43)) + [46, 48, 49]
    assert sla.parse_ranges("") == []
    m = sla.parse_layer_keep("25:31-33;0.2:43; ")
    assert m == {31: 0.25, 32: 0.25, 33: 0.25, 43: 0.2}


def test_resolve_schedule_presets():
    name, keeps = sla.resolve_schedule("off", topk=0.35)
    assert name == "off" and keeps == [0.35] * 50
    name, keeps = sla.resolve_schedule("quality")
    assert [l for l, k in enumerate(keeps) if k == 0.25] == list(range(31, 43)) + [46, 47, 48, 49]
    assert all(k == 0.15 for l, k in enumerate(keeps) if not (31 <= l <= 42 or 46 <= l <= 49))
    assert sla.resolve_schedule("speed")[1].count(0.25) == 9
    assert sla.resolve_schedule("balanced")[1].count(0.25) == 14
    name, keeps = sla.resolve_schedule("custom", topk=0.3, layer_keep="25:0-1;99:60")
    assert keeps[:3] == [0.25, 0.25, 0.3] and len(keeps) == 50
    with pytest.raises(ValueError):
        sla.resolve_schedule("fastest")


def test_keep_count():
    assert sla.keep_count(0.25, 330) == 82
    assert sla.keep_count(0.01, 10) == 1
    assert sla.keep_count(1.0, 7) == 7


# ----------------------------------------------------------------------------- hooks (CPU plumbing)
def _cpu_attention(q, k, v, heads, mask=None, skip_reshape=True, **_):
    return standin_dit._attention_impl(q, k, v, heads, skip_reshape=skip_reshape)


def _model(seed=0):
    torch.manual_seed(seed)
    m = standin_dit.Attention(256, 2)
    with torch.no_grad():
        m.q_norm.weight.mul_(1.1)
        m.k_norm.weight.mul_(0.9)
    return m


class _Attn(standin_dit.Attention):
    """Subclass so patching the class attribute does not leak into other tests."""


def test_install_patch_matches_stock_forward_and_is_idempotent():
    m = _model()
    m.__class__ = _Attn
    x = torch.randn(10, 256)
    rope = h3attn.rope_freqs(10, 128)
    with torch.no_grad():
        want = m(x, rope_freqs=rope)
        want_norope = m(x)
        assert hooks.install(_Attn, prologue=standin_dit.rms_rope_split_half_, attention=_cpu_attention)
        assert not hooks.install(_Attn, prologue=standin_dit.rms_rope_split_half_, attention=_cpu_attention)
        got = m(x, rope_freqs=rope)
        got_norope = m(x)  # rope_freqs=None falls through to the original forward
        assert hooks.uninstall(_Attn) and not hooks.uninstall(_Attn)
    assert torch.equal(got, want)
    assert torch.equal(got_norope, want_norope)


@pytest.mark.parametrize("scope_first", [True, False])
def test_install_and_scope_patch_compose_in_either_order(scope_first):
    """The patched forward sits beneath the scope wrapper whichever is installed first, so the
    override still sees the DiT scope and the layer tag; uninstall keeps the scope wrapper."""
    class A(standin_dit.Attention):
        pass

    torch.manual_seed(2)
    m = A(256, 2)
    m._h3sla_layer = 7
    seen = []

    def attention(q, k, v, heads, **kw):
        seen.append((hooks.in_dit_scope(), hooks._state.layer))
        return _cpu_attention(q, k, v, heads, **kw)

    if scope_first:
        hooks.install_scope_patch(A)
    assert hooks.install(A, prologue=standin_dit.rms_rope_split_half_, attention=attention)
    hooks.install_scope_patch(A)
    assert not hooks.install(A, prologue=standin_dit.rms_rope_split_half_, attention=attention)
    x, rope = torch.randn(10, 256), h3attn.rope_freqs(10, 128)
    with torch.no_grad():
        m(x, rope_freqs=rope)
        assert seen == [(True, 7)]
        assert hooks.uninstall(A) and not hooks.uninstall(A)
        assert getattr(A.forward, "_h3attn_scope", False)
        m(x, rope_freqs=rope)  # stock forward again: the attention above is no longer called
    assert seen == [(True, 7)]


def test_override_gate_and_fallback():
    calls = []

    def func(*a, **kw):
        calls.append("func")
        return "dense"

    def boom(*a, **kw):
        raise RuntimeError("kernel unavailable")

    logs = []
    ov = hooks.make_override(attention=lambda *a, **kw: "fast", log=logs.append)
    q4 = torch.zeros(1, 2, 4, 128)
    assert ov(func, q4, q4, q4, 2, mask=None, skip_reshape=True) == "fast"
    assert ov(func, q4, q4, q4, 2, mask=torch.ones(1), skip_reshape=True) == "dense"      # masked call
    assert ov(func, q4[..., :64], q4[..., :64], q4[..., :64], 2, skip_reshape=True) == "dense"  # D != 128
    assert ov(func, q4[0], q4[0], q4[0], 2, skip_reshape=False) == "dense"               # 3-D
    ov2 = hooks.make_override(attention=boom, log=logs.append)
    assert ov2(func, q4, q4, q4, 2, mask=None, skip_reshape=True) == "dense"
    assert any("kernel unavailable" in s for s in logs)
    assert ov.h3sla is None


def test_sla_override_scope_schedule_and_fallback():
    class _A(standin_dit.Attention):
        pass

    hooks.install_scope_patch(_A)
    f1 = _A.forward
    hooks.install_scope_patch(_A)  # idempotent
    assert _A.forward is f1
    seen = {}

    def func(q, k, v, heads, **kw):
        seen["in_scope"] = hooks.in_dit_scope()
        return standin_dit._attention_impl(q, k, v, heads, **kw)

    sched = hooks.Schedule("custom", [1.0] * 50, blk=64)
    logs = []
    ov = hooks.make_sla_override(schedule=sched, log=logs.append)
    assert ov.h3sla is sched
    assert hooks.get_schedule({"optimized_attention_override": ov}) is sched
    assert hooks.get_schedule({}) is None
    torch.manual_seed(1)
    m = _A(256, 2)
    m._h3sla_layer = 3
    x = torch.randn(12, 256)
    opts = {"optimized_attention_override": lambda fn, *a, **kw: ov(func, *a, **kw)}
    with torch.no_grad():
        m(x, rope_freqs=h3attn.rope_freqs(12, 128), transformer_options=opts)
    assert seen["in_scope"] is True and not hooks.in_dit_scope()
    # keep < 1 on CPU tensors: the sparse kernel refuses them -> logged fallback to dense
    sched.keeps[3] = 0.25
    with torch.no_grad():
        m(x, rope_freqs=h3attn.rope_freqs(12, 128), transformer_options=opts)
    assert any("fell back" in s for s in logs)
    # outside DiT scope (rope_freqs=None): the override passes straight to func
    logs.clear()
    with torch.no_grad():
        m(x, transformer_options=opts)
    assert logs == [] and seen["in_scope"] is False
    assert sched.keep_for(None) == sched.default_keep and sched.keep_for(99) == sched.default_keep


def test_sla_block_size_checked_at_construction():
    """Every size the node offers (16..256 step 16, custom_nodes/h3_sla/__init__.py:315) is accepted;
    others fail when the schedule/override is built (as the node fails at patch time, h3_sla:331),
    not by silently running dense later."""
    assert sla.SUPPORTED_BLOCKS == tuple(range(16, 257, 16))
    for blk in (0, 8, 24, 100, 272, 512, -64):
        with pytest.raises(ValueError, match="block size"):
            hooks.Schedule("custom", [0.5] * 50, blk=blk)
        with pytest.raises(ValueError, match="block size"):
            hooks.make_sla_override(topk=0.5, blk=blk)
        with pytest.raises(ValueError, match="block size"):
            sla.sparse_attention(torch.zeros(1, 1, 8, 128), torch.zeros(1, 1, 8, 128),
                                 torch.zeros(1, 1, 8, 128), 0.5, blk)
    for blk in sla.SUPPORTED_BLOCKS:
        assert hooks.Schedule("custom", [0.5] * 50, blk=blk).blk == blk
        assert callable(hooks.make_sla_override(topk=0.5, blk=blk))


def test_schedule_summary_and_format():
    """schedule_summary / format_summary (custom_nodes/h3_sla/__init__.py:110-136)."""
    name, keeps = sla.resolve_schedule("balanced")
    sm = sla.schedule_summary(name, keeps, 128)
    assert sm["preset"] == "balanced" and sm["research_name"] == "T2" and sm["blk"] == 128
    assert sm["default_keep"] == 0.15
    assert sm["layers_by_keep"] == {"SLA25": "31-42,48-49"}
    assert sm["counts"] == {"15": 36, "25": 14}
    text = sla.format_summary(sm).splitlines()
    assert text == ["[h3_sla] SLA preset: balanced (research T2)", "[h3_sla] default keep: 15%",
                    "[h3_sla] SLA25 layers: 31-42,48-49", "[h3_sla] layer counts: SLA15=36, SLA25=14"]
    sm = sla.schedule_summary("custom", [0.3, 0.3, 0.2, 0.3, 0.2, 0.2, 0.2])
    assert sm["default_keep"] == 0.2 and sm["layers_by_keep"] == {"SLA30": "0-1,3"}
    assert sla._ranges_str([5, 1, 2, 3, 9]) == "1-3,5,9"
    assert hooks.Schedule(name, keeps, blk=64).summary["layers_by_keep"] == {"SLA25": "31-42,48-49"}


def test_schedule_timing_buckets(monkeypatch):
    """H3_SLA_TIMING: events around each sparse layer, resolved at the step's last layer (h3_sla:199-212)."""
    monkeypatch.setattr(torch.cuda, "Event", lambda enable_timing=True: _FakeSyncEvent())
    monkeypatch.setattr(sla, "sparse_attention", lambda q, k, v, keep, blk, **kw: q)
    monkeypatch.setenv("H3_SLA_TIMING", "1")
    sched = hooks.Schedule("custom", [0.5, 1.0, 0.5], blk=64)
    assert sched.timing
    q = torch.zeros(1, 1, 4, 128)
    for _ in range(2):  # two steps of three layers
        for layer in range(3):
            out = sched.run(layer, q, q, q)
            assert (out is None) == (layer == 1)
    assert sched.attn_n == [2, 0, 2] and sched._ev == []
    ms = sched.attn_ms_per_layer_call()
    assert ms[1] is None and ms[0] > 0 and ms[2] > 0
    monkeypatch.setenv("H3_SLA_TIMING", "0")
    assert not hooks.Schedule("custom", [0.5], blk=64).timing


class _FakeSyncEvent:
    clock = [0]

    def record(self):
        _FakeSyncEvent.clock[0] += 1
        self.t = _FakeSyncEvent.clock[0]

    def synchronize(self):
        pass

    def elapsed_time(self, other):
        return float(other.t - self.t)


class _LostEvent(_FakeSyncEvent):
    def synchronize(self):
        raise RuntimeError("event lost")


def test_schedule_timing_with_a_dense_last_layer(monkeypatch):
    """Events are resolved at a step's last layer even when it runs dense, and at layer 0 of the
    next step; a failure while resolving them is logged and never reaches the layer's output."""
    monkeypatch.setattr(torch.cuda, "Event", lambda enable_timing=True: _FakeSyncEvent())
    monkeypatch.setattr(sla, "sparse_attention", lambda q, k, v, keep, blk, **kw: q)
    logs = []
    sched = hooks.Schedule("custom", [0.5, 0.5, 1.0], blk=64, timing=True, log=logs.append)
    q = torch.zeros(1, 1, 4, 128)
    for _ in range(3):
        for layer in range(3):
            sched.run(layer, q, q, q)
        assert sched._ev == []
    assert sched.attn_n == [3, 3, 0]
    # a step cut short after layer 0: its event is resolved by the next step's layer 0
    sched.run(0, q, q, q)
    assert len(sched._ev) == 1
    sched.run(0, q, q, q)
    assert sched.attn_n[0] == 4 and len(sched._ev) == 1
    monkeypatch.setattr(torch.cuda, "Event", lambda enable_timing=True: _LostEvent())
    sched._ev = []
    assert sched.run(0, q, q, q) is q and sched.run(1, q, q, q) is q
    assert sched.run(2, q, q, q) is None  # dense layer: resolves (and drops) the lost events
    assert sched._ev == [] and any("timing events dropped" in s for s in logs)


def _patcher(depth=50, dim=256, heads=2, seed=0):
    class A(standin_dit.Attention):
        pass

    torch.manual_seed(seed)
    return standin_dit.ModelPatcher(standin_dit.MiniMaxH3Model(dim, heads, depth, attention_cls=A)), A


@pytest.mark.parametrize("preset,layer_keep", [("off", ""), ("quality", ""), ("balanced", ""), ("speed", ""),
                                               ("custom", "25:31-42,46-49;20:43;100:0,17")])
def test_patch_model_runs_each_layer_at_its_scheduled_keep(monkeypatch, preset, layer_keep):
    """hooks.patch_model (H3SLAPatch.patch, custom_nodes/h3_sla/__init__.py:328-346) on a 50-block
    stand-in DiT: one forward runs every layer at the keep resolve_schedule gives it (layers at
    keep 1 run dense through the original attention), for every preset."""
    used, dense = [], []

    def fake_sparse(q, k, v, keep, blk, **kw):
        used.append((hooks._state.layer, keep, blk))
        return q.clone()

    monkeypatch.setattr(sla, "sparse_attention", fake_sparse)
    mp, A = _patcher()
    logs = []
    pm = hooks.patch_model(mp, topk=0.35, blk=64, preset=preset, layer_keep=layer_keep, log=logs.append)
    assert pm is not mp and mp.model_options == {"transformer_options": {}}
    assert hooks.in_dit_scope() is False and getattr(A.forward, "_h3attn_scope", False)
    x = torch.randn(12, 256)
    rope = h3attn.rope_freqs(12, 128)
    impl = standin_dit._attention_impl
    monkeypatch.setattr(standin_dit, "_attention_impl",
                        lambda *a, **kw: dense.append(hooks._state.layer) or impl(*a, **kw))
    with torch.no_grad():
        pm(x, rope)
    name, keeps = sla.resolve_schedule(preset, 0.35, layer_keep, 50)
    sched = hooks.get_schedule(pm.model_options["transformer_options"])
    if preset == "off":
        assert sched is None  # one keep everywhere: no schedule, no layer tags
        assert used == [(None, 0.35, 64)] * 50 and dense == []
        assert any("topk=0.350" in s for s in logs)
        return
    assert sched.keeps == keeps and sched.name == name and sched.blk == 64
    assert [layer for layer, _, _ in used] == [i for i, kv in enumerate(keeps) if kv < 1]
    assert [kv for _, kv, _ in used] == [kv for kv in keeps if kv < 1]
    assert dense == [i for i, kv in enumerate(keeps) if kv >= 1]
    assert [b.attn._h3sla_layer for b in mp.model.diffusion_model.blocks] == list(range(50))
    assert sla.format_summary(sched.summary) in "\n".join(logs)
    if preset == "balanced":  # the 14 layers at 0.25 that an untagged model would run at 0.15
        assert [i for i, kv in enumerate(keeps) if kv == 0.25] == list(range(31, 43)) + [48, 49]


def test_patch_model_disabled_and_bad_arguments(monkeypatch):
    mp, A = _patcher(depth=3)
    assert hooks.patch_model(mp, enabled=False) is mp
    with pytest.raises(ValueError, match="preset"):
        hooks.patch_model(mp, preset="fastest")
    with pytest.raises(ValueError, match="block size"):
        hooks.patch_model(mp, blk=40)
    assert mp.model_options == {"transformer_options": {}}


def test_schedule_reports_each_generation_at_its_first_sigma(monkeypatch):
    """Layer 0 at a run's first sigma logs the schedule summary (rank 0) and counts a generation
    (custom_nodes/h3_sla/__init__.py:155-170); later steps of the same run do not."""
    monkeypatch.setattr(sla, "sparse_attention", lambda q, k, v, keep, blk, **kw: q.clone())
    mp, _ = _patcher(depth=4)
    logs = []
    pm = hooks.patch_model(mp, topk=0.15, preset="custom", layer_keep="25:1-2", log=logs.append)
    sched = hooks.get_schedule(pm.model_options["transformer_options"])
    head = "[h3_sla] SLA preset: custom"
    assert sum(s.count(head) for s in logs) == 1  # at patch time
    logs.clear()
    x, rope = torch.randn(12, 256), h3attn.rope_freqs(12, 128)
    sigmas = [14.6, 7.0, 2.0, 0.0]
    with torch.no_grad():
        for _ in range(2):
            for s in sigmas[:-1]:
                pm(x, rope, sigma=s, sample_sigmas=sigmas)
        assert sched.generation == 2 and sum(s.count(head) for s in logs) == 2
        monkeypatch.setenv("RANK", "1")  # other ranks count but do not log
        pm(x, rope, sigma=sigmas[0], sample_sigmas=sigmas)
        monkeypatch.delenv("RANK")
        assert sched.generation == 3 and sum(s.count(head) for s in logs) == 2
        pm(x, rope)  # no sigmas: every call counts as a first step
    assert sched.generation == 4


def test_tag_layers():
    mp, _ = _patcher(depth=5)
    blocks = mp.model.diffusion_model.blocks
    assert hooks.tag_layers(mp) == 5
    assert [b.attn._h3sla_layer for b in blocks] == [0, 1, 2, 3, 4]
    assert hooks.tag_layers(mp.model.diffusion_model) == 5
    assert hooks.tag_layers(list(blocks)[2:]) == 3 and blocks[2].attn._h3sla_layer == 0
    logs = []
    assert hooks.tag_layers(object(), log=logs.append) is None
    assert any("could not tag" in s for s in logs)


def test_comfy_node_interface(monkeypatch):
    """node.H3SLAPatch has the h3_sla node's inputs and output (custom_nodes/h3_sla/__init__.py:308-346)."""
    from h3attn import node
    monkeypatch.setattr(sla, "sparse_attention", lambda q, k, v, keep, blk, **kw: q.clone())
    cls = node.NODE_CLASS_MAPPINGS["H3SLAPatch"]
    spec = cls.INPUT_TYPES()
    assert list(spec["required"]) == ["model", "topk", "blk", "enabled"]
    assert list(spec["optional"]) == ["preset", "layer_keep"]
    assert spec["required"]["topk"][1]["default"] == 0.35 and spec["required"]["blk"][1]["default"] == 64
    assert spec["optional"]["preset"][0] == sla.PRESET_CHOICES
    assert cls.RETURN_TYPES == ("MODEL",) and cls.FUNCTION == "patch"
    lo, hi, step = (spec["required"]["blk"][1][k] for k in ("min", "max", "step"))
    assert set(range(lo, hi + 1, step)) == set(sla.SUPPORTED_BLOCKS)
    mp, _ = _patcher(depth=50)
    (pm,) = cls().patch(mp, 0.35, 64, True, "speed", "")
    assert hooks.get_schedule(pm.model_options["transformer_options"]).keeps == sla.resolve_schedule("speed")[1]
    assert cls().patch(mp, 0.35, 64, False)[0] is mp


def test_installed_optimized_attention_still_calls_the_override():
    """With hooks.install_optimized_attention in place, a transformer_options override (the
    h3_sla sparse path) still receives every call first, as ComfyUI's wrapper does."""
    import types
    mod = types.SimpleNamespace(optimized_attention=standin_dit.optimized_attention)
    assert hooks.install_optimized_attention(mod)
    seen = []

    def override(func, *args, **kwargs):
        seen.append((func, kwargs.get("mask"), "optimized_attention_override" in kwargs["transformer_options"]))
        return func(*args, **kwargs)  # fall back, as a gated-off override does

    q, k, v = (torch.randn(1, 2, 6, 128) for _ in range(3))
    opts = {"optimized_attention_override": override, "other": 1}
    got = mod.optimized_attention(q, k, v, 2, skip_reshape=True, transformer_options=opts)
    want = standin_dit.optimized_attention(q, k, v, 2, skip_reshape=True)
    assert len(seen) == 1 and seen[0][1] is None and seen[0][2]
    assert torch.equal(got, want)  # CPU tensors: the fallback reaches the original exactly once
    assert mod.optimized_attention(q, k, v, 2, skip_reshape=True).shape == (1, 6, 256)
    assert len(seen) == 1


# ----------------------------------------------------------------------------- per-component timing
class _FakeEvent:
    """record() stamps a shared tick counter; elapsed_time is the tick difference."""
    clock = [0]

    def record(self):
        _FakeEvent.clock[0] += 1
        self.t = _FakeEvent.clock[0]

    def elapsed_time(self, other):
        return float(other.t - self.t)


def test_op_timer_bookkeeping():
    from h3attn import profiling
    syncs = []
    t = profiling.OpTimer(event_factory=_FakeEvent, synchronize=lambda: syncs.append(1))
    assert t.mark("x", lambda a: a + 1, 1) == 2  # disarmed: plain call, nothing recorded
    assert t.report()["components_ms"] == {}
    t.arm()
    t.mark("attn.qkv", lambda: None)
    t.mark("attn.softmax", lambda: [e.record() for e in (_FakeEvent(), _FakeEvent())])  # 2 inner ticks
    t.mark("attn.qkv", lambda: None)
    t.disarm()
    t.mark("attn.qkv", lambda: None)  # not counted
    rep = t.report(total_ms=10.0)
    assert rep["calls"] == {"attn.qkv": 2, "attn.softmax": 1}
    assert rep["components_ms"] == {"attn.qkv": 2.0, "attn.softmax": 3.0}
    assert rep["sum_components_ms"] == 5.0 and rep["other_ms"] == 5.0
    assert rep["components_pct"] == {"attn.qkv": 20.0, "attn.softmax": 30.0}
    assert syncs
    t.arm()  # a new measurement starts empty
    assert t.report()["components_ms"] == {}


def test_patched_forward_marks_reference_components():
    from h3attn import profiling

    class A(standin_dit.Attention):
        pass

    m = _model(3)
    m.__class__ = A
    x = torch.randn(12, 256)
    rope = h3attn.rope_freqs(12, 128)
    timer = profiling.OpTimer(event_factory=_FakeEvent, synchronize=lambda: None)
    with torch.no_grad():
        want = m(x, rope_freqs=rope)
        assert hooks.install(A, prologue=standin_dit.rms_rope_split_half_, attention=_cpu_attention,
                             timer=timer)
        got_idle = m(x, rope_freqs=rope)
        timer.arm()
        got = m(x, rope_freqs=rope)
        m(x, rope_freqs=rope)
        timer.disarm()
        hooks.uninstall(A)
    assert torch.equal(got, want) and torch.equal(got_idle, want)
    rep = timer.report()
    assert rep["calls"] == {c: 2 for c in profiling.COMPONENTS}
