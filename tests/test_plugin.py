"""The vLLM-facing surface on the CPU, against stand-in vLLM modules: the
package and entry point (the reference's pyproject.toml:34-35,
src/sluice/__init__.py:4-7), the general_plugins hook
(src/sluice/plugin.py:27-96), the engine settings the offloader applies
(envelope, split points, speculative depth: src/sluice/offloader.py:786-851),
the wrapped quant_method.apply (1085-1122), the forward-context split
signal (1766-1800), the router settings mapped onto the routing kernel
(select_experts as called at 2583-2585) and get_stats' schema (2804-2814)."""

import importlib
import logging
import os
import sys
import types

import pytest
import torch
import torch.nn as nn

from sluice_amd import plugin
from sluice_amd.offloader import ExpertStreamOffloader, route_spec

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _mod(monkeypatch, name, **attrs):
    m = types.ModuleType(name)
    for k, v in attrs.items():
        setattr(m, k, v)
    monkeypatch.setitem(sys.modules, name, m)
    parent, _, leaf = name.rpartition(".")
    if parent and parent in sys.modules:
        monkeypatch.setattr(sys.modules[parent], leaf, m, raising=False)
    return m


def _stub_vllm(monkeypatch, v2=False, cfg=None, ctx=None):
    _mod(monkeypatch, "vllm")
    _mod(monkeypatch, "vllm.envs", VLLM_USE_V2_MODEL_RUNNER=v2)
    _mod(monkeypatch, "vllm.model_executor")
    _mod(monkeypatch, "vllm.model_executor.offloader")
    base = _mod(monkeypatch, "vllm.model_executor.offloader.base",
                create_offloader=lambda cfg: "stock")
    _mod(monkeypatch, "vllm.v1")
    _mod(monkeypatch, "vllm.v1.worker")

    class GPUModelRunner:
        def load_model(self):
            self.model = torch.nn.Linear(2, 2)
            return "loaded"

    gmr = _mod(monkeypatch, "vllm.v1.worker.gpu_model_runner",
               create_offloader=base.create_offloader, GPUModelRunner=GPUModelRunner)
    _mod(monkeypatch, "vllm.config", get_current_vllm_config=lambda: cfg)
    _mod(monkeypatch, "vllm.forward_context", get_forward_context=lambda: ctx)
    return base, gmr


def test_register_is_inert_without_slots_and_warns_on_bad_values(monkeypatch, caplog):
    base, _ = _stub_vllm(monkeypatch)
    monkeypatch.delenv("SLUICE_SLOTS", raising=False)
    plugin.register()
    assert base.create_offloader(None) == "stock"
    for bad in ("abc", "0", "-3"):
        monkeypatch.setenv("SLUICE_SLOTS", bad)
        with caplog.at_level(logging.WARNING, logger="sluice"):
            plugin.register()
        assert "ignoring invalid SLUICE_SLOTS" in caplog.text
        assert base.create_offloader(None) == "stock"


def test_register_refuses_the_v2_runner(monkeypatch):
    _stub_vllm(monkeypatch, v2=True)
    monkeypatch.setenv("SLUICE_SLOTS", "48")
    with pytest.raises(RuntimeError, match="V1 model runner"):
        plugin.register()


def test_entry_point_resolves_to_the_sluice_package():
    """The general_plugins entry point is the reference's
    (sluice = "sluice.plugin:register"), and the sluice package has the
    reference's import surface."""
    import tomli
    from importlib.metadata import EntryPoint

    with open(os.path.join(ROOT, "pyproject.toml"), "rb") as f:
        eps = tomli.load(f)["project"]["entry-points"]["vllm.general_plugins"]
    assert eps == {"sluice": "sluice.plugin:register"}
    ep = EntryPoint(name="sluice", value=eps["sluice"], group="vllm.general_plugins")
    assert ep.load() is plugin.register
    sluice = importlib.import_module("sluice")
    assert sluice.__version__ == "0.1.0"
    assert sluice.ExpertStreamOffloader is ExpertStreamOffloader
    assert importlib.import_module("sluice.offloader").ExpertStreamOffloader is \
        ExpertStreamOffloader
    assert importlib.import_module("sluice.plugin").register is plugin.register


def test_register_patches_factory_and_load_model(monkeypatch):
    base, gmr = _stub_vllm(monkeypatch)
    monkeypatch.setenv("SLUICE_SLOTS", "48")
    orig_load = gmr.GPUModelRunner.load_model
    plugin.register()
    try:
        off = base.create_offloader(None)
        assert isinstance(off, ExpertStreamOffloader) and off.expert_cache_slots == 48
        assert gmr.create_offloader is base.create_offloader
        seen = []
        monkeypatch.setattr(off, "attach_model", lambda m: seen.append(m))
        r = gmr.GPUModelRunner()
        assert r.load_model() == "loaded"
        assert seen == [r.model]  # attach_model runs on the loaded model
    finally:
        gmr.GPUModelRunner.load_model = orig_load


def _cfg(**kw):
    ns = types.SimpleNamespace
    return ns(model_config=ns(hf_config=ns(num_experts_per_tok=kw.get("topk", 6))),
              compilation_config=ns(splitting_ops=list(kw.get("ops", []))),
              scheduler_config=ns(max_num_batched_tokens=kw.get("mbt", 8)),
              speculative_config=(ns(num_speculative_tokens=kw["spec"]) if "spec" in kw
                                  else None))


def _off(monkeypatch, slots=48, **env):
    for k in ("SLUICE_ROUTER_SPLIT", "SLUICE_PIECEWISE"):
        monkeypatch.delenv(k, raising=False)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    return ExpertStreamOffloader(expert_cache_slots=slots)


def test_router_split_envelope_and_split_points(monkeypatch):
    off = _off(monkeypatch, SLUICE_ROUTER_SPLIT="1", SLUICE_PIECEWISE="1")
    cfg = _cfg(mbt=8, ops=["vllm::unified_attention"], spec=2)
    off.post_init(cfg)
    assert off._rs_thr == 8                       # 48 slots // top-6
    assert cfg.compilation_config.splitting_ops == [
        "vllm::unified_attention", "vllm::moe_forward", "vllm::moe_forward_shared",
        "vllm::sluice_stream_gap"]
    assert off._spec_tokens == 2
    with pytest.raises(RuntimeError, match="max_num_batched_tokens=9 > slots//topk=8"):
        off.post_init(_cfg(mbt=9))
    # Qwen3-style config: top-k under text_config
    cfg = _cfg(mbt=8)
    cfg.model_config.hf_config = types.SimpleNamespace(
        text_config=types.SimpleNamespace(num_experts_per_tok=8))
    off = _off(monkeypatch, slots=64, SLUICE_ROUTER_SPLIT="1", SLUICE_PIECEWISE="1")
    off.post_init(cfg)
    assert off._rs_thr == 8


def test_engine_settings_without_router_split_or_piecewise(monkeypatch):
    """Piecewise without router-split: only the MoE ops become split points
    (the classic hook runs in a graph break) and no envelope applies;
    eager: the config only contributes the speculative depth."""
    off = _off(monkeypatch, SLUICE_PIECEWISE="1")
    cfg = _cfg(mbt=4096)
    off.post_init(cfg)
    assert cfg.compilation_config.splitting_ops == ["vllm::moe_forward",
                                                    "vllm::moe_forward_shared"]
    assert off._rs_thr is None
    off = _off(monkeypatch)
    cfg = _cfg(mbt=4096, spec=3)
    off.post_init(cfg)
    assert cfg.compilation_config.splitting_ops == [] and off._spec_tokens == 3


def test_config_must_be_readable_when_vllm_is_present(monkeypatch):
    _stub_vllm(monkeypatch, cfg=None)
    off = _off(monkeypatch)
    with pytest.raises(RuntimeError, match="config is None"):
        off.post_init()


def test_split_signal_reads_the_forward_context(monkeypatch):
    ns = types.SimpleNamespace
    off = _off(monkeypatch)
    _stub_vllm(monkeypatch, ctx=ns(attn_metadata=None))
    assert off._split_signal() == (None, None, False)          # dummy / profiling run
    _stub_vllm(monkeypatch, ctx=ns(attn_metadata={"l0": ns(num_decode_tokens=None)}))
    assert off._split_signal() == (None, None, True)           # non-MLA backend
    _stub_vllm(monkeypatch, ctx=ns(attn_metadata={"l0": ns(num_decode_tokens=6,
                                                            num_decodes=5)}))
    assert off._split_signal() == (6, 5, True)
    off.set_step_signal(3, 3, True)                            # harness override
    assert off._split_signal() == (3, 3, True)
    off.clear_step_signal()
    assert off._split_signal() == (6, 5, True)


def test_apply_wrapper_routes_through_run_moe(monkeypatch):
    off = _off(monkeypatch, SLUICE_PIECEWISE="1")
    calls = []

    class QM:
        is_monolithic = False

        def apply(self, layer, x, topk_weights, topk_ids):
            calls.append("orig")
            return x

    layer = types.SimpleNamespace(quant_method=QM())
    off._install_classic_hook(layer)
    hook = layer.quant_method._sluice_hook
    off._install_classic_hook(layer)  # idempotent
    assert layer.quant_method._sluice_hook is hook

    def fake_run_moe(original_apply, args, kwargs, module, topk_ids):
        calls.append(("hook", module is layer, tuple(topk_ids.shape)))
        return original_apply(*args, **kwargs)

    monkeypatch.setattr(off, "run_moe", fake_run_moe)
    x = torch.zeros(2, 4)
    layer.quant_method.apply(layer=layer, x=x, topk_weights=x, topk_ids=torch.zeros(2, 3))
    assert calls == [("hook", True, (2, 3)), "orig"]
    calls.clear()
    layer.quant_method.apply(layer, x, x, None)  # no topk_ids keyword: straight through
    assert calls == ["orig"]


# ---------------------------------------------------------------------------
# Router settings -> routing kernel
# ---------------------------------------------------------------------------
def _moe(E=64, top_k=6, **attrs):
    m = nn.Module()
    m.global_num_experts = E
    m.local_num_experts = E
    m.top_k = top_k
    defaults = dict(scoring_func="softmax", renormalize=False, use_grouped_topk=False,
                    num_expert_group=None, topk_group=None, routed_scaling_factor=1.0,
                    custom_routing_function=None, e_score_correction_bias=None)
    defaults.update(attrs)
    for k, v in defaults.items():
        setattr(m, k, v)
    return m


def test_route_spec_maps_the_configs_routers():
    # DeepSeek-V2-Lite: softmax greedy, no renorm (vLLM runs it as grouped
    # top-k with one group)
    spec, why = route_spec(_moe(64, 6, use_grouped_topk=True, num_expert_group=1, topk_group=1))
    assert why == "" and (spec.scoring, spec.renormalize, spec.n_group, spec.scale) == (
        "softmax", False, 1, 1.0)
    # Qwen3-30B-A3B: softmax + renorm, not grouped
    spec, _ = route_spec(_moe(128, 8, renormalize=True))
    assert (spec.top_k, spec.scoring, spec.renormalize, spec.n_group) == (8, "softmax", True, 1)
    # DeepSeek-V3: sigmoid + correction bias, 8 groups / top-4 groups, renorm, scale 2.5
    bias = torch.zeros(256)
    spec, _ = route_spec(_moe(256, 8, scoring_func="sigmoid", renormalize=True,
                              use_grouped_topk=True, num_expert_group=8, topk_group=4,
                              routed_scaling_factor=2.5, e_score_correction_bias=bias))
    assert (spec.scoring, spec.n_group, spec.topk_group, spec.scale, spec.renormalize) == (
        "sigmoid", 8, 4, 2.5, True)
    assert spec.bias is bias
    # the scaling factor applies only where vLLM's grouped top-k applies it
    spec, _ = route_spec(_moe(64, 6, routed_scaling_factor=2.0))
    assert spec.scale == 1.0


def test_route_spec_prefers_the_runner_router_and_refuses_what_the_kernel_cannot_do():
    m = _moe(64, 6)
    runner = types.SimpleNamespace(router=types.SimpleNamespace(top_k=4, renormalize=True))
    spec, _ = route_spec(m, runner)
    assert spec.top_k == 4 and spec.renormalize
    refused = {
        "router:custom": _moe(custom_routing_function=lambda *a: None),
        "router:scoring-softplus": _moe(scoring_func="softplus"),
        "router:ungrouped-sigmoid-or-bias": _moe(scoring_func="sigmoid"),
        "router:sigmoid-no-bias": _moe(scoring_func="sigmoid", use_grouped_topk=True,
                                       num_expert_group=8, topk_group=4),
        "router:softmax-bias": _moe(use_grouped_topk=True, num_expert_group=8, topk_group=2,
                                    e_score_correction_bias=torch.zeros(64)),
        "router:groups": _moe(use_grouped_topk=True, num_expert_group=7, topk_group=2),
        "router:weight-on-input": _moe(apply_router_weight_on_input=True),
        "router:shape": _moe(E=2048),
    }
    for reason, m in refused.items():
        spec, why = route_spec(m)
        assert spec is None and why == reason, (reason, why)
    m = _moe()
    m.hash_indices_table = torch.zeros(64, 2)
    assert route_spec(m) == (None, "router:hash")


def test_get_stats_schema(monkeypatch):
    """The reference's keys: per class ("small", "scan") steps, hits, misses,
    bytes, waves; the gap's counters are reported apart."""
    off = _off(monkeypatch)
    st = off.get_stats()
    assert list(st) == ["small", "scan"]
    for kind in st.values():
        assert kind == {"steps": 0, "hits": 0, "misses": 0, "bytes": 0, "waves": 0}
    assert off.get_gap_stats() == {"layers": 0, "gaps": 0, "misses": 0, "fast_hits": 0,
                                   "map_writes": 0, "bytes": 0}
