"""The vLLM-facing surface on the CPU, against stand-in vLLM modules: the
general_plugins hook (src/sluice/plugin.py:27-96), the engine-configuration
guards and envelope (src/sluice/offloader.py:663-851), the wrapped
quant_method.apply (1085-1119) and the forward-context split signal
(1766-1800)."""

import logging
import sys
import types

import pytest
import torch

from sluice_amd import plugin
from sluice_amd.offloader import ExpertStreamOffloader


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
    cfg = ns(parallel_config=ns(data_parallel_size=kw.get("dp", 1),
                                enable_eplb=kw.get("eplb", False)),
             model_config=ns(enforce_eager=kw.get("eager", False),
                             hf_config=ns(num_experts_per_tok=kw.get("topk", 6))),
             compilation_config=ns(cudagraph_mode=ns(name=kw.get("cg", "PIECEWISE")),
                                   splitting_ops=list(kw.get("ops", []))),
             scheduler_config=ns(max_num_batched_tokens=kw.get("mbt", 8)),
             speculative_config=(ns(num_speculative_tokens=kw["spec"]) if "spec" in kw
                                 else None))
    return cfg


def _off(monkeypatch, slots=48, **env):
    for k in ("SLUICE_ROUTER_SPLIT", "SLUICE_PIECEWISE", "SLUICE_GRAPH"):
        monkeypatch.delenv(k, raising=False)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    return ExpertStreamOffloader(expert_cache_slots=slots)


def test_router_split_envelope_and_split_points(monkeypatch):
    off = _off(monkeypatch, SLUICE_ROUTER_SPLIT="1", SLUICE_PIECEWISE="1")
    cfg = _cfg(mbt=8, ops=["vllm::unified_attention"], spec=2)
    off._check_config(cfg)
    assert off._rs_thr == 8                       # 48 slots // top-6
    assert cfg.compilation_config.splitting_ops == [
        "vllm::unified_attention", "vllm::moe_forward", "vllm::moe_forward_shared",
        "vllm::sluice_stream_gap"]
    assert off._spec_tokens == 2
    with pytest.raises(RuntimeError, match="max_num_batched_tokens=9 > slots//topk=8"):
        off._check_config(_cfg(mbt=9))
    # Qwen3-style config: top-k under text_config
    cfg = _cfg(mbt=8)
    cfg.model_config.hf_config = types.SimpleNamespace(
        text_config=types.SimpleNamespace(num_experts_per_tok=8))
    off = _off(monkeypatch, slots=64, SLUICE_ROUTER_SPLIT="1", SLUICE_PIECEWISE="1")
    off._check_config(cfg)
    assert off._rs_thr == 8


def test_engine_guards(monkeypatch):
    off = _off(monkeypatch)
    with pytest.raises(RuntimeError, match="--enforce-eager"):
        off._check_config(_cfg(eager=False, cg="NONE"))
    with pytest.raises(RuntimeError, match="frozen expert map"):
        off._check_config(_cfg(eager=True, cg="PIECEWISE"))
    off._check_config(_cfg(eager=True, cg="NONE"))       # eager, no graphs: fine
    with pytest.raises(RuntimeError, match="data parallelism"):
        off._check_config(_cfg(eager=True, cg="NONE", dp=2))
    with pytest.raises(RuntimeError, match="EPLB"):
        off._check_config(_cfg(eager=True, cg="NONE", eplb=True))
    off = _off(monkeypatch, SLUICE_PIECEWISE="1")
    with pytest.raises(RuntimeError, match="requires PIECEWISE cudagraph"):
        off._check_config(_cfg(cg="FULL_AND_PIECEWISE"))
    cfg = _cfg(cg="PIECEWISE")
    off._check_config(cfg)                                # piecewise relaxes eager
    assert "vllm::sluice_stream_gap" not in cfg.compilation_config.splitting_ops
    off = _off(monkeypatch, SLUICE_GRAPH="1")
    off._check_config(_cfg(cg="FULL"))                    # graph mode: checked at post_init


def test_config_must_be_readable_when_vllm_is_present(monkeypatch):
    _stub_vllm(monkeypatch, cfg=None)
    off = _off(monkeypatch)
    with pytest.raises(RuntimeError, match="config is None"):
        off._check_config()


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
    off._wrap_apply(layer)
    off._wrap_apply(layer)  # idempotent
    assert layer.quant_method._sluice_wrapped

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
