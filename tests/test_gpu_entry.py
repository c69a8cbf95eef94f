"""The armed router-split entry (src/sluice/offloader.py:2578-2603) routes
with the wave64 top-k kernel, mapped from the layer's router settings under
vLLM's attribute names, not with vLLM's select_experts: the stand-in for
vLLM's select_experts here returns wrong ids and records its calls, and the
entry's slot assignment, expert map and layer output still follow the
oracle's routing of the entry's own router logits."""

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import routing as orr
from oracle.slru import LayerCache

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")

# router kinds: (E, k, scoring, renorm, scale, n_group, topk_group, e_bias)
ROUTERS = {
    "v2lite_softmax": (64, 6, "softmax", False, 1.0, 1, 1, False),
    "qwen3_softmax_renorm": (64, 8, "softmax", True, 1.0, 1, 1, False),
    "v3_sigmoid_grouped": (64, 8, "sigmoid", True, 2.5, 8, 4, True),
}


@pytest.mark.parametrize("kind", sorted(ROUTERS))
def test_entry_routes_with_the_topk_kernel(kind):
    from sluice_amd.decoder import SyntheticMoELayer, build_offloaded

    E, k, scoring, renorm, scale, n_group, topk_group, e_bias = ROUTERS[kind]
    H, I, S, T = 256, 128, 32, 4
    print(f"entry routing {kind}", flush=True)
    layer = SyntheticMoELayer(H, I, E, k, scoring=scoring, renorm=renorm, routed_scale=scale,
                              n_group=n_group, topk_group=topk_group, e_bias=e_bias, seed=5,
                              device=DEV)
    calls = []

    def vllm_select(hidden_states, router_logits, input_ids=None):
        calls.append(router_logits.shape)
        n = router_logits.shape[0]
        ids = torch.arange(k, dtype=torch.int32, device=DEV).repeat(n, 1)
        return torch.full((n, k), 1.0 / k, device=DEV), ids

    layer.runner.router.select_experts = vllm_select
    off = build_offloaded([layer], slots=S, device=DEV)
    assert off._rs_routes[0] is not None
    cache = off._caches[id(layer)]
    oracle = LayerCache(E, E, S, off.protect_frac)
    bias = None if layer.e_score_correction_bias is None else \
        layer.e_score_correction_bias.detach().float().cpu().numpy()
    rng = np.random.default_rng(11)
    for step in range(6):
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16)
        out = layer(x.to(DEV))
        torch.cuda.synchronize()
        logits = layer.last_logits.float().cpu().numpy()
        ids, w = orr.route(logits, k=k, scoring=scoring, renorm=renorm, scale=scale, bias=bias,
                           n_group=n_group, topk_group=topk_group)
        oracle.gap(ids.reshape(-1).tolist(), fast_hit=True)
        assert cache._state()["expert_in_slot"] == [
            -1 if v is None else v for v in oracle.expert_in_slot], step
        assert cache.expert_map_buf.cpu().tolist() == oracle.map, step
        ref = om.fused_experts(x.float().numpy(), layer.host_w13.float().numpy(),
                               layer.host_w2.float().numpy(), w, ids)
        err = om.rel_l2(out.float().cpu().numpy(), ref)
        print(f"  step {step} rel_l2={err:.2e}", flush=True)
        assert err <= 1e-2
    assert calls == []  # vLLM's select_experts never ran on the split path
    off.close()


def test_entry_keeps_vllm_routing_when_the_kernel_cannot_express_it():
    """A router the kernel cannot reproduce exactly (a custom routing
    function) keeps vLLM's select_experts inside the split path."""
    from sluice_amd.decoder import SyntheticMoELayer, build_offloaded

    H, I, E, k, S, T = 256, 128, 32, 4, 16, 4
    layer = SyntheticMoELayer(H, I, E, k, scoring="softmax", renorm=True, seed=6, device=DEV)
    layer.custom_routing_function = lambda *a, **kw: None
    calls = []
    select = layer.runner.router.select_experts

    def vllm_select(hidden_states, router_logits, input_ids=None):
        calls.append(1)
        return select(hidden_states=hidden_states, router_logits=router_logits,
                      input_ids=input_ids)

    layer.runner.router.select_experts = vllm_select
    off = build_offloaded([layer], slots=S, device=DEV)
    assert off._rs_routes == [None]
    x = torch.randn((T, H), device=DEV).to(torch.bfloat16)
    out = layer(x)
    torch.cuda.synchronize()
    assert calls == [1]
    ref = om.fused_experts(x.float().cpu().numpy(), layer.host_w13.float().numpy(),
                           layer.host_w2.float().numpy(), layer.last_weights.cpu().numpy(),
                           layer.last_ids.cpu().numpy())
    assert om.rel_l2(out.float().cpu().numpy(), ref) <= 1e-2
    off.close()


@pytest.mark.parametrize("kind", sorted(ROUTERS))
def test_gap_built_plan_gives_the_product_it_plans_itself(kind):
    """After each gap op (misses streaming while the product runs), the
    expert product over the plan the gap kernel built equals, bit for bit,
    the product that plans itself (its align kernel) on the same ids and map,
    shared experts folded in or not; a plan buffer too small for the call or
    of the wrong type is refused before anything is launched."""
    from sluice_amd import ops
    from sluice_amd.decoder import SyntheticMoELayer, build_offloaded

    E, k, scoring, renorm, scale, n_group, topk_group, e_bias = ROUTERS[kind]
    H, I, S, T = 256, 128, 32, 4
    print(f"gap-built plan {kind}", flush=True)
    layer = SyntheticMoELayer(H, I, E, k, scoring=scoring, renorm=renorm, routed_scale=scale,
                              n_group=n_group, topk_group=topk_group, e_bias=e_bias, seed=9,
                              device=DEV, shared_I=2 * I)
    off = build_offloaded([layer], slots=S, device=DEV)
    cache = off._caches[id(layer)]
    rng = np.random.default_rng(17)
    sh = layer.shared

    def route(x):
        logits, _ = layer.runner.gate(x)
        return layer.runner.router.select_experts(hidden_states=x, router_logits=logits)

    for step in range(6):
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(
            torch.bfloat16).to(DEV)
        tw, ti = route(x)
        h = torch.ops.vllm.sluice_stream_gap(x, ti, 0)
        plan = off.gap_plan(0, ti.numel())
        assert plan is not None
        kw = dict(global_num_experts=E, expert_map=cache.expert_map_buf)
        got = ops.fused_experts(h, layer.w13_weight, layer.w2_weight, tw, ti, plan=plan, **kw)
        want = ops.fused_experts(h, layer.w13_weight, layer.w2_weight, tw, ti, **kw)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), step
        # a copy of the map has no slots streaming: the single gemm2 launch
        # (the rows have landed: the product above waited for them)
        one = ops.fused_experts(h, layer.w13_weight, layer.w2_weight, tw, ti,
                                **dict(kw, expert_map=cache.expert_map_buf.clone()))
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), one.view(torch.int16)), step
        if sh is not None:
            kw.update(shared_w1=sh.gate_up, shared_w2=sh.down)
            got = ops.fused_experts(h, layer.w13_weight, layer.w2_weight, tw, ti, plan=plan, **kw)
            want = ops.fused_experts(h, layer.w13_weight, layer.w2_weight, tw, ti, **kw)
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), step
    x = torch.zeros((T, H), dtype=torch.bfloat16, device=DEV)
    tw, ti = route(x)
    for bad in (torch.zeros(8, dtype=torch.int32, device=DEV),
                torch.zeros(cache.plan.numel(), dtype=torch.int64, device=DEV)):
        with pytest.raises(ValueError):
            ops.fused_experts(x, layer.w13_weight, layer.w2_weight, tw, ti, plan=bad,
                              global_num_experts=E, expert_map=cache.expert_map_buf)
    off.close()


def test_fp8_split_launch_equals_single_gemm2_launch():
    """DeepSeek-V3-routed fp8 layer (shared expert folded in): after each
    gap op, the product over the layer's map -- gemm2 of the resident
    experts while the missed ones stream, their gemm1 and gemm2 handed over
    inside one launch -- equals, bit for bit, the product over a copy of the
    map, which has no streaming slots and runs one gemm2 launch after gemm1."""
    from sluice_amd.decoder import SPECS, _expert_store, _StoreMoELayer, build_offloaded

    sp = dict(SPECS["v3"], H=512, I=256, shared_I=256)
    store = _expert_store(sp, 7003, DEV, True)
    layer = _StoreMoELayer(sp, store, 1, DEV, None, "layers.1.mlp")
    off = build_offloaded([layer], slots=64, device=DEV)
    cache = off._caches[id(layer)]
    rng = np.random.default_rng(23)
    pending_blocks = 0
    for step in range(5):
        print(f"fp8 split step {step}", flush=True)
        x = torch.from_numpy(rng.standard_normal((8, 512)).astype(np.float32)).to(
            torch.bfloat16).to(DEV)
        tw, ti = layer.select(layer.logits(x))
        h = torch.ops.vllm.sluice_stream_gap(x, ti, 0)
        plan = off.gap_plan(0, ti.numel())
        assert plan is not None
        got = layer.experts(h, tw, ti, fold_shared=True, plan=plan)
        torch.cuda.synchronize()
        head = plan[:3].cpu().tolist()
        pending_blocks += head[0] - head[2]
        emap = layer._buffers["_expert_map"]
        layer._buffers["_expert_map"] = emap.clone()
        try:
            one = layer.experts(h, tw, ti, fold_shared=True)
        finally:
            layer._buffers["_expert_map"] = emap
        torch.cuda.synchronize()
        assert not torch.isnan(one.float()).any()
        assert torch.equal(got.view(torch.int16), one.view(torch.int16)), step
    assert pending_blocks > 0
    off.close()
