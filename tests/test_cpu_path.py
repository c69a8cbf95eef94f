"""The timed CPU baseline (oracle/cpu_path.py: the reference's per-layer
decode path in torch fp32) computes the path: its routing equals the
oracle's closed form, its slot buffers hold the experts the gap assigned,
and its layer output matches the float64 oracle product plus the shared
experts to fp32 rounding."""

import numpy as np
import torch

from oracle import moe as om
from oracle import routing as orr
from oracle.cpu_path import STAGES, CpuMoELayer, LayerShape, StepTimes, run


def test_cpu_path_matches_the_oracle():
    torch.set_num_threads(4)
    shape = LayerShape(H=256, E=16, I=128, k=4, shared_I=256, slots=8)
    layer = CpuMoELayer(shape, seed=3)
    g = torch.Generator().manual_seed(9)
    times = StepTimes()
    for step in range(12):
        x = torch.randn((4, shape.H), generator=g)
        out, ids, w = layer.step(x, times)
        logits = (x @ layer.gate.T + layer.bias).numpy()
        want_ids, want_w = orr.softmax_topk(logits, shape.k, renorm=False)
        assert np.array_equal(ids.numpy(), want_ids), step
        np.testing.assert_allclose(w.numpy(), want_w, rtol=1e-5)
        for s, loc in enumerate(layer.cache.expert_in_slot):
            if loc is not None:
                assert torch.equal(layer.slot13[s], layer.w13[loc])
                assert torch.equal(layer.slot2[s], layer.w2[loc])
        ref = om.fused_experts(x.numpy(), layer.w13.numpy(), layer.w2.numpy(), want_w, want_ids,
                               shared=om.shared_mlp(x.numpy(), layer.shared_gu.numpy(),
                                                    layer.shared_down.numpy()))
        assert om.rel_l2(out.numpy(), ref) <= 1e-5, step
    assert times.steps == 12 and times.misses > 0
    assert set(times.medians_us()) == set(STAGES)


def test_run_reports_stages_threads_and_cores(monkeypatch):
    import oracle.cpu_path as cp

    small = LayerShape(H=128, E=8, I=64, k=2, shared_I=128, slots=4)
    monkeypatch.setattr(cp, "CpuMoELayer", lambda seed=1: CpuMoELayer(small, seed=seed))
    r = run(T=4, steps=5, warmup=1, budget_s=5.0, threads=2)
    assert r["steps"] == 5 and r["threads"] == 2 and r["affinity"] >= 1
    assert set(r["stages_us"]) == set(STAGES) and r["step_median_s"] > 0
