"""a1 routing kernel vs the oracle: ids bit-exact (same order), weights to
1e-5 relative, over the model shapes, ties and both logit dtypes."""

import numpy as np
import pytest
import torch

from oracle.routing import route

pytestmark = pytest.mark.gpu

CASES = [
    # T, E, k, scoring, renorm, scale, n_group, topk_group, dtype, bias
    (1, 64, 6, "softmax", False, 1.0, 1, 1, torch.bfloat16, False),    # V2-Lite c=1
    (8, 64, 6, "softmax", False, 1.0, 1, 1, torch.bfloat16, False),    # V2-Lite c=8
    (12, 128, 8, "softmax", True, 1.0, 1, 1, torch.bfloat16, False),   # Qwen3 c=12
    (8, 128, 8, "softmax", True, 1.0, 1, 1, torch.float32, False),
    (8, 256, 8, "sigmoid", True, 2.5, 8, 4, torch.float32, True),      # V3
    (8, 256, 8, "sigmoid", True, 2.5, 8, 4, torch.bfloat16, True),
    (16, 160, 6, "softmax", False, 16.0, 8, 3, torch.float32, False),  # V2 group-limited
    (8, 8, 2, "softmax", True, 1.0, 1, 1, torch.bfloat16, False),      # Mixtral top-2
    (8, 64, 8, "softmax", False, 1.0, 1, 1, torch.bfloat16, False),    # OLMoE
    (8, 60, 4, "softmax", False, 1.0, 1, 1, torch.bfloat16, False),    # Qwen1.5-MoE
    (64, 1024, 16, "softmax", True, 1.0, 1, 1, torch.float32, False),  # limits
    (5, 100, 7, "sigmoid", False, 1.0, 1, 1, torch.float32, True),     # ragged E
    (512, 64, 6, "softmax", False, 1.0, 1, 1, torch.bfloat16, False),  # a prompt chunk
    (8, 16, 1, "softmax", True, 1.0, 1, 1, torch.float32, False),      # top-1
    (4, 8, 8, "softmax", True, 1.0, 1, 1, torch.bfloat16, False),      # k == E
    (8, 256, 8, "sigmoid", True, 2.5, 8, 8, torch.float32, True),      # every group kept
]


def _run(T, E, k, scoring, renorm, scale, ng, tg, dtype, use_bias, logits32, bias):
    from sluice_amd import ops

    dev = torch.device("cuda:0")
    lg = torch.from_numpy(logits32).to(dev).to(dtype)
    b = torch.from_numpy(bias).to(dev) if use_bias else None
    w, ids = ops.select_experts(lg, k, scoring=scoring, renormalize=renorm,
                                routed_scaling_factor=scale, e_score_correction_bias=b,
                                num_expert_group=ng, topk_group=tg)
    torch.cuda.synchronize()
    exact = lg.float().cpu().numpy()  # the values the kernel saw
    rid, rw = route(exact, k=k, scoring=scoring, renorm=renorm, scale=scale,
                    bias=bias if use_bias else None, n_group=ng, topk_group=tg)
    return ids.cpu().numpy(), w.cpu().numpy(), rid, rw


@pytest.mark.parametrize("case", CASES, ids=[f"T{c[0]}E{c[1]}k{c[2]}{c[3]}g{c[6]}x{c[7]}{str(c[8])[6:]}" for c in CASES])
@pytest.mark.parametrize("seed", [0, 1])
def test_routing_bit_exact(case, seed):
    T, E, k, scoring, renorm, scale, ng, tg, dtype, use_bias = case
    rng = np.random.default_rng(100 + seed)
    logits = (rng.standard_normal((T, E)) * 1.5).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32)
    ids, w, rid, rw = _run(T, E, k, scoring, renorm, scale, ng, tg, dtype, use_bias, logits, bias)
    print(f"routing case {case} seed {seed}", flush=True)
    assert np.array_equal(ids, rid)
    np.testing.assert_allclose(w, rw, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("scoring", ["softmax", "sigmoid"])
def test_routing_ties(scoring):
    # few distinct values -> ties everywhere; lower id must win on both sides
    rng = np.random.default_rng(7)
    T, E, k = 12, 128, 8
    logits = rng.integers(-2, 3, size=(T, E)).astype(np.float32)
    logits[0] = 0.0
    bias = np.zeros(E, np.float32)
    ids, w, rid, rw = _run(T, E, k, scoring, True, 1.0, 1, 1, torch.float32,
                           scoring == "sigmoid", logits, bias)
    assert np.array_equal(ids, rid)
    assert ids[0].tolist() == list(range(k))
    np.testing.assert_allclose(w, rw, rtol=1e-5, atol=1e-7)


def test_routing_empty_batch():
    from sluice_amd import ops

    lg = torch.zeros((0, 64), device="cuda:0")
    w, ids = ops.select_experts(lg, 6)
    assert ids.shape == (0, 6) and w.shape == (0, 6)


def test_routing_half_logits_route_as_float32():
    # fp16 logits are widened to fp32 before the kernel: the same ids and
    # weights as the fp32 logits of the same values
    rng = np.random.default_rng(11)
    T, E, k = 8, 64, 6
    logits = (rng.standard_normal((T, E)) * 1.5).astype(np.float16).astype(np.float32)
    bias = np.zeros(E, np.float32)
    ids, w, rid, rw = _run(T, E, k, "softmax", False, 1.0, 1, 1, torch.float16, False,
                           logits, bias)
    assert np.array_equal(ids, rid)
    np.testing.assert_allclose(w, rw, rtol=1e-5, atol=1e-7)
