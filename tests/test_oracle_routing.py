"""Pin the routing oracle: transformers' routers (DeepSeek-V2 greedy /
group_limited_greedy, Qwen3-MoE softmax+renorm, DeepSeek-V3 sigmoid
group-limited) on tie-free logits, brute force over all k-subsets for tiny
E, and the tie rule on constructed ties."""

import itertools

import numpy as np
import pytest
import torch

from oracle.routing import sigmoid_fp32, sigmoid_topk, softmax_topk


def _logits(T, E, seed, scale=2.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((T, E)) * scale).astype(np.float32)


def _route_with(router, logits):
    """Drive a transformers router so that its router_logits == logits:
    hidden = I_T, weight = logits^T."""
    T, E = logits.shape
    with torch.no_grad():
        router.weight.copy_(torch.from_numpy(logits.T.copy()))
        out = router(torch.eye(T, dtype=torch.float32))
    _, w, ids = out
    return w.numpy(), ids.numpy()


def _same_sets(ids_a, w_a, ids_b, w_b, rtol=2e-6):
    for t in range(ids_a.shape[0]):
        da = dict(zip(ids_a[t].tolist(), w_a[t].tolist()))
        db = dict(zip(ids_b[t].tolist(), w_b[t].tolist()))
        assert set(da) == set(db), t
        for e in da:
            assert da[e] == pytest.approx(db[e], rel=rtol, abs=1e-9), (t, e)


@pytest.mark.parametrize("E,k,seed", [(64, 6, 0), (160, 6, 1)])
def test_softmax_greedy_matches_deepseek_v2(E, k, seed):
    from transformers.models.deepseek_v2.configuration_deepseek_v2 import DeepseekV2Config
    from transformers.models.deepseek_v2.modeling_deepseek_v2 import DeepseekV2TopkRouter

    T = 16
    cfg = DeepseekV2Config(hidden_size=T, num_attention_heads=1, num_key_value_heads=1,
                           n_routed_experts=E, num_experts_per_tok=k,
                           topk_method="greedy", routed_scaling_factor=1.0, n_group=1,
                           topk_group=1)
    L = _logits(T, E, seed)
    w_hf, ids_hf = _route_with(DeepseekV2TopkRouter(cfg), L)
    ids, w = softmax_topk(L, k, renorm=False, scale=1.0)
    _same_sets(ids, w, ids_hf, w_hf)


def test_softmax_group_limited_matches_deepseek_v2():
    from transformers.models.deepseek_v2.configuration_deepseek_v2 import DeepseekV2Config
    from transformers.models.deepseek_v2.modeling_deepseek_v2 import DeepseekV2TopkRouter

    T, E, k = 16, 160, 6
    cfg = DeepseekV2Config(hidden_size=T, num_attention_heads=1, num_key_value_heads=1,
                           n_routed_experts=E, num_experts_per_tok=k,
                           topk_method="group_limited_greedy", routed_scaling_factor=16.0,
                           n_group=8, topk_group=3)
    L = _logits(T, E, 7)
    w_hf, ids_hf = _route_with(DeepseekV2TopkRouter(cfg), L)
    ids, w = softmax_topk(L, k, renorm=False, scale=16.0, n_group=8, topk_group=3)
    _same_sets(ids, w, ids_hf, w_hf)


def test_softmax_renorm_matches_qwen3_moe():
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeTopKRouter

    T, E, k = 16, 128, 8
    cfg = Qwen3MoeConfig(hidden_size=T, num_attention_heads=1, num_key_value_heads=1,
                         num_experts=E, num_experts_per_tok=k,
                         norm_topk_prob=True)
    L = _logits(T, E, 3)
    w_hf, ids_hf = _route_with(Qwen3MoeTopKRouter(cfg), L)
    ids, w = softmax_topk(L, k, renorm=True)
    _same_sets(ids, w, ids_hf, w_hf, rtol=1e-6)


def test_sigmoid_group_limited_matches_deepseek_v3():
    from transformers.models.deepseek_v3.configuration_deepseek_v3 import DeepseekV3Config
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3TopkRouter

    T, E, k = 16, 256, 8
    cfg = DeepseekV3Config(hidden_size=T, num_attention_heads=1, num_key_value_heads=1,
                           n_routed_experts=E, num_experts_per_tok=k, n_group=8,
                           topk_group=4, norm_topk_prob=True, routed_scaling_factor=2.5)
    router = DeepseekV3TopkRouter(cfg)
    rng = np.random.default_rng(5)
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32)
    router.e_score_correction_bias.copy_(torch.from_numpy(bias))
    L = _logits(T, E, 5)
    w_hf, ids_hf = _route_with(router, L)
    ids, w = sigmoid_topk(L, bias, k, n_group=8, topk_group=4, renorm=True, scale=2.5)
    _same_sets(ids, w, ids_hf, w_hf, rtol=1e-6)


@pytest.mark.parametrize("seed", range(5))
def test_brute_force_tiny(seed):
    rng = np.random.default_rng(seed)
    E, k = 7, 3
    L = rng.integers(-3, 4, size=(6, E)).astype(np.float32)  # many ties
    ids, _ = softmax_topk(L, k)
    for t in range(L.shape[0]):
        # best subset: maximise the sorted key vector, then prefer lower ids
        best = min(itertools.combinations(range(E), k),
                   key=lambda c: (sorted((-L[t, e] for e in c)), sorted(c)))
        assert sorted(ids[t].tolist()) == sorted(best)
        # order: key descending, id ascending on ties
        keys = [(-L[t, e], e) for e in ids[t]]
        assert keys == sorted(keys)


def test_tie_rule_lower_id_wins():
    L = np.zeros((1, 64), dtype=np.float32)
    ids, w = softmax_topk(L, 6)
    assert ids[0].tolist() == [0, 1, 2, 3, 4, 5]
    assert np.allclose(w, 1 / 64)
    L[0, 40] = 1.0
    L[0, 50] = 1.0
    ids, _ = softmax_topk(L, 3)
    assert ids[0].tolist() == [40, 50, 0]


def test_sigmoid_fp32_is_rounded_fp64():
    x = np.array([0.0, 1.0, -1.0, 20.0, -20.0, 1e-8], dtype=np.float32)
    s = sigmoid_fp32(x)
    ref = np.array([1 / (1 + np.exp(-float(v))) for v in x]).astype(np.float32)
    assert np.array_equal(s, ref)
    assert s[0] == np.float32(0.5)
