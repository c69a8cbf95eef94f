"""Pin the expert-product oracle against transformers' experts forward
(Qwen3MoeExperts / DeepseekV2Experts: gate rows first in gate_up_proj,
silu(gate)*up, down_proj, routing-weight multiply, index_add over tokens),
closed-form special cases, fp8 e4m3fn decode against torch, and the
align-to-block grouping."""

import numpy as np
import pytest
import torch

from oracle import moe


def _rand(shape, rng, std=1.0):
    return (rng.standard_normal(shape) * std).astype(np.float32)


@pytest.mark.parametrize("family", ["qwen3_moe", "deepseek_v2"])
def test_matches_transformers_experts(family):
    rng = np.random.default_rng(0)
    T, H, I, E, k = 5, 64, 32, 8, 3
    if family == "qwen3_moe":
        from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
        from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeExperts as X

        cfg = Qwen3MoeConfig(hidden_size=H, num_attention_heads=1, num_key_value_heads=1,
                             moe_intermediate_size=I, num_experts=E, num_experts_per_tok=k)
    else:
        from transformers.models.deepseek_v2.configuration_deepseek_v2 import DeepseekV2Config
        from transformers.models.deepseek_v2.modeling_deepseek_v2 import DeepseekV2Experts as X

        cfg = DeepseekV2Config(hidden_size=H, num_attention_heads=1, num_key_value_heads=1,
                               moe_intermediate_size=I, n_routed_experts=E,
                               num_experts_per_tok=k)
    ex = X(cfg).double()
    w13 = _rand((E, 2 * I, H), rng, 0.1)
    w2 = _rand((E, H, I), rng, 0.1)
    with torch.no_grad():
        ex.gate_up_proj.copy_(torch.from_numpy(w13))
        ex.down_proj.copy_(torch.from_numpy(w2))
    x = _rand((T, H), rng)
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    tw = rng.random((T, k)).astype(np.float32)
    with torch.no_grad():
        ref = ex(torch.from_numpy(x).double(), torch.from_numpy(ids),
                 torch.from_numpy(tw).double())
    got = moe.fused_experts(x, w13, w2, tw, ids)
    assert moe.rel_l2(got, ref.numpy()) < 1e-12


def test_shared_mlp_matches_transformers_mlp():
    """The shared-expert oracle against DeepseekV2MLP (gate_proj, up_proj,
    down_proj, silu) in float64, and against the expert oracle with the MLP
    as one expert of weight 1; splitting its channels into groups sums to it."""
    from transformers.models.deepseek_v2.configuration_deepseek_v2 import DeepseekV2Config
    from transformers.models.deepseek_v2.modeling_deepseek_v2 import DeepseekV2MLP

    rng = np.random.default_rng(7)
    T, H, Is = 5, 64, 96
    cfg = DeepseekV2Config(hidden_size=H, intermediate_size=Is, num_attention_heads=1,
                           num_key_value_heads=1)
    mlp = DeepseekV2MLP(cfg, intermediate_size=Is).double()
    gu = _rand((2 * Is, H), rng, 0.1)
    d = _rand((H, Is), rng, 0.1)
    with torch.no_grad():
        mlp.gate_proj.weight.copy_(torch.from_numpy(gu[:Is]))
        mlp.up_proj.weight.copy_(torch.from_numpy(gu[Is:]))
        mlp.down_proj.weight.copy_(torch.from_numpy(d))
    x = _rand((T, H), rng)
    with torch.no_grad():
        ref = mlp(torch.from_numpy(x).double()).numpy()
    got = moe.shared_mlp(x, gu, d)
    assert moe.rel_l2(got, ref) < 1e-12
    one = moe.fused_experts(x, gu[None], d[None], np.ones((T, 1)), np.zeros((T, 1), np.int64))
    assert moe.rel_l2(one, ref) < 1e-12
    # three groups of 32 channels, each one expert of intermediate 32
    I = 32
    w13 = np.stack([np.concatenate([gu[v * I:(v + 1) * I], gu[Is + v * I:Is + (v + 1) * I]])
                    for v in range(3)])
    w2 = np.stack([d[:, v * I:(v + 1) * I] for v in range(3)])
    grouped = moe.fused_experts(x, w13, w2, np.ones((T, 3)), np.tile(np.arange(3), (T, 1)))
    assert moe.rel_l2(grouped, ref) < 1e-12


def test_expert_map_slots_and_unmapped_contribute_zero():
    rng = np.random.default_rng(1)
    T, H, I, E, S, k = 4, 32, 16, 10, 4, 2
    full13 = _rand((E, 2 * I, H), rng, 0.1)
    full2 = _rand((E, H, I), rng, 0.1)
    emap = np.full(E, -1)
    resident = [7, 2, 9, 4]
    slots13 = np.zeros((S, 2 * I, H), np.float32)
    slots2 = np.zeros((S, H, I), np.float32)
    for s, g in enumerate(resident):
        emap[g] = s
        slots13[s], slots2[s] = full13[g], full2[g]
    x = _rand((T, H), rng)
    ids = np.array([[7, 2], [9, 0], [3, 1], [4, 4]])
    tw = rng.random((T, k)).astype(np.float32)
    got = moe.fused_experts(x, slots13, slots2, tw, ids, expert_map=emap)
    # same as the unmapped full computation with non-resident pairs' weight zeroed
    tw0 = tw.copy()
    for t in range(T):
        for j in range(k):
            if emap[ids[t, j]] < 0:
                tw0[t, j] = 0
    ref = moe.fused_experts(x, full13, full2, tw0, ids)
    assert moe.rel_l2(got, ref) < 1e-12
    assert np.all(got[2] == 0)  # both of token 2's experts are absent


def test_closed_form_single_expert():
    # one expert, I=1, H=1: out = w * w2 * silu(a x) * (b x)
    x = np.array([[0.75]], np.float32)
    w13 = np.array([[[1.5], [-2.0]]], np.float32)
    w2 = np.array([[[3.0]]], np.float32)
    got = moe.fused_experts(x, w13, w2, np.array([[0.25]]), np.array([[0]]))
    g, u = 1.5 * 0.75, -2.0 * 0.75
    assert got[0, 0] == pytest.approx(0.25 * 3.0 * (g / (1 + np.exp(-g))) * u, rel=1e-12)


def test_scale_and_shared():
    rng = np.random.default_rng(2)
    x = _rand((2, 32), rng)
    w13 = _rand((3, 32, 32), rng, 0.1)
    w2 = _rand((3, 32, 16), rng, 0.1)
    ids = np.array([[0, 1], [2, 0]])
    tw = np.ones((2, 2), np.float32)
    sh = _rand((2, 32), rng)
    base = moe.fused_experts(x, w13, w2, tw, ids)
    got = moe.fused_experts(x, w13, w2, tw, ids, scale=2.5, shared=sh)
    assert np.allclose(got, 2.5 * base + sh)


def test_fp8_table_matches_torch_e4m3fn():
    b = torch.arange(256, dtype=torch.uint8)
    ref = b.view(torch.float8_e4m3fn).float().numpy()
    got = moe.fp8_e4m3fn_to_f32(np.arange(256))
    finite = ~np.isnan(ref)
    assert np.array_equal(got[finite], ref[finite])
    assert np.array_equal(np.isnan(got), np.isnan(ref))


def test_block_dequant():
    rng = np.random.default_rng(3)
    q = rng.integers(0, 126, size=(256, 384), dtype=np.uint8)
    sc = rng.random((2, 3)).astype(np.float32)
    w = moe.dequant_block(q, sc)
    assert w[5, 7] == moe.fp8_e4m3fn_to_f32(q[5, 7]) * sc[0, 0]
    assert w[200, 300] == moe.fp8_e4m3fn_to_f32(q[200, 300]) * sc[1, 2]


def test_bf16_round_trip():
    x = np.array([1.0, -2.5, 3.14159, 1e-3, 65504.0], np.float32)
    b = moe.f32_to_bf16(x)
    ref = torch.from_numpy(x).bfloat16().view(torch.uint16).numpy()
    assert np.array_equal(b, ref)
    assert np.array_equal(moe.bf16_to_f32(b), torch.from_numpy(x).bfloat16().float().numpy())


def test_align_blocks():
    emap = np.array([3, -1, 0, 1, 2, -1])
    ids = np.array([[0, 2], [2, 1], [0, 5], [4, 2]])
    blocks, valid = moe.align_blocks(ids, emap, S=4, block_m=2)
    assert valid == [1, 1, 1, 0, 1, 0, 1, 1]
    # slot 0 <- expert 2 (pairs 1, 2, 7), slot 2 <- expert 4 (pair 6), slot 3 <- expert 0 (0, 4)
    assert blocks == [(0, [1, 2]), (0, [7]), (2, [6]), (3, [0, 4])]
