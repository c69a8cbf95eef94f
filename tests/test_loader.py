"""Expert host-store builder: a Hugging Face safetensors checkpoint's expert
rows land in the slot layout bit for bit (bf16 and block-quantised fp8, all
experts or an EP rank's subset, shards across files), and the offloader's
per-expert parameter filter keeps shared tensors out of the slot buffers."""

import os
import time
import types

import pytest
import torch
import torch.nn as nn
from safetensors.torch import save_file

from sluice_amd import loader

KEY = "model.layers.{layer}.mlp.experts.{e}.{proj}.{kind}"


def _write_ckpt(d, layers, E, I, H, fp8=False, shards=2, seed=0):
    g = torch.Generator().manual_seed(seed)
    want = {}
    tensors = [dict() for _ in range(shards)]
    n = 0
    for L in layers:
        tensors[n % shards][f"model.layers.{L}.mlp.gate.weight"] = torch.randn((E, H), generator=g)
        for e in range(E):
            for proj, shp in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
                w = torch.randn(shp, generator=g)
                name = KEY.format(layer=L, e=e, proj=proj, kind="weight")
                if fp8:
                    wq = (w * 16).to(torch.float8_e4m3fn)
                    sc = torch.rand(((shp[0] + 127) // 128, (shp[1] + 127) // 128),
                                    generator=g) + 0.5
                    tensors[n % shards][name] = wq
                    sname = KEY.format(layer=L, e=e, proj=proj, kind="weight_scale_inv")
                    tensors[n % shards][sname] = sc
                    want[sname] = sc
                    want[name] = wq
                else:
                    tensors[n % shards][name] = w.to(torch.bfloat16)
                    want[name] = tensors[n % shards][name]
                n += 1
    for i, t in enumerate(tensors):
        save_file(t, os.path.join(d, f"model-{i:05d}.safetensors"))
    return want


def _rows(want, L, e, proj, kind="weight"):
    return want[KEY.format(layer=L, e=e, proj=proj, kind=kind)]


def test_bf16_checkpoint_into_slot_layout(tmp_path):
    E, I, H = 4, 64, 128
    want = _write_ckpt(str(tmp_path), [0, 1], E, I, H)
    st = loader.expert_stores_from_checkpoint(str(tmp_path), 1, pinned=False)
    w13, w2 = st["w13_weight"].tensor, st["w2_weight"].tensor
    assert w13.shape == (E, 2 * I, H) and w2.shape == (E, H, I) and w13.dtype == torch.bfloat16
    for e in range(E):
        assert torch.equal(w13[e, :I], _rows(want, 1, e, "gate_proj"))
        assert torch.equal(w13[e, I:], _rows(want, 1, e, "up_proj"))
        assert torch.equal(w2[e], _rows(want, 1, e, "down_proj"))


def test_fp8_checkpoint_with_block_scales(tmp_path):
    E, I, H = 3, 256, 320   # H not a multiple of 128: ceil-divided scale blocks
    want = _write_ckpt(str(tmp_path), [2], E, I, H, fp8=True, shards=3)
    ck = loader.Checkpoint(str(tmp_path))
    assert loader.expert_layout(ck, 2) == (E, I, H, True)
    shapes = loader.store_shapes(E, I, H, True)
    assert shapes["w13_weight_scale"][0] == (E, 4, 3) and shapes["w2_weight_scale"][0] == (E, 3, 2)
    with pytest.raises(ValueError):  # a scale block would straddle gate and up rows
        loader.store_shapes(E, 192, H, True)
    stores = {n: torch.empty(s, dtype=dt) for n, (s, dt) in shapes.items()}
    nbytes = loader.load_experts(ck, 2, stores)
    assert nbytes == sum(t.numel() * t.element_size() for t in stores.values())
    for e in range(E):
        assert torch.equal(stores["w13_weight"][e, :I].view(torch.uint8),
                           _rows(want, 2, e, "gate_proj").view(torch.uint8))
        assert torch.equal(stores["w13_weight"][e, I:].view(torch.uint8),
                           _rows(want, 2, e, "up_proj").view(torch.uint8))
        assert torch.equal(stores["w13_weight_scale"][e, :2],
                           _rows(want, 2, e, "gate_proj", "weight_scale_inv"))
        assert torch.equal(stores["w13_weight_scale"][e, 2:],
                           _rows(want, 2, e, "up_proj", "weight_scale_inv"))
        assert torch.equal(stores["w2_weight_scale"][e],
                           _rows(want, 2, e, "down_proj", "weight_scale_inv"))
    ck.close()


def test_ep_subset_and_errors(tmp_path):
    E, I, H = 6, 64, 64
    want = _write_ckpt(str(tmp_path), [0], E, I, H, shards=1)
    ck = loader.Checkpoint(str(tmp_path))
    shapes = loader.store_shapes(2, I, H, False)
    stores = {n: torch.empty(s, dtype=dt) for n, (s, dt) in shapes.items()}
    loader.load_experts(ck, 0, stores, experts=[1, 4])   # an EP rank owning experts 1 and 4
    assert torch.equal(stores["w2_weight"][1], _rows(want, 0, 4, "down_proj"))
    with pytest.raises(ValueError):
        loader.load_experts(ck, 0, stores, experts=[1])
    with pytest.raises(KeyError):
        loader.load_experts(ck, 0, stores, experts=[1, 9])
    bad = {n: torch.empty(s, dtype=dt) for n, (s, dt) in loader.store_shapes(2, I, 2 * H,
                                                                             False).items()}
    with pytest.raises(ValueError):
        loader.load_experts(ck, 0, bad, experts=[0, 1])
    with pytest.raises(KeyError):
        loader.expert_layout(ck, 5)
    ck.close()


def test_load_throughput_page_cache(tmp_path):
    """~200 MB of expert rows from the page cache into the slot layout; the
    rate is printed (host memory bandwidth bound), not asserted."""
    E, I, H = 16, 768, 2048
    _write_ckpt(str(tmp_path), [0], E, I, H, shards=2)
    ck = loader.Checkpoint(str(tmp_path))
    shapes = loader.store_shapes(E, I, H, False)
    stores = {n: torch.empty(s, dtype=dt) for n, (s, dt) in shapes.items()}
    loader.load_experts(ck, 0, stores)  # warm the page cache
    t0 = time.perf_counter()
    nb = loader.load_experts(ck, 0, stores, threads=8)
    dt = time.perf_counter() - t0
    print(f"loaded {nb / 1e6:.0f} MB in {dt * 1e3:.1f} ms = {nb / dt / 1e9:.2f} GB/s")
    assert nb == E * 3 * I * H * 2
    ck.close()


def test_per_expert_param_filter_keeps_shared_tensors_out():
    """NON_EXPERT_WEIGHTS (src/sluice/offloader.py:89-96): tensors with a
    leading dim equal to local_n that are NOT per-expert stay resident."""
    from sluice_amd.offloader import _streamed_params

    E = 8
    m = nn.Module()
    m.w13_weight = nn.Parameter(torch.zeros(E, 4, 2), requires_grad=False)
    m.w2_weight = nn.Parameter(torch.zeros(E, 2, 2), requires_grad=False)
    m.w13_weight_scale = nn.Parameter(torch.zeros(E, 1, 1), requires_grad=False)
    m.e_score_correction_bias = nn.Parameter(torch.zeros(E), requires_grad=False)
    m.w13_input_scale = nn.Parameter(torch.zeros(E), requires_grad=False)
    m.hash_indices_table = nn.Parameter(torch.zeros(E, 3), requires_grad=False)
    m.other = nn.Parameter(torch.zeros(E + 1), requires_grad=False)
    got = _streamed_params(m, E)
    assert sorted(got) == ["w13_weight", "w13_weight_scale", "w2_weight"]
