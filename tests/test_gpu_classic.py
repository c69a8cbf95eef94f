"""The classic (wave) path on the GPU: steps above the router-split envelope
run through the wrapped ``quant_method.apply`` (run_moe / _run_waves).

  * the reference's golden traces (gap steps interleaved with classic
    steps) replay bit for bit: the map each wave's kernel reads, the state
    after every step, and the rows each wave's kernel sees in its slots --
    so a wave never runs before its copies land, and a copy never lands
    before the kernel that last read its slot has finished;
  * a multi-wave layer's output equals the dense oracle's;
  * the decoder above the envelope (captured pieces around the eager hook)
    decodes the same tokens as eager steps, and a decoder that alternates
    gap-sized and classic-sized batches keeps the gap's map consistent."""

import numpy as np
import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


class _RecordingMethod:
    """quant_method stand-in whose apply records, at kernel time (enqueued
    on the stream), the expert map and the marker element of every slot."""

    is_monolithic = False

    def __init__(self):
        self.maps, self.markers = [], []

    def apply(self, layer, x, topk_weights, topk_ids):
        self.maps.append(layer._expert_map.clone())
        self.markers.append(layer.w13_weight[:, 0, 0].clone())
        return torch.zeros_like(x)


class _Layer(nn.Module):
    """FusedMoE-shaped layer whose expert l has w13[l, 0, 0] == l."""

    def __init__(self, E, local_n, H=64, I=32, expert_map=None):
        super().__init__()
        self.global_num_experts = E
        self.local_num_experts = local_n
        self.quant_method = _RecordingMethod()
        g = torch.Generator().manual_seed(E * 1000 + local_n)
        w13 = torch.randn((local_n, 2 * I, H), generator=g)
        w13[:, 0, 0] = torch.arange(local_n, dtype=torch.float32)
        self.w13_weight = nn.Parameter(w13.to(torch.bfloat16), requires_grad=False)
        self.w2_weight = nn.Parameter(
            torch.randn((local_n, H, I), generator=g).to(torch.bfloat16), requires_grad=False)
        if expert_map is not None:
            self.register_buffer("_orig_map", expert_map)

    @property
    def expert_map(self):
        if "_expert_map" in self._buffers:
            return self._buffers["_expert_map"]
        return self._buffers.get("_orig_map")


def _offloader(monkeypatch, slots, frac):
    monkeypatch.setenv("SLUICE_ROUTER_SPLIT", "1")
    monkeypatch.setenv("SLUICE_PROTECT_FRAC", str(frac))
    monkeypatch.setenv("SLUICE_RS_FAST_HIT", "1")
    from sluice_amd.offloader import ExpertStreamOffloader

    return ExpertStreamOffloader(expert_cache_slots=slots)


def _check_slots(cache):
    torch.cuda.synchronize()
    for name in cache.param_names:
        slot_t = cache.gpu_cache[name].cpu()
        host_t = cache.cpu_store[name]
        for s, loc in enumerate(cache.expert_in_slot):
            if loc is not None:
                assert torch.equal(slot_t[s].view(torch.int16), host_t[loc].view(torch.int16)), (
                    name, s, loc)


def _classic_cases():
    from conftest import classic_vectors

    return classic_vectors()["cases"]


@pytest.mark.parametrize("case", _classic_cases(), ids=lambda c: c["name"])
def test_device_classic_replays_reference(monkeypatch, tmp_path, case):
    import json

    print(f"classic case {case['name']}", flush=True)
    E, local_n, k = case["E"], case["local_n"], case["k"]
    emap = None
    if case["local_of"] is not None:
        emap = torch.tensor(case["local_of"], dtype=torch.int32)
    layer = _Layer(E, local_n, expert_map=emap)
    qm = layer.quant_method
    pol = case.get("policy", {})
    if pol.get("lfu"):
        monkeypatch.setenv("SLUICE_LFU", "1")
    if pol.get("counts_every"):
        monkeypatch.setenv("SLUICE_EXPERT_COUNTS", str(tmp_path))
        monkeypatch.setenv("SLUICE_EXPERT_COUNTS_EVERY", str(pol["counts_every"]))
    off = _offloader(monkeypatch, case["slots"], case["protect_frac"])
    if case["pins"]:
        off._pin_layers = {0: list(case["pins"])}  # what SLUICE_PIN_FILE would hold
    off.wrap_modules(iter([layer]))
    with torch.cuda.device(DEV):
        off.post_init()
    cache = off._caches[id(layer)]
    off._rs_caches.append(cache)
    lof = case["local_of"] or list(range(E))
    n_classic = n_waves = 0
    for n, step in enumerate(case["steps"]):
        ids = torch.tensor(step["ids"], dtype=torch.int32, device=DEV).view(-1, k)
        T = ids.shape[0]
        hs = torch.zeros((T, 64), dtype=torch.bfloat16, device=DEV)
        if step["kind"] == "gap":
            try:
                torch.ops.vllm.sluice_stream_gap(hs, ids, 0)
                overflow = False
            except RuntimeError as e:
                assert "exceeds slots" in str(e)
                overflow = True
            assert overflow == step["overflow"], n
            if overflow:
                break
        else:
            off.set_step_signal(step["nd"], step["ndec"], step["real_step"])
            qm.maps.clear()
            qm.markers.clear()
            tw = torch.ones((T, k), dtype=torch.float32, device=DEV)
            out = layer.quant_method.apply(layer=layer, x=hs, topk_weights=tw, topk_ids=ids)
            torch.cuda.synchronize()
            assert out.shape == hs.shape and out.dtype == torch.bfloat16
            assert len(qm.maps) == len(step["waves"]), n
            for m, mk, want in zip(qm.maps, qm.markers, step["waves"]):
                m = m.cpu().tolist()
                mk = mk.float().cpu().tolist()
                pairs = [[g, s] for g, s in enumerate(m) if s >= 0]
                assert pairs == want["pairs"], (n, "map")
                for g, s in pairs:  # the wave's kernel sees its experts' rows
                    assert mk[s] == float(lof[g]), (n, g, s)
            n_classic += 1
            n_waves += len(step["waves"])
        st = cache._state()
        want = step["state"]
        for key in ("slot_of", "expert_in_slot", "probation", "protected", "free_slots"):
            assert st[key] == want[key], (n, key)
        assert cache.map_is_standing == want["map_is_standing"], n
        torch.cuda.synchronize()
        assert cache.expert_map_buf.cpu().tolist() == want["map"], n
        if "policy" in step:
            got, wp = cache.policy_state(), step["policy"]
            assert sorted([l, f] for l, f in got["freq"].items()) == wp["freq"], n
            assert (got["steps_small"], got["steps_scan"], got["lfu_steps"]) == (
                wp["steps_small"], wp["steps_scan"], wp["lfu_steps"]), n
            if "counts_decode" in wp:
                assert got["counts_decode"] == wp["counts_decode"], n
                assert got["counts_scan"] == wp["counts_scan"], n
        if n % 20 == 0 or n == len(case["steps"]) - 1:
            _check_slots(cache)
    _check_slots(cache)
    assert off.classic_counters() == {"steps": n_classic, "waves": n_waves}
    if case.get("counts_jsonl"):
        # the snapshots the offloader wrote == the ones the reference wrote
        recs = []
        for fn in sorted(p.name for p in tmp_path.iterdir()):
            for line in open(tmp_path / fn):
                r = json.loads(line)
                r.pop("ts")
                recs.append({"file": fn, "record": r})
        assert recs == case["counts_jsonl"]
    off._counts_dir = None
    off.close()


@pytest.mark.parametrize("slots,Ts", [(6, [12, 3, 40, 2, 12]), (16, [5, 9, 24])])
def test_classic_layer_output_matches_dense_oracle(slots, Ts):
    """A bf16 layer above the envelope (multi-wave steps at slots=6) against
    the oracle's dense product over the host weights, shared expert
    included; decode, prefill and dummy signals."""
    from oracle import moe as om
    from sluice_amd.decoder import SyntheticMoELayer, build_offloaded

    E, k, H, I = 32, 4, 256, 128
    torch.manual_seed(0)
    layer = SyntheticMoELayer(H, I, E, k, scoring="softmax", renorm=True, shared_I=128, seed=5,
                              device=DEV)
    off = build_offloaded([layer], slots, DEV)
    cache = off._caches[id(layer)]
    rng = np.random.default_rng(1)
    signals = [(None, None, True), (0, 0, True), (None, None, False)]
    multi = 0
    for i, T in enumerate(Ts):
        print(f"  slots={slots} T={T}", flush=True)
        nd, ndec, real = signals[i % 3] if i % 2 else (T, T, True)
        off.set_step_signal(nd, ndec, real)
        before = off.classic_counters()["waves"]
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(
            torch.bfloat16).to(DEV)
        out = layer(x)
        torch.cuda.synchronize()
        waves = off.classic_counters()["waves"] - before
        multi += waves > 1
        ref = om.fused_experts(x.float().cpu().numpy(), layer.host_w13.float().numpy(),
                               layer.host_w2.float().numpy(), layer.last_weights.cpu().numpy(),
                               layer.last_ids.cpu().numpy(),
                               shared=layer.shared(x).float().cpu().numpy())
        err = om.rel_l2(out.float().cpu().numpy(), ref)
        print(f"    waves={waves} rel_l2={err:.2e}", flush=True)
        assert waves >= 1 and err <= 1e-2
        _check_slots(cache)
    if slots == 6:
        assert multi >= 2
    off.close()


def _decode(spec, layers, slots, schedule, graphs, gap_server):
    from sluice_amd.decoder import SyntheticDecoder

    cmax = max(schedule)
    dec = SyntheticDecoder(spec, max_batch=cmax, slots=slots, gen_len=len(schedule) + 16,
                           layers=layers, device=DEV, seed=4, gap_server=gap_server)
    for c in sorted(set(schedule)):
        if graphs:
            dec.capture(c)
        else:
            for _ in range(2):
                dec.step_eager(c)
            dec.reset(c)
    toks = []
    for c in schedule:
        if graphs:
            dec.step_graphs(c)
        else:
            dec.step_eager(c)
        toks.append(dec.state[c].tokens.clone())
    dec.sync()
    toks = [t.cpu().numpy() for t in toks]
    state = [cache._state() for cache in dec.caches]
    maps = [cache.expert_map_buf.cpu().tolist() for cache in dec.caches]
    cl = dec.off.classic_counters()
    dec.close()
    return toks, state, maps, cl


@pytest.mark.parametrize("spec,layers,slots,schedule", [
    ("qwen3", 2, 64, [12] * 6),
    ("qwen3", 2, 64, [4, 12, 4, 4, 12, 12, 4]),
    ("v2lite", 3, 48, [12, 2, 12, 2]),
])
def test_decoder_above_envelope_graphs_match_eager(spec, layers, slots, schedule):
    """Captured pieces around the eager classic hook (gap server attached)
    against eager steps with inline gaps: identical tokens, slot state and
    maps, over schedules that alternate gap-sized and classic-sized
    batches."""
    print(f"decoder {spec} layers={layers} schedule={schedule}", flush=True)
    a, sa, ma, ca = _decode(spec, layers, slots, schedule, graphs=False, gap_server=False)
    b, sb, mb, cb = _decode(spec, layers, slots, schedule, graphs=True, gap_server=True)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    for x, y in zip(sa, sb):
        assert x["expert_in_slot"] == y["expert_in_slot"]
        assert x["probation"] == y["probation"] and x["protected"] == y["protected"]
        assert x["counters"][:4] == y["counters"][:4]
    assert ma == mb
    assert ca == cb and ca["steps"] > 0


def test_prefill_sized_classic_step_matches_dense_oracle():
    """A prefill-sized step (700 tokens x top-8 = 5600 pairs, more than one
    expert-product launch takes) on the classic path: prefill signal, every
    expert selected, several waves, against the oracle."""
    from oracle import moe as om
    from sluice_amd.decoder import SyntheticMoELayer, build_offloaded

    E, k, H, I, T = 32, 8, 128, 64, 700
    layer = SyntheticMoELayer(H, I, E, k, scoring="softmax", renorm=True, seed=9, device=DEV)
    off = build_offloaded([layer], 12, DEV)
    off.set_step_signal(0, 0, True)
    rng = np.random.default_rng(2)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(
        torch.bfloat16).to(DEV)
    out = layer(x)
    torch.cuda.synchronize()
    assert off.classic_counters()["waves"] > 1
    ref = om.fused_experts(x.float().cpu().numpy(), layer.host_w13.float().numpy(),
                           layer.host_w2.float().numpy(), layer.last_weights.cpu().numpy(),
                           layer.last_ids.cpu().numpy())
    err = om.rel_l2(out.float().cpu().numpy(), ref)
    print(f"  T={T} waves={off.classic_counters()['waves']} rel_l2={err:.2e}", flush=True)
    assert err <= 1e-2
    _check_slots(off._caches[id(layer)])
    off.close()


def test_checkpoint_loaded_layer_matches_oracle(tmp_path):
    """Expert rows from a safetensors checkpoint -> pinned stores (loader)
    -> adopted by the offloader -> slots -> the expert product: a layer's
    outputs on the gap path (T <= thr) and the classic path (T > thr)
    against the oracle over the checkpoint's own tensors."""
    from safetensors.torch import save_file

    from oracle import moe as om
    from sluice_amd import loader
    from sluice_amd.decoder import _StoreMoELayer, build_offloaded

    E, k, H, I = 16, 4, 256, 128
    sp = dict(E=E, H=H, I=I, k=k, fp8=False, e_bias=False, shared_I=0, scoring="softmax",
              renorm=True, routed_scale=1.0, n_group=1, topk_group=1)
    g = torch.Generator().manual_seed(11)
    t = {}
    for e in range(E):
        for proj, shp in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            t[f"model.layers.3.mlp.experts.{e}.{proj}.weight"] = (
                torch.randn(shp, generator=g) * 0.05).to(torch.bfloat16)
    save_file(t, str(tmp_path / "model.safetensors"))
    store = loader.expert_stores_from_checkpoint(str(tmp_path), 3)
    host13 = torch.stack([torch.cat([t[f"model.layers.3.mlp.experts.{e}.gate_proj.weight"],
                                     t[f"model.layers.3.mlp.experts.{e}.up_proj.weight"]])
                          for e in range(E)]).float().numpy()
    host2 = torch.stack([t[f"model.layers.3.mlp.experts.{e}.down_proj.weight"]
                         for e in range(E)]).float().numpy()
    layer = _StoreMoELayer(sp, store, 0, DEV, None, "layers.3.mlp", gate_std=0.05)
    off = build_offloaded([layer], 8, DEV)  # thr = 2
    cache = off._caches[id(layer)]
    assert cache.cpu_store["w13_weight"].data_ptr() == store["w13_weight"].tensor.data_ptr()
    rng = np.random.default_rng(4)
    for T in (1, 2, 6, 2):
        off.set_step_signal(T, T, True)
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(
            torch.bfloat16).to(DEV)
        out = layer(x)
        torch.cuda.synchronize()
        tw, ti = layer.select(layer.logits(x))
        ref = om.fused_experts(x.float().cpu().numpy(), host13, host2, tw.cpu().numpy(),
                               ti.cpu().numpy())
        err = om.rel_l2(out.float().cpu().numpy(), ref)
        print(f"  T={T} rel_l2={err:.2e}", flush=True)
        assert err <= 1e-2
    _check_slots(cache)
    off.close()


def test_fp8_checkpoint_loaded_layer_matches_oracle(tmp_path):
    """A block-quantised fp8 checkpoint (DeepSeek-V3 naming: e4m3fn
    ``weight`` plus 128x128 ``weight_scale_inv``) -> pinned stores (loader:
    four per-expert params) -> the offloader's slots (each miss streams four
    rows) -> the fp8 expert product, on the gap path (T <= thr) and the
    classic path (T > thr): slot rows equal the checkpoint's bytes and the
    layer output is within the fp8 tolerance (3e-2) of the oracle over the
    checkpoint's dequantised tensors."""
    from safetensors.torch import save_file

    from oracle import moe as om
    from sluice_amd import loader
    from sluice_amd.decoder import _StoreMoELayer, build_offloaded

    E, k, H, I = 16, 4, 256, 128
    sp = dict(E=E, H=H, I=I, k=k, fp8=True, e_bias=False, shared_I=0, scoring="softmax",
              renorm=True, routed_scale=1.0, n_group=1, topk_group=1)
    g = torch.Generator().manual_seed(12)
    t = {}
    key = "model.layers.5.mlp.experts.{e}.{proj}.{kind}"
    for e in range(E):
        for proj, shp in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            t[key.format(e=e, proj=proj, kind="weight")] = (
                torch.randn(shp, generator=g) * 4).to(torch.float8_e4m3fn)
            t[key.format(e=e, proj=proj, kind="weight_scale_inv")] = (
                torch.rand((shp[0] // 128, shp[1] // 128), generator=g) * 0.005 + 0.005)
    save_file(t, str(tmp_path / "model.safetensors"))
    store = loader.expert_stores_from_checkpoint(str(tmp_path), 5)
    assert sorted(store) == ["w13_weight", "w13_weight_scale", "w2_weight", "w2_weight_scale"]

    def deq(proj, e):
        q = t[key.format(e=e, proj=proj, kind="weight")].view(torch.uint8).numpy()
        s = t[key.format(e=e, proj=proj, kind="weight_scale_inv")].numpy()
        return om.dequant_block(q, s)

    host13 = np.stack([np.concatenate([deq("gate_proj", e), deq("up_proj", e)])
                       for e in range(E)])
    host2 = np.stack([deq("down_proj", e) for e in range(E)])
    layer = _StoreMoELayer(sp, store, 0, DEV, None, "layers.5.mlp", gate_std=0.05)
    off = build_offloaded([layer], 8, DEV)  # thr = 2
    cache = off._caches[id(layer)]
    assert len(cache.param_names) == 4
    rng = np.random.default_rng(6)
    for T in (1, 2, 6, 2, 1):
        off.set_step_signal(T, T, True)
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(
            torch.bfloat16).to(DEV)
        out = layer(x)
        torch.cuda.synchronize()
        tw, ti = layer.select(layer.logits(x))
        ref = om.fused_experts(x.float().cpu().numpy(), host13, host2, tw.cpu().numpy(),
                               ti.cpu().numpy())
        err = om.rel_l2(out.float().cpu().numpy(), ref)
        print(f"  T={T} rel_l2={err:.2e}", flush=True)
        assert err <= 3e-2
        _check_slots(cache)
    assert off.classic_counters()["steps"] >= 1
    off.close()
