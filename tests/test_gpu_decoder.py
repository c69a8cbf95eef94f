"""End-to-end decode through the router-split path: graph-piece decoding
(pieces replayed around the eager gap) produces exactly the tokens and the
gap state of eager decoding through the registered ops, and the offloaded
decoder's MoE layers agree with the oracle."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _run(spec, layers, c, steps, graphs, slots, gap_server, uniform=False, pipelined=True):
    from sluice_amd import _lib
    from sluice_amd.decoder import SyntheticDecoder

    dec = SyntheticDecoder(spec, max_batch=c, slots=slots, gen_len=steps + 16, layers=layers,
                           device=DEV, seed=3, gap_server=gap_server, uniform_routing=uniform)
    try:
        if not pipelined:
            dec.set_gap_mode(server=gap_server, pipelined=False)
        return _decode(dec, c, steps, graphs)
    finally:
        _lib.load().sluice_gap_set_pipelined(1)  # process-wide: restore the default


def _decode(dec, c, steps, graphs):
    toks = []

    def out_of_step():
        # the next tokens; a MoE stack without attention: its output rows' bits
        st = dec.state[c]
        return st.tokens.clone() if st.tokens is not None else st.x.view(torch.int16).clone()

    if graphs:
        dec.capture(c)
        for _ in range(steps):
            dec.step_graphs(c)
            toks.append(out_of_step())
    else:
        for _ in range(2):  # the same warm-up capture() does
            dec.step_eager(c)
        dec.reset(c)
        for _ in range(steps):
            dec.step_eager(c)
            toks.append(out_of_step())
    dec.sync()
    out = torch.stack(toks).cpu().numpy()
    state = [cache._state() for cache in dec.caches]
    maps = [cache.expert_map_buf.cpu().tolist() for cache in dec.caches]
    dec.close()
    return out, state, maps


@pytest.mark.parametrize("spec,layers,c,slots", [("v2lite", 3, 4, 48), ("qwen3", 2, 8, 64),
                                                ("v3", 2, 8, 64)])
def test_one_graph_step_with_gap_server_matches_eager_inline_gaps(spec, layers, c, slots):
    """Reference structure (eager gaps served inline between ops) against the
    MI355X structure (gap server, whole step one hipGraph): identical tokens,
    slot assignment, segment order, counters and maps."""
    print(f"decoder {spec} layers={layers} c={c}", flush=True)
    a, sa, ma = _run(spec, layers, c, 12, graphs=False, slots=slots, gap_server=False)
    b, sb, mb = _run(spec, layers, c, 12, graphs=True, slots=slots, gap_server=True)
    assert np.array_equal(a, b)
    for x, y in zip(sa, sb):
        assert x["expert_in_slot"] == y["expert_in_slot"]
        assert x["probation"] == y["probation"] and x["protected"] == y["protected"]
        assert x["counters"][:4] == y["counters"][:4]
    assert ma == mb
    assert sum(x["counters"][1] for x in sa) > 0  # the miss path was exercised


@pytest.mark.parametrize("spec,layers,c,slots,steps", [("qwen3", 2, 4, 32, 10),
                                                      ("v3", 2, 8, 64, 5)])
def test_miss_heavy_graph_decode_matches_eager(spec, layers, c, slots, steps):
    """Uniform routing over few slots: nearly every selected expert misses,
    so in the replayed graph each layer's expert product computes its
    resident experts while the misses' rows stream and waits per filled
    slot (the gap server answers before the rows land).  Tokens, slot state,
    counters and maps equal eager decoding, whose inline gaps return only
    after every row has landed."""
    print(f"miss-heavy decoder {spec} layers={layers} c={c} slots={slots}", flush=True)
    a, sa, ma = _run(spec, layers, c, steps, graphs=False, slots=slots, gap_server=False,
                     uniform=True)
    b, sb, mb = _run(spec, layers, c, steps, graphs=True, slots=slots, gap_server=True,
                     uniform=True)
    assert np.array_equal(a, b)
    for x, y in zip(sa, sb):
        assert x["expert_in_slot"] == y["expert_in_slot"]
        assert x["counters"][:4] == y["counters"][:4]
    assert ma == mb
    # most of each step's (token, expert) pairs missed
    misses = sum(y["counters"][1] for y in sb)
    assert misses >= steps * layers * c * 2, misses


@pytest.mark.parametrize("spec,layers,c,slots,steps", [("qwen3", 2, 4, 32, 8),
                                                      ("v3", 2, 8, 64, 4)])
def test_copies_before_compute_matches_pipelined_gap(spec, layers, c, slots, steps):
    """The reference's order -- a missing gap answered only after its rows
    landed (sluice_gap_set_pipelined(0)), so the expert product never
    overlaps the copies -- in both orchestrations (one graph with the gap
    server; captured pieces around inline gaps, the host waiting for each
    layer's ids) decodes the same tokens, with the same slot state, counters
    and maps, as the pipelined one-graph step, on miss-heavy routing."""
    print(f"copy order {spec} layers={layers} c={c} slots={slots}", flush=True)
    a, sa, ma = _run(spec, layers, c, steps, graphs=True, slots=slots, gap_server=True,
                     uniform=True)
    for server in (True, False):
        b, sb, mb = _run(spec, layers, c, steps, graphs=True, slots=slots, gap_server=server,
                         uniform=True, pipelined=False)
        assert np.array_equal(a, b), server
        for x, y in zip(sa, sb):
            assert x["expert_in_slot"] == y["expert_in_slot"]
            assert x["counters"][:4] == y["counters"][:4]
        assert ma == mb
    assert sum(x["counters"][1] for x in sa) >= steps * layers * c * 2


def test_piece_graphs_with_inline_gaps_match_eager():
    a, sa, ma = _run("v2lite", 2, 2, 8, graphs=False, slots=48, gap_server=False)
    b, sb, mb = _run("v2lite", 2, 2, 8, graphs=True, slots=48, gap_server=False)
    assert np.array_equal(a, b)
    assert [x["expert_in_slot"] for x in sa] == [y["expert_in_slot"] for y in sb]
    assert ma == mb


def test_moe_layer_against_oracle():
    """One offloaded v2lite-shaped MoE layer (shared experts included) vs the
    oracle on the same routing."""
    from oracle import moe as om
    from sluice_amd.decoder import SyntheticDecoder

    dec = SyntheticDecoder("v2lite", max_batch=8, slots=48, gen_len=16, layers=2, device=DEV,
                           gap_server=False)
    m = dec.moe_layers[0]
    cache = dec.caches[0]
    rng = np.random.default_rng(0)
    for step in range(3):
        x = torch.from_numpy(rng.standard_normal((8, 2048)).astype(np.float32)).to(
            torch.bfloat16).to(DEV)
        out = m(x)  # patched router-split entry: gate, routing, gap op, experts, shared
        torch.cuda.synchronize()
        tw, ti = m.select(m.logits(x))
        ids = ti.cpu().numpy()
        host13 = cache.cpu_store["w13_weight"].float().numpy()
        host2 = cache.cpu_store["w2_weight"].float().numpy()
        ref = om.fused_experts(x.float().cpu().numpy(), host13, host2, tw.cpu().numpy(), ids,
                               shared=m.shared(x).float().cpu().numpy())
        err = om.rel_l2(out.float().cpu().numpy(), ref)
        print(f"  step {step} rel_l2={err:.2e}", flush=True)
        assert err <= 1e-2
    dec.close()


def test_v3_routed_fp8_layer_against_oracle():
    """A DeepSeek-V3-routed fp8 MoE layer through the armed entry: 256
    experts top-8, sigmoid + correction bias over 8 groups (top-4 groups),
    renormalised, scale 2.5; e4m3fn experts and shared expert with 128x128
    block scales; 64 slots, 8 tokens per step (hidden 512, intermediate 256,
    so the float64 oracle stays small).  Slot assignment follows the oracle's
    routing of the entry's own logits, and the layer output is within the
    fp8 tolerance of the oracle on the dequantised weights."""
    from oracle import moe as om
    from oracle import routing as orr
    from oracle.slru import LayerCache
    from sluice_amd.decoder import SPECS, _expert_store, _StoreMoELayer, build_offloaded

    sp = dict(SPECS["v3"], H=512, I=256, shared_I=256)
    store = _expert_store(sp, 7001, DEV, True)
    layer = _StoreMoELayer(sp, store, 1, DEV, None, "layers.1.mlp")
    off = build_offloaded([layer], slots=64, device=DEV)
    assert off._rs_routes[0] is not None and off._rs_routes[0].scoring == "sigmoid"
    cache = off._caches[id(layer)]
    assert len(cache.param_names) == 4
    oracle = LayerCache(256, 256, 64, off.protect_frac)
    deq = {n: om.dequant_block(cache.cpu_store[n].numpy(), cache.cpu_store[n + "_scale"].numpy())
           for n in ("w13_weight", "w2_weight")}
    sh = layer.shared
    sh_ref_w = (om.dequant_block(sh.gate_up.cpu().numpy(), sh.gate_up_scale.cpu().numpy()),
                om.dequant_block(sh.down.cpu().numpy(), sh.down_scale.cpu().numpy()))
    bias = layer.e_score_correction_bias.detach().float().cpu().numpy()
    rng = np.random.default_rng(3)
    misses = 0
    for step in range(4):
        x = torch.from_numpy(rng.standard_normal((8, 512)).astype(np.float32)).to(
            torch.bfloat16).to(DEV)
        out = layer(x)
        logits = layer.logits(x)  # the gate kernel the entry ran, on the same input
        torch.cuda.synchronize()
        ids, w = orr.sigmoid_topk(logits.cpu().numpy(), bias, 8, 8, 4, True, 2.5)
        misses += len(oracle.gap(ids.reshape(-1).tolist(), fast_hit=True))
        assert cache._state()["expert_in_slot"] == [
            -1 if v is None else v for v in oracle.expert_in_slot], step
        xf = x.float().cpu().numpy()
        ref = om.fused_experts(xf, deq["w13_weight"], deq["w2_weight"], w, ids,
                               shared=om.shared_mlp(xf, *sh_ref_w))
        err = om.rel_l2(out.float().cpu().numpy(), ref)
        print(f"  step {step} rel_l2={err:.2e}", flush=True)
        assert err <= 3e-2
    assert misses > 0
    off.close()



@pytest.mark.parametrize("spec,slots,c,steps,uniform", [
    ("v2lite", 48, 8, 24, False), ("qwen3", 64, 8, 16, False), ("qwen3", 96, 12, 40, False),
    ("v3", 64, 8, 8, False), ("qwen3", 32, 4, 64, True)])
def test_full_size_decode_slots_follow_the_oracle(spec, slots, c, steps, uniform):
    """The configured models at full depth and shape (DeepSeek-V2-Lite: 26
    MoE layers of 64 experts at 48 slots; Qwen3-30B-A3B: 48 layers of 128 at
    64 and 96 slots; the DeepSeek-V3 fp8 stack: 8 layers of 256 at 64),
    decoded from empty slot caches with the Zipf + AR(1) routing -- two eager
    steps, then the captured one-graph step with the gap server: after every
    step every layer's expert map, and at the end its slot assignment, SLRU
    segment order and counters, equal the oracle's SLRU replaying the ids the
    layer routed; the last layer's occupied slots hold their experts' host
    rows byte for byte.  The miss-dominated stress runs the same checks:
    Qwen3 shape at 48 layers, 32 slots, 4 tokens per step with uniform
    i.i.d. top-8 routing, where nearly every step of every layer evicts
    (src/sluice/offloader.py:2036-2081, the victim scan under constant
    eviction)."""
    from oracle.slru import LayerCache
    from sluice_amd.decoder import SyntheticDecoder

    print(f"full-size decode {spec} slots={slots} c={c} steps={steps} uniform={uniform}",
          flush=True)
    dec = SyntheticDecoder(spec, max_batch=c, slots=slots, gen_len=steps + 16, device=DEV,
                           host_pool="shared", uniform_routing=uniform)
    try:
        E = dec.sp["E"]
        oracles = [LayerCache(E, E, slots, dec.off.protect_frac) for _ in dec.moe_layers]

        def check_step(label):
            dec.sync()
            for n, (io, m) in enumerate(zip(dec.layer_io[c], dec.moe_layers)):
                ids = io["ti"].cpu().numpy().reshape(-1).tolist()
                oracles[n].gap(ids, fast_hit=True)
                assert m._expert_map.cpu().tolist() == oracles[n].map, (label, n)

        for i in range(2):
            dec.step_eager(c)
            check_step(f"eager {i}")
        dec.capture(c, warmup=0)
        for i in range(steps):
            dec.step_graphs(c)
            check_step(f"graph {i}")
        misses = 0
        for n, (cache, o) in enumerate(zip(dec.caches, oracles)):
            st = cache._state()
            assert st["expert_in_slot"] == [-1 if v is None else v for v in o.expert_in_slot], n
            assert st["probation"] == list(o.probation) and st["protected"] == list(o.protected), n
            assert st["counters"][:3] == [o.gaps, o.misses, o.fast_hits], n
            misses += o.misses
        # past the cold fill: some layer evicted and streamed into used slots
        assert any(o.misses > slots for o in oracles), misses
        if uniform:  # every layer evicts on most steps
            assert all(o.misses > (steps + 2) * slots // 2 for o in oracles), misses
        cache = dec.caches[-1]
        occ = [(s, e) for s, e in enumerate(cache.expert_in_slot) if e is not None]
        sl = torch.tensor([s for s, _ in occ], device=DEV)
        ex = torch.tensor([e for _, e in occ])
        for name in cache.param_names:
            got = cache.gpu_cache[name].index_select(0, sl)
            want = cache.cpu_store[name].index_select(0, ex).to(DEV)
            assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), name
        print(f"  {len(oracles)} layers, {misses} misses, {len(occ)} slots checked", flush=True)
    finally:
        dec.close()


def test_full_size_mixed_classic_and_gap_steps_follow_the_oracle():
    """Qwen3-30B-A3B at full depth (48 MoE layers of 128 experts, 64 slots)
    decoding a schedule that alternates batches above the router-split
    envelope (12 tokens x top-8 > 64 slots: the classic hook, waves planned
    on the host between captured pieces) with batches inside it (8 tokens:
    the gap), from empty caches: every layer's expert map after every step,
    and at the end its slot assignment, segment order and counters, equal
    the oracle replaying the same ids through the same kind of step."""
    from oracle.slru import LayerCache
    from sluice_amd.decoder import SyntheticDecoder

    schedule = [12, 8, 12, 12, 8, 8, 12, 8, 12, 12, 12, 8]
    print(f"full-size mixed decode qwen3 slots=64 schedule={schedule}", flush=True)
    dec = SyntheticDecoder("qwen3", max_batch=12, slots=64, gen_len=len(schedule) + 16,
                           device=DEV, host_pool="shared")
    try:
        E = dec.sp["E"]
        oracles = [LayerCache(E, E, 64, dec.off.protect_frac) for _ in dec.moe_layers]
        classic_steps = 0

        def check_step(c, label):
            nonlocal classic_steps
            dec.sync()
            classic = dec.classic(c)
            classic_steps += classic
            for n, (io, m) in enumerate(zip(dec.layer_io[c], dec.moe_layers)):
                ids = io["ti"].cpu().numpy().reshape(-1).tolist()
                if classic:
                    oracles[n].classic(ids, c, c, c, True)
                else:
                    oracles[n].gap(ids, fast_hit=True)
                assert m._expert_map.cpu().tolist() == oracles[n].map, (label, n)

        assert dec.classic(12) and not dec.classic(8)
        for c in (8, 12):  # one recorded eager step per batch size, then capture
            dec.step_eager(c)
            check_step(c, f"eager c={c}")
            dec.capture(c, warmup=0)
        for i, c in enumerate(schedule):
            dec.step_graphs(c)
            check_step(c, f"step {i} c={c}")
        for n, (cache, o) in enumerate(zip(dec.caches, oracles)):
            st = cache._state()
            assert st["expert_in_slot"] == [-1 if v is None else v for v in o.expert_in_slot], n
            assert st["probation"] == list(o.probation) and st["protected"] == list(o.protected), n
            assert st["counters"][:3] == [o.gaps, o.misses, o.fast_hits], n
        assert classic_steps == 1 + schedule.count(12)
        print(f"  {classic_steps} classic steps, {sum(o.misses for o in oracles)} misses",
              flush=True)
    finally:
        dec.close()


@pytest.mark.parametrize("spec,layers,slots,c,steps,coded", [
    ("v2lite", None, 48, 8, 24, False), ("qwen3", None, 64, 8, 16, False),
    ("v3", 2, 64, 8, 8, False), ("v2lite", 8, 48, 8, 24, True), ("qwen3", 8, 64, 8, 16, True)])
def test_offloaded_decode_equals_fully_resident_decode(monkeypatch, spec, layers, slots, c,
                                                       steps, coded):
    """Streaming experts must not change the output (the reference's own
    correctness demo, examples/bitcompare_v2lite.py: greedy ids of an
    offloaded run diffed against an all-resident one).  The same seeded
    decoder decodes the same steps twice through the captured one-graph
    step: with fewer slots than experts (gaps streaming and evicting) and
    with a slot for every expert, pre-filled and pinned, the hook kept on
    (SLUICE_NO_STATIC_FULL=1, src/sluice/offloader.py:289-293, 948-1012:
    nothing streams); the next tokens of every step (the output rows' bits
    for the MoE stack without attention) are identical.  The streaming runs
    keep the default staging rows, and on V2-Lite and Qwen3 some of their
    misses are copied from staged rows.  Coded: the host stores coded
    (SLUICE_CODEC=1), every miss decoded into its slot; on Qwen3 a pinned
    budget leaves part of the layers uncoded."""
    from sluice_amd.decoder import SyntheticDecoder

    def decode(n_slots):
        dec = SyntheticDecoder(spec, max_batch=c, slots=n_slots, gen_len=steps + 16,
                               layers=layers, device=DEV, host_pool="shared")
        try:
            dec.capture(c)
            out = []
            for _ in range(steps):
                dec.step_graphs(c)
                st = dec.state[c]
                out.append(st.tokens.clone() if st.tokens is not None
                           else st.x.view(torch.int16).clone())
            dec.sync()
            streamed = dec.gap_counters()["misses"]
            staged = dec.off.stage_counters()["hits"]
            if coded and n_slots < E:
                cc = dec.off.codec_counters()
                print(f"  codec {cc}", flush=True)
                n_moe = len(dec.off._rs_caches)
                if spec == "qwen3":  # a pinned budget for part of the layers
                    assert 0 < cc["params"] < 2 * n_moe and 0 < cc["decodes"] < streamed
                else:
                    assert cc["params"] == 2 * n_moe and cc["decodes"] == streamed
            return torch.stack(out).cpu().numpy(), streamed, staged
        finally:
            dec.close()

    E = __import__("sluice_amd.decoder", fromlist=["SPECS"]).SPECS[spec]["E"]
    print(f"bitcompare {spec} slots {slots} vs {E}, c={c}, {steps} steps, coded={coded}",
          flush=True)
    monkeypatch.setenv("SLUICE_CODEC", "1" if coded else "0")
    if coded and spec == "qwen3":
        # room for the coded stores of about half the layers: coded and
        # uncoded layers stream side by side under one gap server
        monkeypatch.setenv("SLUICE_CODEC_PIN_GB", "5")
    off, misses, staged = decode(slots)
    print(f"  misses {misses}, from staged rows {staged}", flush=True)
    monkeypatch.setenv("SLUICE_NO_STATIC_FULL", "1")
    full, full_misses, _ = decode(E)
    assert misses > slots and full_misses == 0, (misses, full_misses)
    if spec != "v3":
        assert staged > 0
    assert np.array_equal(off, full)


def test_decode_on_streams_that_share_hardware_queues():
    """With more streams than the process has hardware queues (HIP shares an
    in-order queue between streams beyond GPU_MAX_HW_QUEUES), a miss-heavy
    pipelined decode runs on every stream: streams made before the decoder's
    copy machinery and after it, 6 each, the one-graph step with the gap
    server on each in turn.  The gap's row copies go to the SDMA engines with
    HSA completion signals, and the coded rows' decodes run on an HSA queue
    of the library's own, so neither waits behind the expert product that
    waits for it; every gap wait is bounded at 5 s here, so a copy or decode
    stuck behind a kernel ends as an error, not a hang."""
    from sluice_amd import _lib
    from sluice_amd.decoder import SyntheticDecoder

    lib = _lib.load()
    before = [torch.cuda.Stream(device=DEV) for _ in range(6)]
    for s in before:
        with torch.cuda.stream(s):
            torch.zeros(1, device=DEV).add_(1)
    torch.cuda.synchronize()
    assert lib.sluice_gap_set_timeout(5.0) == 0
    dec = SyntheticDecoder("qwen3", max_batch=4, slots=32, gen_len=96, layers=4, device=DEV,
                           seed=3, uniform_routing=True)
    try:
        after = [torch.cuda.Stream(device=DEV) for _ in range(6)]
        misses = 0
        for n, s in enumerate(before + after):
            print(f"decode on extra stream {n}", flush=True)
            with torch.cuda.stream(s):
                dec.graphs = {}
                dec.capture(4)
                for _ in range(4):
                    dec.step_graphs(4)
                dec.sync()  # raises on a gap wait that reached its bound
            now = dec.gap_counters()["misses"]
            assert now > misses, n  # every stream's steps streamed experts
            misses = now
        # the misses were decoded from the coded stores (the default)
        assert dec.off.codec_counters()["decodes"] == misses
    finally:
        dec.close()
        lib.sluice_gap_set_timeout(0.0)
