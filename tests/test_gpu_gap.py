"""a3-a8 on the GPU: the device gap (slot-lookup kernel -> host record ->
native SLRU -> SDMA copies of missing rows -> map kernel) replays the
reference's golden traces bit for bit: stream-in order, slot assignment,
segment order and the device expert map after every step, and every
occupied slot's bytes equal the pinned host row of the expert it holds."""

import types

import numpy as np
import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


class _Layer(nn.Module):
    def __init__(self, E, local_n, H=64, I=32, expert_map=None):
        super().__init__()
        self.global_num_experts = E
        self.local_num_experts = local_n
        self.quant_method = types.SimpleNamespace()
        g = torch.Generator().manual_seed(E * 1000 + local_n)
        self.w13_weight = nn.Parameter(
            torch.randn((local_n, 2 * I, H), generator=g).to(torch.bfloat16), requires_grad=False)
        self.w2_weight = nn.Parameter(
            torch.randn((local_n, H, I), generator=g).to(torch.bfloat16), requires_grad=False)
        if expert_map is not None:
            self.register_buffer("_orig_map", expert_map)

    @property
    def expert_map(self):
        return getattr(self, "_expert_map", None) if hasattr(self, "_expert_map") else getattr(
            self, "_orig_map", None)


def _offloader(monkeypatch, slots, frac, fast_hit):
    monkeypatch.setenv("SLUICE_ROUTER_SPLIT", "1")
    monkeypatch.setenv("SLUICE_PROTECT_FRAC", str(frac))
    monkeypatch.setenv("SLUICE_RS_FAST_HIT", "1" if fast_hit else "0")
    from sluice_amd.offloader import ExpertStreamOffloader

    return ExpertStreamOffloader(expert_cache_slots=slots)


def _check_slots(cache, layer):
    torch.cuda.synchronize()
    for name in cache.param_names:
        slot_t = cache.gpu_cache[name].cpu()
        host_t = cache.cpu_store[name]
        for s, loc in enumerate(cache.expert_in_slot):
            if loc is not None:
                assert torch.equal(slot_t[s].view(torch.int16), host_t[loc].view(torch.int16)), (
                    name, s, loc)


def _cases(golden):
    return list(range(len(golden["cases"])))


def _check_plan(cache, ids, k, E):
    """The expert product's plan the gap kernel built equals the align
    kernel's plan of the same ids over the map (and pending slots) the gap
    left: block count, each block's slot field, count and pairs, and the
    validity flags."""
    from sluice_amd import _lib

    lib = _lib.load()
    P = ids.numel()
    ref = torch.full_like(cache.plan, -7)
    rc = lib.sluice_moe_align(ids.data_ptr(), P // k, k, cache.expert_map_buf.data_ptr(), E,
                              cache.num_slots, ref.data_ptr(),
                              torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "sluice_moe_align")
    torch.cuda.synchronize()
    got, want = cache.plan.cpu().numpy(), ref.cpu().numpy()
    nb = int(want[0])
    assert int(got[0]) == nb and int(got[1]) == P
    # plan[2]: the blocks of slots not pending, which come first
    pend = [bool(int(want[4 + 18 * b]) & (1 << 30)) for b in range(nb)]
    assert int(got[2]) == int(want[2]) == pend.count(False)
    assert not any(pend[:pend.count(False)])
    for b in range(nb):
        g, w = got[4 + 18 * b: 4 + 18 * (b + 1)], want[4 + 18 * b: 4 + 18 * (b + 1)]
        assert g[0] == w[0] and g[1] == w[1], b
        assert g[2:2 + w[1]].tolist() == w[2:2 + w[1]].tolist(), b
    assert got[4 + 18 * P: 4 + 19 * P].tolist() == want[4 + 18 * P: 4 + 19 * P].tolist()


def _case_ids():
    from conftest import slru_vectors

    g = slru_vectors()
    return [f"{g['cases'][i]['name']}-fh{int(g['cases'][i]['fast_hit'])}" for i in _cases(g)]


@pytest.mark.parametrize("rows", ["pulled", "sdma"])
@pytest.mark.parametrize("idx", range(len(_case_ids())), ids=_case_ids())
def test_device_gap_replays_reference(monkeypatch, slru_golden, idx, rows):
    """A golden trace replayed through the device gap: per step the slot
    state, the device map and the plan of the reference; every cached
    slot's rows equal its host rows.  rows="pulled": 8 KB and 4 KB rows,
    which the gap kernel copies itself; rows="sdma": 256 KB and 128 KB rows
    on the copy engines."""
    case = slru_golden["cases"][_cases(slru_golden)[idx]]
    print(f"gap case {case['name']} fast_hit={case['fast_hit']} rows={rows}", flush=True)
    E, local_n, k = case["E"], case["local_n"], case["k"]
    emap = None
    if case["local_of"] is not None:
        emap = torch.tensor(case["local_of"], dtype=torch.int32)
    H, I = (64, 32) if rows == "pulled" else (1024, 64)
    layer = _Layer(E, local_n, H=H, I=I, expert_map=emap)
    off = _offloader(monkeypatch, case["slots"], case["protect_frac"], case["fast_hit"])
    if case["pins"]:
        off._pin_layers = {0: list(case["pins"])}  # what SLUICE_PIN_FILE would hold
    off.wrap_modules(iter([layer]))
    with torch.cuda.device(DEV):
        off.post_init()
    cache = off._caches[id(layer)]
    off._rs_caches.append(cache)
    # the buffer attach_router_split gives a router-split layer: each gap
    # kernel also builds the expert product's plan into it
    from sluice_amd import _lib
    cache.plan = torch.zeros(_lib.load().sluice_moe_plan_ints(1, cache.num_slots),
                             dtype=torch.int32, device=DEV)
    assert _lib.load().sluice_layer_pulled_params(cache.handle) == (2 if rows == "pulled" else 0)
    assert cache.free_slots == case["init"]["free_slots"]
    assert cache.expert_in_slot == [None if v < 0 else v
                                    for v in case["init"]["expert_in_slot"]]
    _check_slots(cache, layer)  # pinned rows were copied in at install
    hs = torch.zeros((1, H), dtype=torch.bfloat16, device=DEV)
    for n, step in enumerate(case["steps"]):
        ids = torch.tensor(step["ids"], dtype=torch.int32, device=DEV).view(-1, k)
        overflow = False
        try:
            out = torch.ops.vllm.sluice_stream_gap(hs, ids, len(off._rs_caches) - 1)
            assert out.data_ptr() != hs.data_ptr()
        except RuntimeError as e:
            assert "exceeds slots" in str(e)
            overflow = True
        assert overflow == step["overflow"], n
        st = cache._state()
        want = step["state"]
        assert st["slot_of"] == want["slot_of"], n
        assert st["expert_in_slot"] == want["expert_in_slot"], n
        assert st["probation"] == want["probation"], n
        assert st["protected"] == want["protected"], n
        assert st["free_slots"] == want["free_slots"], n
        if not overflow:
            torch.cuda.synchronize()
            assert cache.expert_map_buf.cpu().tolist() == want["map"], n
        if ids.numel() <= cache.num_slots:
            _check_plan(cache, ids, k, E)
        if n % 25 == 0 or n == len(case["steps"]) - 1:
            _check_slots(cache, layer)
    s = cache.stats()
    assert s["gaps"] == case["counters"]["gaps"]
    assert s["misses"] == case["counters"]["misses"]
    assert s["fast_hits"] == case["counters"]["fast_hits"]
    off.close()


def test_slot_lookup_record(lib):
    """The lookup kernel's record: sorted unique in-range ids and the count of
    owned-but-unmapped ones, published with the requested stamp."""
    import ctypes

    from sluice_amd import _lib

    E = 128
    rng = np.random.default_rng(3)
    ids = rng.integers(-5, E + 5, size=96).astype(np.int32)
    emap = np.full(E, -1, np.int32)
    emap[rng.choice(E, 40, replace=False)] = np.arange(40)
    local_of = np.arange(E, dtype=np.int32)
    local_of[::7] = -1
    rec = torch.zeros(4 + 1024, dtype=torch.int32, device=DEV)
    d = {n: torch.from_numpy(a).to(DEV) for n, a in
         (("ids", ids), ("map", emap), ("lof", local_of))}
    rc = lib.sluice_slot_lookup(d["ids"].data_ptr(), 96, d["map"].data_ptr(),
                                d["lof"].data_ptr(), E, ctypes.c_void_p(rec.data_ptr()), 77,
                                torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "lookup")
    torch.cuda.synchronize()
    r = rec.cpu().numpy()
    uniq = sorted({int(g) for g in ids if 0 <= g < E})
    assert r[0] == 77 and r[1] == len(uniq)
    assert r[4:4 + r[1]].tolist() == uniq
    assert r[2] == sum(1 for g in uniq if local_of[g] >= 0 and emap[g] < 0)


class _Fp8Layer(nn.Module):
    """An fp8 layer's per-expert params, as vLLM's block-quantised FusedMoE
    holds them: e4m3fn w13 [E, 2I, H] and w2 [E, H, I] plus their fp32
    128x128 block scales [E, 2I/128, H/128] and [E, H/128, I/128] -- four
    rows stream per missing expert (src/sluice/offloader.py:2709-2723)."""

    def __init__(self, E, H=256, I=128):
        super().__init__()
        self.global_num_experts = E
        self.local_num_experts = E
        self.quant_method = types.SimpleNamespace()
        g = torch.Generator().manual_seed(4242)

        def codes(*shape):
            return (torch.randn(shape, generator=g) * 0.5).to(torch.float8_e4m3fn).view(torch.uint8)

        self.w13_weight = nn.Parameter(codes(E, 2 * I, H), requires_grad=False)
        self.w2_weight = nn.Parameter(codes(E, H, I), requires_grad=False)
        self.w13_weight_scale = nn.Parameter(
            torch.rand((E, 2 * I // 128, H // 128), generator=g) + 0.01, requires_grad=False)
        self.w2_weight_scale = nn.Parameter(
            torch.rand((E, H // 128, I // 128), generator=g) + 0.01, requires_grad=False)
        # shared by every expert: stays resident, never streamed
        self.e_score_correction_bias = nn.Parameter(torch.zeros(E), requires_grad=False)


def _slot_bytes_match_host(cache):
    torch.cuda.synchronize()
    for name in cache.param_names:
        slot_t = cache.gpu_cache[name].cpu().contiguous().view(torch.uint8)
        host_t = cache.cpu_store[name].contiguous().view(torch.uint8)
        for s, loc in enumerate(cache.expert_in_slot):
            if loc is not None:
                assert torch.equal(slot_t[s], host_t[loc]), (name, s, loc)


@pytest.mark.parametrize("fast_hit", [False, True])
@pytest.mark.parametrize("H,I,pulled", [(256, 128, 2), (512, 256, 2)])
def test_device_gap_v3_fp8_streams_four_rows_per_miss(monkeypatch, slru_golden, fast_hit, H, I,
                                                      pulled):
    """The DeepSeek-V3-shaped golden trace (E = 256, 64 slots, top-8, 8
    tokens per step), replayed on an fp8 layer: per step the stream-ins
    (local -> slot) and the slot state, segment order and device map of the
    reference; the bytes of all four per-expert params of every slot equal
    their host rows; bytes streamed = misses x the four rows' size.  The
    rows of at most 32 KB in whole 16-byte vectors are copied by the gap
    kernel itself, the others go over the copy lanes (H=512: both scale rows
    pulled; H=256: the 32 KB w2 row and the 16-byte w13 scale row pulled,
    the 64 KB w13 row and the 8-byte w2 scale row on the lanes)."""
    case = [c for c in slru_golden["cases"]
            if c["name"] == "v3_s64_zipf" and c["fast_hit"] == fast_hit][0]
    print(f"v3 fp8 gap fast_hit={fast_hit} H={H} I={I}", flush=True)
    E, k = case["E"], case["k"]
    layer = _Fp8Layer(E, H, I)
    off = _offloader(monkeypatch, case["slots"], case["protect_frac"], fast_hit)
    off.wrap_modules(iter([layer]))
    with torch.cuda.device(DEV):
        off.post_init()
    cache = off._caches[id(layer)]
    assert sorted(cache.param_names) == ["w13_weight", "w13_weight_scale", "w2_weight",
                                         "w2_weight_scale"]
    nh, ni = H // 128, I // 128
    assert cache.bytes_per_expert == 2 * I * H + H * I + (2 * ni * nh + nh * ni) * 4
    off._rs_caches.append(cache)
    from sluice_amd import _lib
    assert _lib.load().sluice_layer_pulled_params(cache.handle) == pulled
    cache.plan = torch.zeros(_lib.load().sluice_moe_plan_ints(1, cache.num_slots),
                             dtype=torch.int32, device=DEV)
    hs = torch.zeros((8, 256), dtype=torch.bfloat16, device=DEV)
    prev = list(cache.expert_in_slot)
    for n, step in enumerate(case["steps"]):
        ids = torch.tensor(step["ids"], dtype=torch.int32, device=DEV).view(-1, k)
        torch.ops.vllm.sluice_stream_gap(hs, ids, len(off._rs_caches) - 1)
        st = cache._state()
        want = step["state"]
        for key in ("slot_of", "expert_in_slot", "probation", "protected", "free_slots"):
            assert st[key] == want[key], (n, key)
        now = [None if v < 0 else v for v in st["expert_in_slot"]]
        streamed = sorted([loc, s] for s, loc in enumerate(now) if loc is not None
                          and loc != prev[s])
        assert streamed == sorted(step["streams"]), n
        prev = now
        torch.cuda.synchronize()
        assert cache.expert_map_buf.cpu().tolist() == want["map"], n
        _check_plan(cache, ids, k, E)
        if n % 20 == 0 or n == len(case["steps"]) - 1:
            _slot_bytes_match_host(cache)
    s = cache.stats()
    assert (s["gaps"], s["misses"], s["fast_hits"]) == (
        case["counters"]["gaps"], case["counters"]["misses"], case["counters"]["fast_hits"])
    assert s["bytes"] == s["misses"] * cache.bytes_per_expert
    off.close()


_STAGED_CASES = [("v2lite_zipf", True, "bf16"), ("qwen3_s64_zipf", True, "bf16"),
                 ("ep_half_owned", False, "bf16"), ("pinned", True, "bf16"),
                 ("v3_s64_zipf", True, "fp8"), ("v2lite_zipf", True, "bf16-coded"),
                 ("qwen3_s64_zipf", True, "bf16-coded"), ("ep_half_owned", False, "bf16-coded"),
                 ("pinned", True, "bf16-coded")]


@pytest.mark.parametrize("name,fast_hit,kind", _STAGED_CASES,
                         ids=[f"{n}-fh{int(f)}-{k}" for n, f, k in _STAGED_CASES])
def test_staged_rows_leave_the_golden_replay_unchanged(monkeypatch, slru_golden, name, fast_hit,
                                                       kind):
    """A golden trace replayed through the gap server with two staging rows
    per layer: the server fills them while the link idles (a pause after
    most steps; every third step follows at once, so gaps also meet chunks
    in flight), misses on staged experts are copied into their slots from
    HBM.  Slot state, segment order and device map follow the reference at
    every step, every cached slot's bytes equal its host rows, the bytes
    filled stay misses x expert bytes, and on the Zipf traces some misses
    were served from staged rows.  bf16 rows of 2 MB and 1 MB (two and one
    staging chunks); fp8: the w13 and w2 rows staged, the scale rows pulled
    by the gap kernel.  bf16-coded: the host stores coded, every miss
    decoded into its slot (from the ring or from its staging row), fewer
    bytes over the link."""
    import time

    from sluice_amd import _lib

    case = [c for c in slru_golden["cases"] if c["name"] == name and c["fast_hit"] == fast_hit][0]
    print(f"staged gap case {name} fast_hit={fast_hit} {kind}", flush=True)
    monkeypatch.setenv("SLUICE_STAGE_ROWS", "2")
    monkeypatch.setenv("SLUICE_CODEC", "1" if kind == "bf16-coded" else "0")
    E, local_n, k = case["E"], case["local_n"], case["k"]
    emap = None
    if case["local_of"] is not None:
        emap = torch.tensor(case["local_of"], dtype=torch.int32)
    if kind == "fp8":
        layer, H = _Fp8Layer(E, 512, 256), 512
    else:
        H = 2048
        layer = _Layer(E, local_n, H=H, I=256, expert_map=emap)
    off = _offloader(monkeypatch, case["slots"], case["protect_frac"], fast_hit)
    if case["pins"]:
        off._pin_layers = {0: list(case["pins"])}
    off.wrap_modules(iter([layer]))
    with torch.cuda.device(DEV):
        off.post_init()
    cache = off._caches[id(layer)]
    off._rs_caches.append(cache)
    lib = _lib.load()
    assert lib.sluice_layer_pulled_params(cache.handle) == (2 if kind == "fp8" else 0)
    off.start_gap_server()
    assert off.stage_counters()["rows"] == 2
    hs = torch.zeros((1, H), dtype=torch.bfloat16, device=DEV)
    for n, step in enumerate(case["steps"]):
        assert not step["overflow"]
        ids = torch.tensor(step["ids"], dtype=torch.int32, device=DEV).view(-1, k)
        torch.ops.vllm.sluice_stream_gap(hs, ids, 0)
        off.drain()
        st = cache._state()
        want = step["state"]
        for key in ("slot_of", "expert_in_slot", "probation", "protected", "free_slots"):
            assert st[key] == want[key], (n, key)
        assert cache.expert_map_buf.cpu().tolist() == want["map"], n
        if n % 25 == 0 or n == len(case["steps"]) - 1:
            _slot_bytes_match_host(cache)
        if n % 3 != 2:
            time.sleep(0.002)  # the link idles: the server fills staging rows
    sc = off.stage_counters()
    s = cache.stats()
    print(f"staging: {sc}, misses {s['misses']}", flush=True)
    assert s["bytes"] == s["misses"] * cache.bytes_per_expert
    assert sc["filled"] > 0 and sc["h2d_bytes"] > 0
    assert sc["hits"] <= s["misses"]
    if "zipf" in name:
        assert sc["hits"] > 0
    cc = off.codec_counters()
    print(f"codec: {cc}", flush=True)
    # the rows that cross the link (fp8: the scale rows are pulled by the gap kernel)
    row_bytes = sum(cache.gpu_cache[n][0].nbytes for n in cache.param_names if "scale" not in n)
    over_link = (s["misses"] - sc["hits"]) * row_bytes
    if kind == "bf16-coded":
        assert cc["params"] == 2 and cc["decodes"] == s["misses"]
        assert cc["decodes_staged"] == sc["hits"]
        assert 0.7 * over_link < cc["link_bytes"] < 0.8 * over_link
    else:
        assert cc["params"] == 0 and cc["decodes"] == 0
        assert cc["link_bytes"] == over_link
    off.close()


def test_add_param_takes_only_whole_runtime_allocations():
    """A device layer copies its rows with the SDMA engines, which neither
    stage pageable memory nor check bounds: sluice_layer_add_param refuses a
    host store that is not a runtime allocation or is smaller than local_n
    rows (the check is against allocations: a tensor inside a larger cached
    device block passes), and takes exact-size pinned and device buffers."""
    import ctypes
    from sluice_amd import _lib, ops

    lib = _lib.load()
    E, S, row = 16, 8, 1 << 20
    emap = torch.full((E,), -1, dtype=torch.int32, device=DEV)
    h = ctypes.c_void_p()
    assert lib.sluice_layer_create(E, E, S, S // 2, _lib.int32_array(range(E)), emap.data_ptr(),
                                   ctypes.byref(h)) == 0
    try:
        slots = torch.empty((S, row), dtype=torch.uint8, device=DEV)
        pinned = ops.HostStore((E, row), torch.uint8)
        half = ops.HostStore((E // 2, row), torch.uint8)
        pageable = np.zeros((E, row), dtype=np.uint8)
        bad = _lib.SLUICE_E_INVAL
        assert lib.sluice_layer_add_param(h, slots.data_ptr(), pageable.ctypes.data, row) == bad
        assert lib.sluice_layer_add_param(h, slots.data_ptr(), half.data_ptr(), row) == bad
        assert lib.sluice_layer_add_param(h, slots.data_ptr(), pinned.data_ptr(), row) == 0
    finally:
        assert lib.sluice_layer_destroy(h) == 0


def test_resync_restores_the_pulled_rows_of_every_cached_slot(monkeypatch):
    """The gap kernel copies an fp8 layer's scale rows into the slots it
    fills; a gap the host answered but the device never installed (its wait
    ended first) would leave them out, and the resync after such a failure
    copies them again for every slot the cache holds.  Forced from the host:
    after a few served gaps the slots' scale rows are zeroed, and
    sluice_layer_gap_resync brings back every cached slot's host rows."""
    from sluice_amd import _lib

    E, S, k = 64, 16, 4
    print("resync re-pulls scale rows", flush=True)
    layer = _Fp8Layer(E, 512, 256)
    off = _offloader(monkeypatch, S, 0.5, False)
    off.wrap_modules(iter([layer]))
    with torch.cuda.device(DEV):
        off.post_init()
    cache = off._caches[id(layer)]
    off._rs_caches.append(cache)
    lib = _lib.load()
    assert lib.sluice_layer_pulled_params(cache.handle) == 2
    hs = torch.zeros((2, 512), dtype=torch.bfloat16, device=DEV)
    rng = np.random.default_rng(5)
    for _ in range(4):
        ids = torch.from_numpy(rng.choice(E, 2 * k, replace=False).astype(np.int32)).to(DEV)
        torch.ops.vllm.sluice_stream_gap(hs, ids.view(-1, k), 0)
    torch.cuda.synchronize()
    _slot_bytes_match_host(cache)
    cached = [s for s, loc in enumerate(cache.expert_in_slot) if loc is not None]
    assert len(cached) >= 8
    for name in ("w13_weight_scale", "w2_weight_scale"):
        cache.gpu_cache[name].zero_()
    torch.cuda.synchronize()
    assert lib.sluice_layer_gap_resync(cache.handle) == 0
    _slot_bytes_match_host(cache)
    off.close()


@pytest.mark.parametrize("mode", ["abort", "timeout"])
def test_unserved_gap_wait_ends_and_resync_resumes(monkeypatch, mode):
    """Failure handling forced from the host: a gap whose ids miss is
    launched and never served, with the process-wide abort flag raised
    ("abort") or the wait bound set to 0.3 s ("timeout").  The device wait
    ends by itself (the stream completes), the device map and the host's slot
    state stay as they were, and the layer reports SLUICE_E_ABORTED or
    SLUICE_E_TIMEOUT.  After the flag or bound is restored and the layer
    resynchronised, later gaps assign slots exactly as an oracle that never
    saw the failed step."""
    import time

    from oracle.slru import LayerCache
    from sluice_amd import _lib

    E, S, k = 64, 16, 4
    print(f"unserved gap: {mode}", flush=True)
    layer = _Layer(E, E)
    off = _offloader(monkeypatch, S, 0.5, False)
    off.wrap_modules(iter([layer]))
    with torch.cuda.device(DEV):
        off.post_init()
    cache = off._caches[id(layer)]
    off._rs_caches.append(cache)
    lib = _lib.load()
    oracle = LayerCache(E, E, S, 0.5)
    hs = torch.zeros((2, 64), dtype=torch.bfloat16, device=DEV)
    rng = np.random.default_rng(5)

    def served_step():
        ids_np = rng.choice(E, 2 * k, replace=False).astype(np.int32)
        torch.ops.vllm.sluice_stream_gap(hs, torch.from_numpy(ids_np).to(DEV).view(-1, k), 0)
        oracle.gap(ids_np.tolist(), fast_hit=False)
        torch.cuda.synchronize()
        assert cache._state()["expert_in_slot"] == [
            -1 if v is None else v for v in oracle.expert_in_slot]
        assert cache.expert_map_buf.cpu().tolist() == oracle.map

    for _ in range(3):
        served_step()
    map_before = cache.expert_map_buf.cpu().tolist()
    state_before = cache._state()
    missing = np.array([g for g in range(E) if map_before[g] < 0][:2 * k], dtype=np.int32)
    ids = torch.from_numpy(missing).to(DEV).view(-1, k)
    st = torch.cuda.current_stream(DEV).cuda_stream
    if mode == "abort":
        assert lib.sluice_gap_abort(1) == 0
    else:
        assert lib.sluice_gap_set_timeout(0.3) == 0
    try:
        t0 = time.time()
        _lib.check(lib.sluice_layer_gap_launch(cache.handle, ids.data_ptr(), ids.numel(), None,
                                               None, 0, None, st), "sluice_layer_gap_launch")
        torch.cuda.synchronize()
        waited = time.time() - t0
        print(f"  device wait ended after {waited:.3f} s", flush=True)
        assert waited < 10.0  # the default bound is 20 s
        if mode == "timeout":
            assert waited >= 0.25
        want = _lib.SLUICE_E_ABORTED if mode == "abort" else _lib.SLUICE_E_TIMEOUT
        assert lib.sluice_layer_gap_serve(cache.handle, 0, st) == want
    finally:
        lib.sluice_gap_abort(0)
        lib.sluice_gap_set_timeout(0.0)
    assert cache.expert_map_buf.cpu().tolist() == map_before
    after = cache._state()
    for key in ("expert_in_slot", "probation", "protected", "free_slots"):
        assert after[key] == state_before[key], key
    assert lib.sluice_layer_gap_resync(cache.handle) == 0
    for _ in range(6):
        served_step()
    off.close()


def test_server_overflow_raises_at_drain_and_reset_resumes(monkeypatch):
    """With the gap server serving the records, a step whose working set
    exceeds the slots makes drain() raise the reference's overflow error;
    the device map stays as it was and the host keeps the reference's
    partial acquisition.  reset_gaps() then brings the layer back: later
    gaps follow the oracle again."""
    from oracle.slru import GapOverflow, LayerCache

    E, S, k = 64, 16, 4
    print("gap server overflow + reset", flush=True)
    layer = _Layer(E, E)
    off = _offloader(monkeypatch, S, 0.5, False)
    off.wrap_modules(iter([layer]))
    with torch.cuda.device(DEV):
        off.post_init()
    cache = off._caches[id(layer)]
    off._rs_caches.append(cache)
    off.start_gap_server()
    oracle = LayerCache(E, E, S, 0.5)
    rng = np.random.default_rng(9)

    def step(T, expect_overflow=False):
        ids_np = rng.choice(E, T * k, replace=False).astype(np.int32)
        hs = torch.zeros((T, 64), dtype=torch.bfloat16, device=DEV)
        torch.ops.vllm.sluice_stream_gap(hs, torch.from_numpy(ids_np).to(DEV).view(-1, k), 0)
        if expect_overflow:
            with pytest.raises(RuntimeError, match="exceeds slots"):
                off.drain()
            with pytest.raises(GapOverflow):
                oracle.gap(ids_np.tolist(), fast_hit=False)
        else:
            off.drain()
            oracle.gap(ids_np.tolist(), fast_hit=False)
        st = cache._state()
        assert st["expert_in_slot"] == [-1 if v is None else v for v in oracle.expert_in_slot]
        assert st["probation"] == list(oracle.probation)
        assert st["protected"] == list(oracle.protected)

    for _ in range(4):
        step(2)
        assert cache.expert_map_buf.cpu().tolist() == oracle.map
    map_before = cache.expert_map_buf.cpu().tolist()
    step(5, expect_overflow=True)  # 20 unique experts > 16 slots
    assert cache.expert_map_buf.cpu().tolist() == map_before
    off.reset_gaps()
    # the reference's map variable still holds the map before the overflow,
    # whose slots the partial acquisition has refilled; the resync installs
    # the host's standing map on the device instead
    oracle.map = oracle.standing_map()
    assert cache.expert_map_buf.cpu().tolist() == oracle.map
    for _ in range(5):
        step(2)
        assert cache.expert_map_buf.cpu().tolist() == oracle.map
    _check_slots(cache, layer)
    off.close()


@pytest.mark.parametrize("fast_hit", [False, True])
def test_device_gap_with_no_tokens(monkeypatch, fast_hit):
    """A step with no tokens (an empty batch reaching the gap op): the op
    returns an empty fresh tensor; before the first standing map the empty
    step still installs one (src/sluice/offloader.py:2427-2467 with an empty
    sorted set: no touch, no fill, the standing map written), after it the
    step changes nothing -- slots, segments, counters and the device map
    follow the oracle through empty steps mixed with routed ones."""
    from oracle.slru import LayerCache
    from sluice_amd import _lib

    E, local_n, k, S = 16, 16, 2, 6
    layer = _Layer(E, local_n)
    off = _offloader(monkeypatch, S, 0.5, fast_hit)
    off.wrap_modules(iter([layer]))
    with torch.cuda.device(DEV):
        off.post_init()
    cache = off._caches[id(layer)]
    off._rs_caches.append(cache)
    cache.plan = torch.zeros(_lib.load().sluice_moe_plan_ints(1, cache.num_slots),
                             dtype=torch.int32, device=DEV)
    oracle = LayerCache(E, local_n, S, 0.5)
    rng = np.random.default_rng(5)
    schedule = [0, 0, 3, 0, 2, 0, 0, 3, 1, 0]  # T*k <= S: within the envelope
    for n, T in enumerate(schedule):
        ids_np = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32) \
            if T else np.zeros((0, k), np.int32)
        ids = torch.from_numpy(ids_np).to(DEV)
        hs = torch.randn((T, 64), device=DEV).to(torch.bfloat16)
        out = torch.ops.vllm.sluice_stream_gap(hs, ids, 0)
        assert out.shape == hs.shape and (T == 0 or out.data_ptr() != hs.data_ptr())
        assert torch.equal(out, hs)
        oracle.gap(ids_np.reshape(-1).tolist(), fast_hit=fast_hit)
        torch.cuda.synchronize()
        st = cache._state()
        assert st["expert_in_slot"] == [-1 if v is None else v for v in oracle.expert_in_slot], n
        assert st["probation"] == list(oracle.probation), n
        assert st["protected"] == list(oracle.protected), n
        assert st["counters"][:3] == [oracle.gaps, oracle.misses, oracle.fast_hits], n
        assert cache.expert_map_buf.cpu().tolist() == oracle.map, n
    _check_slots(cache, layer)
    off.close()


def test_failed_stream_in_drops_unlanded_fills_and_resync_installs_host_map(monkeypatch):
    """Failure handling forced from the host: in a gap whose 8 ids all miss
    (Qwen3-sized experts, two row copies each, one completion signal per
    expert), the 13th row copy -- the first of the seventh expert -- is made
    to fail (sluice_gap_inject_copy_failure).  The inline gap reports the
    error; the device waited for nothing (its slots were marked ready); the
    six experts seen to land stay cached and hold their host rows, the last
    two leave the host's slot cache (their slots free, taken next).  sluice_layer_gap_resync then writes the host's
    standing map into the device map, and later gaps -- selecting the
    dropped experts again -- follow the oracle after the same drops."""
    from oracle.slru import LayerCache
    from sluice_amd import _lib

    E, S, k, H, I = 32, 16, 4, 2048, 768
    print("failed stream-in: 8 misses, copy 13 fails", flush=True)
    layer = _Layer(E, E, H=H, I=I)
    off = _offloader(monkeypatch, S, 0.5, False)
    off.wrap_modules(iter([layer]))
    with torch.cuda.device(DEV):
        off.post_init()
    cache = off._caches[id(layer)]
    off._rs_caches.append(cache)
    lib = _lib.load()
    oracle = LayerCache(E, E, S, 0.5)
    hs = torch.zeros((2, 64), dtype=torch.bfloat16, device=DEV)
    rng = np.random.default_rng(21)

    def gap(ids_np):
        torch.ops.vllm.sluice_stream_gap(hs[: len(ids_np) // k],
                                         torch.from_numpy(ids_np).to(DEV).view(-1, k), 0)
        torch.cuda.synchronize()

    def check_state():
        st = cache._state()
        assert st["expert_in_slot"] == [-1 if v is None else v for v in oracle.expert_in_slot]
        assert st["probation"] == list(oracle.probation)
        assert st["protected"] == list(oracle.protected)
        assert st["free_slots"] == list(oracle.free_slots)

    for _ in range(2):
        ids_np = rng.choice(E, 2 * k, replace=False).astype(np.int32)
        gap(ids_np)
        oracle.gap(ids_np.tolist())
        check_state()
    m = cache.expert_map_buf.cpu().tolist()
    missing = np.array([g for g in range(E) if m[g] < 0][:2 * k], dtype=np.int32)
    assert len(missing) == 2 * k
    assert lib.sluice_gap_inject_copy_failure(12) == 0
    try:
        with pytest.raises(RuntimeError):
            gap(missing)
    finally:
        lib.sluice_gap_inject_copy_failure(-1)
    streams = oracle.gap(missing.tolist())
    assert len(streams) == 8
    for _, slot in streams[6:]:  # the fills whose rows did not land
        assert oracle.unfill(slot)
    check_state()
    assert lib.sluice_layer_gap_resync(cache.handle) == 0
    # the device map is now the host's standing map
    oracle.map, oracle.map_is_standing = oracle.standing_map(), True
    assert cache.expert_map_buf.cpu().tolist() == oracle.map
    _check_slots(cache, layer)
    dropped = [oracle.global_of_local[loc] for loc, _ in streams[6:]]
    for n in range(5):
        if n == 0:  # the dropped experts are selected again: they miss and stream
            others = rng.permutation([g for g in range(E) if g not in dropped])
            ids_np = np.array(dropped + others[: 2 * k - len(dropped)].tolist(), np.int32)
        else:
            ids_np = rng.choice(E, 2 * k, replace=False).astype(np.int32)
        gap(ids_np)
        oracle.gap(ids_np.tolist())
        check_state()
        assert cache.expert_map_buf.cpu().tolist() == oracle.map, n
    _check_slots(cache, layer)
    off.close()


@pytest.mark.parametrize("coded", [False, True], ids=["rows", "coded"])
def test_failed_stream_in_with_staged_misses_keeps_what_landed(monkeypatch, coded):
    """Failure handling with staged rows, forced from the host.  Under the
    gap server with four staging rows and a plain LRU (no protected
    segment), eight experts X are selected four times, then evicted by
    sixteen others: X are then the layer's most selected experts it does
    not hold, and the four lowest ids of X get staged.  A gap selecting X
    copies those four from HBM first, then the other four over the link;
    the 10th row copy (the second of the first expert over the link) is
    made to fail.  Coded: the staged experts are decoded from their rows
    (no copies), so the 2nd row copy is the one that fails.  The gap reports the error, the four staged experts were
    served from their rows and stay cached with their host rows, the other
    four leave the slot cache; after reset_gaps later gaps follow the
    oracle with the same drops."""
    import time

    from oracle.slru import LayerCache
    from sluice_amd import _lib

    E, S, k, H, I = 32, 16, 4, 2048, 768
    print(f"failed stream-in with staged misses coded={coded}", flush=True)
    monkeypatch.setenv("SLUICE_STAGE_ROWS", "4")
    monkeypatch.setenv("SLUICE_CODEC", "1" if coded else "0")
    layer = _Layer(E, E, H=H, I=I)
    off = _offloader(monkeypatch, S, 0.0, False)
    off.wrap_modules(iter([layer]))
    with torch.cuda.device(DEV):
        off.post_init()
    cache = off._caches[id(layer)]
    off._rs_caches.append(cache)
    off.start_gap_server()
    lib = _lib.load()
    oracle = LayerCache(E, E, S, 0.0)
    hs = torch.zeros((2, 64), dtype=torch.bfloat16, device=DEV)
    rng = np.random.default_rng(5)

    def gap(ids_np):
        torch.ops.vllm.sluice_stream_gap(hs[: len(ids_np) // k],
                                         torch.from_numpy(ids_np).to(DEV).view(-1, k), 0)
        off.drain()

    def check_state():
        st = cache._state()
        assert st["expert_in_slot"] == [-1 if v is None else v for v in oracle.expert_in_slot]
        assert st["probation"] == list(oracle.probation)
        assert st["free_slots"] == list(oracle.free_slots)

    perm = rng.permutation(E).astype(np.int32)
    x, others = perm[:8], perm[8:24]
    for ids_np in [x] * 4 + [others[:8], others[8:]]:
        gap(ids_np)
        oracle.gap(ids_np.tolist())
        check_state()
    assert all(oracle.slot_of.get(int(g)) is None for g in x)
    t0 = time.monotonic()
    while off.stage_counters()["ready"] < 4 and time.monotonic() - t0 < 5.0:
        time.sleep(0.001)
    assert off.stage_counters()["ready"] == 4
    assert lib.sluice_gap_inject_copy_failure(1 if coded else 9) == 0
    try:
        with pytest.raises(RuntimeError):
            gap(np.sort(x))
    finally:
        lib.sluice_gap_inject_copy_failure(-1)
    streams = oracle.gap(np.sort(x).tolist())
    assert len(streams) == 8
    for _, slot in streams[4:]:  # over the link: the first of them failed, none landed
        assert oracle.unfill(slot)
    check_state()
    assert off.stage_counters()["hits"] == 4
    if coded:
        assert off.codec_counters()["decodes_staged"] == 4
    off.reset_gaps()
    oracle.map, oracle.map_is_standing = oracle.standing_map(), True
    assert cache.expert_map_buf.cpu().tolist() == oracle.map
    _slot_bytes_match_host(cache)
    for n in range(6):
        ids_np = rng.choice(E, 2 * k, replace=False).astype(np.int32)
        gap(ids_np)
        oracle.gap(ids_np.tolist())
        check_state()
        assert cache.expert_map_buf.cpu().tolist() == oracle.map, n
    _slot_bytes_match_host(cache)
    off.close()


def test_wait_bound_set_after_capture_applies_to_replays(monkeypatch):
    """The bound of the gap's device waits is read when a wait begins, so a
    hipGraph captured under the default bound (20 s) follows a bound set
    after the capture: a captured gap whose ids miss, replayed unserved
    after sluice_gap_set_timeout(0.3), ends its wait after ~0.3 s and
    reports SLUICE_E_TIMEOUT; after a resync the layer follows the oracle.
    (A host timer raises the abort flag after 5 s, so the replay ends even
    if the new bound were not read.)"""
    import threading
    import time

    from oracle.slru import LayerCache
    from sluice_amd import _lib

    E, S, k = 64, 16, 4
    print("captured gap, bound set after capture", flush=True)
    layer = _Layer(E, E)
    off = _offloader(monkeypatch, S, 0.5, False)
    off.wrap_modules(iter([layer]))
    with torch.cuda.device(DEV):
        off.post_init()
    cache = off._caches[id(layer)]
    off._rs_caches.append(cache)
    lib = _lib.load()
    oracle = LayerCache(E, E, S, 0.5)
    hs = torch.zeros((2, 64), dtype=torch.bfloat16, device=DEV)
    rng = np.random.default_rng(8)

    def served_step():
        ids_np = rng.choice(E, 2 * k, replace=False).astype(np.int32)
        torch.ops.vllm.sluice_stream_gap(hs, torch.from_numpy(ids_np).to(DEV).view(-1, k), 0)
        oracle.gap(ids_np.tolist(), fast_hit=False)
        torch.cuda.synchronize()
        assert cache.expert_map_buf.cpu().tolist() == oracle.map

    for _ in range(3):
        served_step()
    m = cache.expert_map_buf.cpu().tolist()
    ids = torch.from_numpy(np.array([g for g in range(E) if m[g] < 0][:2 * k],
                                    dtype=np.int32)).to(DEV).view(-1, k)
    stream = torch.cuda.Stream(device=DEV)
    stream.wait_stream(torch.cuda.current_stream(DEV))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        _lib.check(lib.sluice_layer_gap_launch(cache.handle, ids.data_ptr(), ids.numel(), None,
                                               None, 0, None, stream.cuda_stream),
                   "sluice_layer_gap_launch")
    torch.cuda.synchronize()
    backstop = threading.Timer(5.0, lambda: lib.sluice_gap_abort(1))
    assert lib.sluice_gap_set_timeout(0.3) == 0
    try:
        backstop.start()
        t0 = time.time()
        g.replay()
        torch.cuda.synchronize()
        waited = time.time() - t0
        backstop.cancel()
        print(f"  replayed wait ended after {waited:.3f} s", flush=True)
        assert 0.25 <= waited < 4.0
        rc = lib.sluice_layer_gap_serve(cache.handle, 0, torch.cuda.current_stream(DEV).cuda_stream)
        assert rc == _lib.SLUICE_E_TIMEOUT
    finally:
        backstop.cancel()
        lib.sluice_gap_abort(0)
        lib.sluice_gap_set_timeout(0.0)
    del g
    assert cache.expert_map_buf.cpu().tolist() == oracle.map
    assert lib.sluice_layer_gap_resync(cache.handle) == 0
    for _ in range(4):
        served_step()
    off.close()
