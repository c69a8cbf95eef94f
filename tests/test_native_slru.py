"""The native (C++) slot cache reproduces the reference's slot assignment bit
for bit: against the golden vectors and against the oracle on long random
traces (host path of libsluice_hip.so; no GPU work)."""

import ctypes
import random

import pytest

from native_cache import NativeCache
from sluice_amd import _lib
from oracle.slru import GapOverflow, LayerCache


def _native_for(case):
    pol = case.get("policy", {})
    c = NativeCache(case["E"], case["local_n"], case["slots"], case["protect_frac"],
                    local_of=case["local_of"], lfu=bool(pol.get("lfu")),
                    counts=bool(pol.get("counts_every")))
    lof = case["local_of"] or list(range(case["E"]))
    cap = c.state()["protected_cap"]
    for g in case["pins"] or []:
        loc = lof[g]
        if loc >= 0 and cap > 0 and c.pin(loc, debit=True) is not None:
            cap -= 1
    return c


def _slru_cases():
    from tests.conftest import slru_vectors

    return range(len(slru_vectors()["cases"]))


@pytest.mark.parametrize("idx", _slru_cases())
def test_native_matches_reference_vectors(slru_golden, idx):
    case = slru_golden["cases"][idx]
    c = _native_for(case)
    st = c.state()
    for key in ("slot_of", "expert_in_slot", "probation", "protected", "free_slots",
                "protected_cap"):
        assert st[key] == case["init"][key], key
    for n, step in enumerate(case["steps"]):
        streams, overflow = c.gap(step["ids"], fast_hit=case["fast_hit"])
        assert overflow == step["overflow"], n
        if not overflow:
            assert streams == step["streams"], n
        st = c.state()
        want = step["state"]
        for key in ("slot_of", "expert_in_slot", "probation", "protected", "free_slots",
                    "map_is_standing", "protected_cap"):
            assert st[key] == want[key], (case["name"], n, key)
        if want["map_is_standing"]:
            assert st["standing_map"] == want["map"], (case["name"], n)
    cnt = c.state()["counters"]
    assert cnt["gaps"] == case["counters"]["gaps"]
    assert cnt["misses"] == case["counters"]["misses"]
    assert cnt["fast_hits"] == case["counters"]["fast_hits"]


@pytest.mark.parametrize("E,S,k,frac,seed", [
    (64, 48, 6, 0.5, 1), (128, 64, 8, 0.5, 2), (128, 96, 8, 0.3, 3), (256, 64, 8, 0.5, 4),
    (128, 32, 8, 0.9, 5), (1024, 512, 16, 0.5, 6),
])
def test_native_matches_oracle_long_random(E, S, k, frac, seed):
    rnd = random.Random(seed)
    o = LayerCache(E, E, S, frac)
    n = NativeCache(E, E, S, frac)
    hot = rnd.sample(range(E), min(E, 3 * S // 2))
    for step in range(1500):
        T = rnd.randint(1, max(1, S // k))
        pool = hot if rnd.random() < 0.8 else list(range(E))
        ids = [g for _ in range(T) for g in rnd.sample(pool, k)]
        fh = rnd.random() < 0.5
        try:
            ws = o.gap(ids, fast_hit=fh)
            oo = False
        except GapOverflow:
            oo = True
        ns, no = n.gap(ids, fast_hit=fh)
        assert oo == no
        if not oo:
            assert [list(x) for x in ws] == ns, step
        st = n.state()
        snap = o.snapshot()
        assert st["slot_of"] == snap["slot_of"]
        assert st["probation"] == snap["probation"]
        assert st["protected"] == snap["protected"]
        if oo:
            break


def test_full_residency_prefill_pins_every_slot():
    c = NativeCache(16, 16, 16, 0.5)
    for l in range(16):
        assert c.pin(l, debit=False) == l
    streams, overflow = c.gap(list(range(16)))
    assert streams == [] and not overflow
    st = c.state()
    assert st["probation"] == [] and st["protected"] == []
    assert st["standing_map"] == list(range(16))


# ---------------------------------------------------------------------------
# Classic (wave) steps
# ---------------------------------------------------------------------------
def _classic_vectors():
    from tests.conftest import classic_vectors

    return classic_vectors()


@pytest.mark.parametrize("idx", range(len(_classic_vectors()["cases"])))
def test_native_classic_matches_reference_vectors(classic_golden, idx):
    case = classic_golden["cases"][idx]
    c = _native_for(case)
    for key in ("slot_of", "expert_in_slot", "probation", "protected", "free_slots",
                "protected_cap"):
        assert c.state()[key] == case["init"][key], key
    for n, step in enumerate(case["steps"]):
        last_map = None
        if step["kind"] == "gap":
            _, overflow = c.gap(step["ids"], fast_hit=True)
            assert overflow == step["overflow"], n
        else:
            waves = c.classic(step["ids"], step["T"], step["nd"], step["ndec"],
                              step["real_step"])
            assert len(waves) == len(step["waves"]), (case["name"], n)
            for w, want in zip(waves, step["waves"]):
                assert sorted([list(p) for p in w["pairs"]]) == want["pairs"], (case["name"], n)
                assert [list(x) for x in w["streams"]] == want["streams"], (case["name"], n)
            last_map = [-1] * case["E"]
            for g, s in waves[-1]["pairs"]:
                last_map[g] = s
        st = c.state()
        want = step["state"]
        for key in ("slot_of", "expert_in_slot", "probation", "protected", "free_slots",
                    "map_is_standing", "protected_cap"):
            assert st[key] == want[key], (case["name"], n, key)
        if "stats" in step:
            got = c.step_stats()
            for kind, want_s in step["stats"].items():
                for key in ("steps", "hits", "misses", "waves"):
                    assert got[kind][key] == want_s[key], (case["name"], n, kind, key)
                assert want_s["bytes"] == want_s["misses"] * step["bytes_per_expert"]
        if "policy" in step:
            pol, want_pol = c.policy(), step["policy"]
            for key in ("freq", "lfu_steps", "steps_small", "steps_scan"):
                assert pol[key] == want_pol[key], (case["name"], n, key)
            if "counts_decode" in want_pol:
                assert pol["counts_decode"] == want_pol["counts_decode"], (case["name"], n)
                assert pol["counts_scan"] == want_pol["counts_scan"], (case["name"], n)
        if step.get("overflow"):
            break  # the reference raised: its map is left stale, and the trace ends
        if want["map_is_standing"]:
            assert st["standing_map"] == want["map"], (case["name"], n)
        elif last_map is not None:
            assert last_map == want["map"], (case["name"], n)


@pytest.mark.parametrize("E,S,k,frac,seed,lfu", [
    (64, 48, 6, 0.5, 7, False), (128, 64, 8, 0.5, 8, False), (128, 32, 8, 0.9, 9, False),
    (256, 64, 8, 0.3, 10, False), (64, 16, 6, 0.5, 11, True), (128, 64, 8, 0.7, 12, True)])
def test_native_classic_matches_oracle_long_random(E, S, k, frac, seed, lfu):
    rnd = random.Random(seed)
    o = LayerCache(E, E, S, frac, lfu=lfu, counts=True)
    n = NativeCache(E, E, S, frac, lfu=lfu, counts=True)
    hot = rnd.sample(range(E), min(E, 3 * S // 2))
    thr = max(1, S // k)
    for step in range(600):
        T = rnd.choice([rnd.randint(1, thr), rnd.randint(thr + 1, 4 * thr + 8)])
        pool = hot if rnd.random() < 0.7 else list(range(E))
        ids = [g for _ in range(T) for g in rnd.sample(pool, k)]
        if T <= thr and rnd.random() < 0.6:
            try:
                o.gap(ids, fast_hit=True)
                oo = False
            except GapOverflow:
                oo = True
            _, no = n.gap(ids, fast_hit=True)
            assert oo == no
            if oo:
                break
        else:
            sig = rnd.choice([(T, T, True), (0, 0, True), (T // 2, T // 2, True),
                              (T // 2 + 1, T // 2, True), (None, None, True),
                              (None, None, False)])
            ow = o.classic(ids, T, *sig)
            nw = n.classic(ids, T, *sig)
            assert [sorted(w["pairs"]) for w in ow] == [sorted(w["pairs"]) for w in nw], step
            assert [w["streams"] for w in ow] == [w["streams"] for w in nw], step
        st = n.state()
        snap = o.snapshot()
        for key in ("slot_of", "expert_in_slot", "probation", "protected", "free_slots"):
            assert st[key] == snap[key], (step, key)
        assert st["map_is_standing"] == snap["map_is_standing"]
        assert st["counters"]["misses"] == o.misses
        pol = n.policy()
        assert pol["freq"] == sorted([l, f] for l, f in o.freq.items())
        assert (pol["counts_decode"], pol["counts_scan"]) == o.counts
        assert (pol["steps_small"], pol["steps_scan"], pol["lfu_steps"]) == (
            o.steps_small, o.steps_scan, o.lfu_steps)


def test_native_classic_argument_checks():
    c = NativeCache(16, 16, 4, 0.5)
    lib, h = c.lib, c.h
    nw = ctypes.c_int()
    arr = _lib.int32_array([1, 2, 3])
    assert lib.sluice_layer_classic_host(h, arr, 3, 2, -1, -1, 1, 0, ctypes.byref(nw)) \
        == _lib.SLUICE_E_INVAL  # 3 ids are not [2, k]
    assert lib.sluice_layer_classic_host(h, arr, 3, 0, -1, -1, 1, 0, ctypes.byref(nw)) \
        == _lib.SLUICE_E_INVAL
    assert lib.sluice_layer_classic_host(h, None, 0, 0, -1, -1, 1, 0, ctypes.byref(nw)) \
        == _lib.SLUICE_OK and nw.value == 1
    # the device entry points need a device map
    assert lib.sluice_layer_classic_plan(h, arr, 3, 3, -1, -1, 1, 0, None, ctypes.byref(nw)) \
        == _lib.SLUICE_E_STATE
    assert lib.sluice_layer_classic_wave(h, 5, None) == _lib.SLUICE_E_STATE


@pytest.mark.parametrize("E,S,k,frac,seed", [(64, 48, 6, 0.5, 11), (128, 32, 8, 0.5, 12),
                                             (128, 64, 8, 0.0, 13)])
def test_unfill_after_failed_fills_matches_oracle(E, S, k, frac, seed):
    """Recovery from a stream-in whose rows did not land (the served gap drops
    every fill of a failed stream-in that was not seen to land): the dropped
    experts leave their segment and their slots go back on the free list
    (taken next), the map stops being standing, and later gaps -- which
    miss on the dropped experts and stream them again -- assign slots as the
    oracle does after the same drops.  A free or pinned slot is refused."""
    rnd = random.Random(seed)
    o = LayerCache(E, E, S, frac)
    n = NativeCache(E, E, S, frac)
    hot = rnd.sample(range(E), min(E, 3 * S // 2))
    dropped = 0
    for step in range(600):
        T = rnd.randint(1, max(1, S // k))
        ids = [g for _ in range(T) for g in rnd.sample(hot if rnd.random() < 0.8 else
                                                       list(range(E)), k)]
        ws = o.gap(ids, fast_hit=True)
        ns, _ = n.gap(ids, fast_hit=True)
        assert [list(x) for x in ws] == ns, step
        if ns and rnd.random() < 0.3:
            # the copies failed after the first `landed` fills
            landed = rnd.randint(0, len(ns) - 1)
            for _, slot in ns[landed:]:
                assert o.unfill(slot) and n.unfill(slot)
                dropped += 1
            assert not n.state()["map_is_standing"] and not o.map_is_standing
        st = n.state()
        snap = o.snapshot()
        for key in ("slot_of", "probation", "protected", "free_slots"):
            assert st[key] == snap[key], (step, key)
        assert st["map_is_standing"] == o.map_is_standing
        assert st["standing_map"] == o.standing_map()
    assert dropped > 20
    free = n.state()["free_slots"]
    if free:
        assert not n.unfill(free[0]) and not o.unfill(free[0])


def test_unfill_refuses_pinned_slots():
    o = LayerCache(16, 16, 8, 0.5)
    n = NativeCache(16, 16, 8, 0.5)
    s_o, s_n = o.pin(3), n.pin(3)
    assert s_o == s_n is not None
    assert not o.unfill(s_o) and not n.unfill(s_n)
    assert n.state()["expert_in_slot"][s_n] == 3
