"""The native (C++) slot cache reproduces the reference's slot assignment bit
for bit: against the golden vectors and against the oracle on long random
traces (host path of libsluice_hip.so; no GPU work)."""

import random

import pytest

from native_cache import NativeCache
from oracle.slru import GapOverflow, LayerCache


def _native_for(case):
    c = NativeCache(case["E"], case["local_n"], case["slots"], case["protect_frac"],
                    local_of=case["local_of"])
    lof = case["local_of"] or list(range(case["E"]))
    cap = c.state()["protected_cap"]
    for g in case["pins"] or []:
        loc = lof[g]
        if loc >= 0 and cap > 0 and c.pin(loc, debit=True) is not None:
            cap -= 1
    return c


@pytest.mark.parametrize("idx", range(20))
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
