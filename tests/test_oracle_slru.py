"""Pin the slot-cache oracle: golden vectors written by the reference's own
gap (tests/golden/make_slru_vectors.py), hand-worked traces and invariants."""

import random

import pytest

from conftest import slru_vectors
from oracle.slru import GapOverflow, LayerCache


def _oracle_for(case):
    c = LayerCache(case["E"], case["local_n"], case["slots"], case["protect_frac"],
                   local_of=case["local_of"])
    for g in case["pins"] or []:
        loc = c.local_of[g]
        if loc >= 0 and c.protected_cap > 0:
            c.pin(loc, debit_protected=True)
    return c


def _state(c):
    s = c.snapshot()
    s["protected_cap"] = c.protected_cap
    return s


def test_golden_cases_cover_both_fast_hit_settings(slru_golden):
    names = {(c["name"], c["fast_hit"]) for c in slru_golden["cases"]}
    assert len(names) == len(slru_golden["cases"]) >= 20
    assert any(c["steps"][-1]["overflow"] for c in slru_golden["cases"])


@pytest.mark.parametrize("idx", range(len(slru_vectors()["cases"])))
def test_oracle_matches_reference_vectors(slru_golden, idx):
    case = slru_golden["cases"][idx]
    c = _oracle_for(case)
    init = _state(c)
    for key in ("slot_of", "expert_in_slot", "probation", "protected", "free_slots",
                "protected_cap"):
        assert init[key] == case["init"][key], key
    for n, step in enumerate(case["steps"]):
        try:
            streams = c.gap(step["ids"], fast_hit=case["fast_hit"])
            overflow = False
        except GapOverflow:
            overflow = True
            streams = None
        assert overflow == step["overflow"], n
        if not overflow:
            assert [list(x) for x in streams] == step["streams"], n
        got = _state(c)
        for key, want in step["state"].items():
            assert got[key] == want, (case["name"], n, key)
    assert c.gaps == case["counters"]["gaps"]
    assert c.misses == case["counters"]["misses"]
    assert c.fast_hits == case["counters"]["fast_hits"]


def test_hand_worked_trace():
    # S=4, cap=2.  Free list pops slot 0 first; new entries are probationary;
    # a hit promotes into protected, demoting the protected LRU when full.
    c = LayerCache(8, 8, 4, 0.5)
    assert c.protected_cap == 2 and c.free_slots == [3, 2, 1, 0]
    assert c.gap([5, 2]) == [(2, 0), (5, 1)]          # sorted unique -> 2 then 5
    assert list(c.probation) == [0, 1] and c.map[2] == 0 and c.map[5] == 1
    assert c.gap([5]) == []                            # hit: slot 1 -> protected
    assert list(c.protected) == [1] and list(c.probation) == [0]
    assert c.gap([2, 5]) == []                         # slot 0 promoted, then 1 refreshed
    assert list(c.protected) == [0, 1]
    assert c.gap([7, 6]) == [(6, 2), (7, 3)]           # free slots 2, 3
    assert c.gap([3]) == [(3, 2)]                      # probation LRU (slot 2) evicted
    assert c.map[6] == -1 and c.map[3] == 2
    assert c.gap([3, 7]) == []                         # both hit: 2, 3 promoted, 0, 1 demoted
    assert list(c.protected) == [2, 3] and list(c.probation) == [0, 1]
    # hits 2, 3, 5 promote one by one (each demoting the protected LRU), so
    # probation ends [3, 0]; slot 3 (expert 7) is the first unclaimed victim
    assert c.gap([1, 2, 5, 3]) == [(1, 3)]
    assert list(c.protected) == [2, 1] and list(c.probation) == [0, 3]
    assert c.map[7] == -1 and c.map[1] == 3


def test_claimed_hits_never_evicted_and_overflow():
    c = LayerCache(16, 16, 3, 0.5)
    c.gap([0, 1, 2])
    with pytest.raises(GapOverflow):
        c.gap([0, 1, 2, 3])  # 4 unique > 3 slots: every victim is claimed


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_invariants_random(seed):
    rnd = random.Random(seed)
    E, S, k = 32, 12, 3
    c = LayerCache(E, E, S, 0.5)
    for _ in range(400):
        T = rnd.choice([1, 2, 3, 4])
        ids = [g for _ in range(T) for g in rnd.sample(range(E), k)]
        c.gap(ids, fast_hit=rnd.random() < 0.5)
        # every selected expert resident; map == residency; segments partition occupancy
        for g in ids:
            assert g in c.slot_of
        assert c.map == c.standing_map()
        for g in range(E):
            s = c.map[g]
            assert (s >= 0) == (g in c.slot_of)
            if s >= 0:
                assert c.expert_in_slot[s] == g
        occ = {s for s, v in enumerate(c.expert_in_slot) if v is not None}
        assert occ == set(c.protected) | set(c.probation)
        assert not (set(c.protected) & set(c.probation))
        assert len(c.protected) <= c.protected_cap
