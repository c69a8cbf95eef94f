"""Pin the classic (wave) step of the slot-cache oracle against golden
vectors written by the reference's own run_moe / _run_waves, driven on traces
that interleave router-split gaps with classic steps
(tests/golden/make_classic_vectors.py)."""

import pytest

from oracle.slru import GapOverflow, LayerCache
from tests.conftest import classic_vectors


def _oracle_for(case):
    pol = case.get("policy", {})
    c = LayerCache(case["E"], case["local_n"], case["slots"], case["protect_frac"],
                   local_of=case["local_of"], lfu=bool(pol.get("lfu")),
                   counts=bool(pol.get("counts_every")))
    for g in case["pins"] or []:
        loc = c.local_of[g]
        if loc >= 0 and c.protected_cap > 0:
            c.pin(loc, debit_protected=True)
    return c


def _state(c):
    s = c.snapshot()
    s["protected_cap"] = c.protected_cap
    return s


def test_golden_cases_exercise_waves_and_every_signal(classic_golden):
    cases = classic_golden["cases"]
    steps = [s for c in cases for s in c["steps"] if s["kind"] == "classic"]
    assert sum(1 for s in steps if len(s["waves"]) > 2) > 50       # multi-wave steps
    assert sum(1 for s in steps if len(s["waves"]) == 1) > 50      # single-wave steps
    signals = {(s["nd"] is None, s["real_step"], s["nd"] == s["T"] if s["nd"] is not None
                else None) for s in steps}
    assert len(signals) >= 4
    assert any(s["kind"] == "gap" for c in cases for s in c["steps"])
    # the opt-in policies: LFU aged at least once, counts with JSONL snapshots
    lfu = [c for c in cases if c.get("policy", {}).get("lfu")]
    assert lfu and all(any(s["policy"]["lfu_steps"] == 0 for s in c["steps"][50:]
                           if s["kind"] == "classic") for c in lfu)
    assert any(len(c.get("counts_jsonl", [])) >= 3 for c in cases)


@pytest.mark.parametrize("idx", range(len(classic_vectors()["cases"])))
def test_oracle_classic_matches_reference_vectors(classic_golden, idx):
    case = classic_golden["cases"][idx]
    c = _oracle_for(case)
    init = _state(c)
    for key in ("slot_of", "expert_in_slot", "probation", "protected", "free_slots",
                "protected_cap"):
        assert init[key] == case["init"][key], key
    for n, step in enumerate(case["steps"]):
        if step["kind"] == "gap":
            try:
                c.gap(step["ids"], fast_hit=True)
                overflow = False
            except GapOverflow:
                overflow = True
            assert overflow == step["overflow"], n
        else:
            waves = c.classic(step["ids"], step["T"], step["nd"], step["ndec"],
                              step["real_step"])
            assert len(waves) == len(step["waves"]), (case["name"], n)
            for w, want in zip(waves, step["waves"]):
                assert sorted([list(p) for p in w["pairs"]]) == want["pairs"], (case["name"], n)
                assert [list(x) for x in w["streams"]] == want["streams"], (case["name"], n)
        got = _state(c)
        for key, want in step["state"].items():
            assert got[key] == want, (case["name"], n, key)
        if "policy" in step:
            pol = step["policy"]
            assert sorted([l, f] for l, f in c.freq.items()) == pol["freq"], (case["name"], n)
            assert c.lfu_steps == pol["lfu_steps"], n
            assert (c.steps_small, c.steps_scan) == (pol["steps_small"], pol["steps_scan"]), n
            if "counts_decode" in pol:
                assert c.counts == (pol["counts_decode"], pol["counts_scan"]), (case["name"], n)


def test_classic_hand_worked_waves():
    # S=4 (cap 2), a 6-token decode step needing 12 experts: wave 0 takes the
    # 4 free slots; the 8 leftovers rotate through probation in two groups of 2.
    c = LayerCache(16, 16, 4, 0.5)
    waves = c.classic(list(range(12)), 6, nd=6, ndec=6)
    assert [w["pairs"] for w in waves] == [
        [(0, 0), (1, 1), (2, 2), (3, 3)], [(4, 0), (5, 1)], [(6, 2), (7, 3)],
        [(8, 0), (9, 1)], [(10, 2), (11, 3)]]
    assert c.expert_in_slot == [8, 9, 10, 11] and not c.map_is_standing
    assert c.map[10] == 2 and c.map[8] == -1          # the last wave's sparse map
    # scan-class (prefill) misses never take protected slots
    c = LayerCache(8, 8, 4, 0.5)
    c.gap([0]), c.gap([0]), c.gap([1]), c.gap([1])    # slots 0, 1 -> protected
    assert list(c.protected) == [0, 1]
    waves = c.classic([2, 3, 4, 5], 4, nd=0, ndec=0)  # 4 scan misses, 2 free slots
    assert waves[0]["streams"] == [(2, 2), (3, 3)]
    assert [w["pairs"] for w in waves[1:]] == [[(4, 2)], [(5, 3)]]
    assert list(c.protected) == [0, 1]                # the decode-hot set survives
