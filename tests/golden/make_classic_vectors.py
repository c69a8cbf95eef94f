"""Write golden vectors for the classic (wave) step of the slot cache.

Runs the reference's own ExpertStreamOffloader on the CPU, in this
container only: _install_cache, then a trace that mixes router-split gap
steps (T <= thr: _router_split_gap, src/sluice/offloader.py:2362-2467) with
classic steps (T > thr or non-decode steps: run_moe, 1452-1765, and
_run_waves, 1846-1933).  For every classic step it records the map each wave
ran with (read by the stand-in kernel at call time), the stream-ins issued
before each wave, and the full cache state after the step.  The output JSON
holds data only; the reference never leaves this container.

Three more traces run with the opt-in policies the classic hook carries:
SLUICE_LFU (frequency-ordered victims) and SLUICE_EXPERT_COUNTS (selection
counts and their JSONL snapshots); for those the LFU frequencies, step
classes and counts after every classic step, and the JSONL records the
reference itself wrote (timestamps dropped), are kept too.

Stand-ins, beyond the three vLLM names make_slru_vectors.py supplies:
  - the kernel (`original_apply`) records the layer's expert map and returns
    a scalar zero tensor;
  - the forward-context signal (_split_signal) returns the step's
    (num_decode_tokens, num_decodes, is_real_step);
  - torch.cuda.current_stream / torch.cuda.Event, which _run_waves calls even
    without a copy stream, are no-op objects (CPU tensors: no copy stream, no
    events take part).

    python tests/golden/make_classic_vectors.py     # rewrites classic_vectors.json.gz
"""

import gzip
import json
import logging
import os
import shutil
import sys
import tempfile

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import make_slru_vectors as base  # noqa: E402  (stand-ins, fake module, traces)

OUT = os.path.join(HERE, "classic_vectors.json.gz")


class _NoopEvent:
    def record(self, *a, **k):
        pass

    def synchronize(self):
        pass


class _NoopStream:
    def wait_event(self, *a, **k):
        pass

    def wait_stream(self, *a, **k):
        pass


# signal schedules for the classic steps: (nd, ndec, real_step) given T
SIGNALS = {
    "decode": lambda T, i: (T, T, True),
    "prefill": lambda T, i: (0, 0, True),
    "mixed": lambda T, i: (T // 2, T // 2, True),
    "extend": lambda T, i: (T // 2 + 1, T // 2, True),   # nd > ndec: forced scan
    "nonmla": lambda T, i: (None, None, True),            # real step, no split published
    "dummy": lambda T, i: (None, None, False),
    "cycle": lambda T, i: [(T, T, True), (0, 0, True), (T // 2, T // 2, True),
                           (None, None, True), (T // 2 + 1, T // 2, True)][i % 5],
}

CASES = [
    # name, E, local_n, slots, frac, k, T choices, steps, trace kind, seed, ep, pins, signal
    ("tiny_waves_decode", 16, 16, 4, 0.5, 2, [1, 2, 6], 120, "uniform", 111, None, None,
     "decode"),
    ("tiny_waves_cycle", 16, 16, 4, 0.5, 2, [1, 2, 6, 9], 150, "uniform", 112, None, None,
     "cycle"),
    ("tiny_prefill", 16, 16, 6, 0.5, 2, [1, 3, 12], 120, "uniform", 113, None, None, "prefill"),
    ("tiny_pins_frac09", 32, 32, 8, 0.9, 3, [1, 2, 8], 150, "zipf", 114, None, [3, 4, 5, 6],
     "cycle"),
    ("ep_half_owned", 32, 16, 6, 0.5, 4, [1, 6], 120, "uniform", 115, "even", None, "cycle"),
    ("v2lite_c12", 64, 64, 48, 0.5, 6, [8, 12], 120, "zipf", 121, None, None, "decode"),
    ("qwen3_s64_c12", 128, 128, 64, 0.5, 8, [8, 12], 120, "zipf", 131, None, None, "decode"),
    ("qwen3_s32_scan", 128, 128, 32, 0.5, 8, [4, 16], 80, "uniform", 132, None, None, "cycle"),
    ("nonmla_dummy", 32, 32, 8, 0.5, 2, [2, 5], 100, "uniform", 141, None, None, "nonmla"),
    ("dummy_runs", 32, 32, 8, 0.5, 2, [2, 5], 100, "uniform", 142, None, None, "dummy"),
]

# Opt-in policies: SLUICE_LFU (frequency-ordered demotion and protected
# victims, aged every 256 real classic steps) and SLUICE_EXPERT_COUNTS
# (per-expert selection counts, JSONL snapshots every `every` hook calls).
POLICY_CASES = [
    # name, E, local_n, slots, frac, k, T choices, steps, trace, seed, ep, pins, signal, policy
    ("lfu_cycle", 24, 24, 8, 0.5, 2, [1, 2, 6, 9], 700, "zipf", 151, None, None, "cycle",
     {"lfu": True, "counts_every": 37}),
    ("lfu_decode_pins", 32, 32, 10, 0.6, 3, [1, 4, 8], 450, "zipf", 152, None, [2, 9], "decode",
     {"lfu": True}),
    ("counts_ep", 32, 16, 6, 0.5, 4, [1, 6], 160, "uniform", 153, "even", None, "cycle",
     {"counts_every": 23}),
]


def _policy_state(off, cache, mod):
    out = {"freq": sorted([int(l), int(c)] for l, c in cache.freq.items()),
           "lfu_steps": int(cache.lfu_steps),
           "steps_small": int(off._stats["small"].steps),
           "steps_scan": int(off._stats["scan"].steps)}
    cnt = off._counts.get(id(mod))
    if cnt is not None:
        out["counts_decode"] = [int(v) for v in cnt[0]]
        out["counts_scan"] = [int(v) for v in cnt[1]]
    return out


def run_case(ESO, name, E, local_n, slots, frac, k, T_choices, steps, kind, seed, ep, pins,
             signal, policy=None):
    policy = policy or {}
    os.environ["SLUICE_PROTECT_FRAC"] = str(frac)
    counts_dir = None
    for key in ("SLUICE_LFU", "SLUICE_EXPERT_COUNTS", "SLUICE_EXPERT_COUNTS_EVERY"):
        os.environ.pop(key, None)
    if policy.get("lfu"):
        os.environ["SLUICE_LFU"] = "1"
    if policy.get("counts_every"):
        counts_dir = tempfile.mkdtemp(prefix="sluice_counts_")
        os.environ["SLUICE_EXPERT_COUNTS"] = counts_dir
        os.environ["SLUICE_EXPERT_COUNTS_EVERY"] = str(policy["counts_every"])
    off = ESO(expert_cache_slots=slots)
    emap = None
    local_of = None
    if ep == "even":
        local_of = [-1] * E
        for g in range(0, E, 2):
            local_of[g] = g // 2
        emap = torch.tensor(local_of, dtype=torch.int32)
    if pins:
        off._pin_layers = {0: list(pins)}
    mod = base._FakeMoE(E, local_n, emap)
    off._install_cache(mod)
    cache = off._caches[id(mod)]
    off._rs_caches = [cache]
    off._rs_fast_hit = True
    thr = max(1, cache.num_slots // k)

    waves = []  # per classic step: [{"pairs": [...], "streams": [...]}]

    def rec_stream_in(c, local, slot, cs, on_stream=False):
        if waves:  # inside a classic step (gap steps' stream-ins are in the state)
            waves[-1]["streams"].append([int(local), int(slot)])
        for name_, gpu in c.gpu_cache.items():
            gpu[slot].copy_(c.cpu_store[name_][local])

    def fake_apply(*a, **kw):
        m = cache.expert_map_buf.tolist()
        waves[-1]["pairs"] = [[g, int(s)] for g, s in enumerate(m) if s >= 0]
        waves.append({"pairs": None, "streams": []})
        return torch.zeros(1)

    off._stream_in = rec_stream_in
    trace = base._trace(kind, E, k, T_choices, steps, seed)
    init = base._snapshot(cache)
    recs = []
    n_classic = 0
    for ids in trace:
        T = len(ids) // k
        t = torch.tensor(ids, dtype=torch.int64).view(T, k)
        if T <= thr:
            overflow = False
            try:
                off._router_split_gap(0, t)
            except RuntimeError:
                overflow = True
            recs.append({"kind": "gap", "ids": ids, "T": T, "overflow": overflow,
                         "state": base._snapshot(cache)})
            if overflow:
                break
            continue
        nd, ndec, real = SIGNALS[signal](T, n_classic)
        n_classic += 1
        type(off)._split_signal = staticmethod(lambda nd=nd, ndec=ndec, real=real:
                                               (nd, ndec, real))
        waves.clear()
        waves.append({"pairs": None, "streams": []})
        off.run_moe(fake_apply, (), {}, mod, t)
        waves.pop()  # the slot opened after the last kernel
        rec_waves = [dict(w) for w in waves]
        waves.clear()
        for s, loc in enumerate(cache.expert_in_slot):
            if loc is not None:
                assert float(cache.gpu_cache["w13_weight"][s, 0, 0]) == float(loc)
        recs.append({"kind": "classic", "ids": ids, "T": T, "nd": nd, "ndec": ndec,
                     "real_step": real, "waves": rec_waves,
                     "state": base._snapshot(cache),
                     # the reference's per-class step stats after this step
                     "stats": {kind_: {k_: int(v) for k_, v in st.items()}
                               for kind_, st in off.get_stats().items()},
                     "bytes_per_expert": int(cache.bytes_per_expert)})
        if policy:
            recs[-1]["policy"] = _policy_state(off, cache, mod)
    out = {
        "name": name, "E": E, "local_n": local_n, "slots": slots, "protect_frac": frac,
        "k": k, "local_of": local_of, "pins": pins, "thr": thr, "signal": signal,
        "init": init, "steps": recs,
    }
    if policy:
        out["policy"] = policy
    if counts_dir is not None:
        # the reference's own periodic snapshots so far (the atexit one is
        # not taken): the JSONL record format, "ts" dropped
        if off._counts_file is not None:
            off._counts_file.close()
            off._counts_file = None
        off._counts_dir = None  # its atexit hook then writes nothing
        lines = []
        for fn in sorted(os.listdir(counts_dir)):
            with open(os.path.join(counts_dir, fn)) as f:
                for line in f:
                    rec = json.loads(line)
                    rec.pop("ts", None)
                    lines.append({"file": fn, "record": rec})
        out["counts_jsonl"] = lines
        shutil.rmtree(counts_dir, ignore_errors=True)
    return out


def main():
    base._install_vllm_standins()
    sys.path.insert(0, base.REF_SRC)
    from sluice.offloader import ExpertStreamOffloader  # the reference, read from REF_SRC

    torch.cuda.current_stream = lambda *a, **k: _NoopStream()
    torch.cuda.Event = lambda *a, **k: _NoopEvent()
    logging.getLogger("sluice").setLevel(logging.ERROR)
    cases = [run_case(ExpertStreamOffloader, *case) for case in CASES]
    cases += [run_case(ExpertStreamOffloader, *case) for case in POLICY_CASES]
    with gzip.open(OUT, "wt") as f:
        json.dump({"source": "src/sluice/offloader.py _install_cache + _router_split_gap + "
                             "run_moe/_run_waves", "cases": cases}, f, separators=(",", ":"))
    n_cl = sum(1 for c in cases for s in c["steps"] if s["kind"] == "classic")
    n_wv = sum(len(s["waves"]) for c in cases for s in c["steps"] if s["kind"] == "classic")
    print(f"wrote {OUT}: {len(cases)} traces, {sum(len(c['steps']) for c in cases)} steps, "
          f"{n_cl} classic steps, {n_wv} waves")


if __name__ == "__main__":
    main()
