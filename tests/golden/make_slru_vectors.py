"""Write golden vectors for the slot cache / gap state machine.

Runs the reference's own ExpertStreamOffloader._install_cache and
_router_split_gap (src/sluice/offloader.py:895-1044, 2362-2467) on the CPU,
in this container only, over seeded expert-id traces, and records for every
step the stream-ins (local, slot) in issue order plus the full cache state
(slot_of, expert_in_slot, probation/protected order, free list, expert map).
The output JSON holds data only; the reference never leaves this container.

vLLM is not installed here, and the reference imports three names from it
at module top (a logger factory, the BaseOffloader base class and a
pin-memory probe, plus vllm.platforms on the device-inference fallback).
Those three imports are satisfied with minimal stand-ins before the import;
none of them takes part in the code paths exercised (CPU tensors: no copy
stream, no events, no pinned memory).

    python tests/golden/make_slru_vectors.py            # rewrites slru_vectors.json.gz
"""

import gzip
import json
import logging
import os
import sys
import types

import numpy as np
import torch
import torch.nn as nn

REF_SRC = "/root/reference/src"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "slru_vectors.json.gz")


def _install_vllm_standins():
    def mod(name):
        m = types.ModuleType(name)
        sys.modules[name] = m
        return m

    vllm = mod("vllm")
    lg = mod("vllm.logger")
    lg.init_logger = lambda name: logging.getLogger(name)
    me = mod("vllm.model_executor")
    off = mod("vllm.model_executor.offloader")
    base = mod("vllm.model_executor.offloader.base")

    class BaseOffloader:  # only subclassed
        pass

    base.BaseOffloader = BaseOffloader
    base.should_pin_memory = lambda: False
    plat = mod("vllm.platforms")
    plat.current_platform = types.SimpleNamespace(device_type="cpu")
    vllm.logger, vllm.model_executor, vllm.platforms = lg, me, plat
    me.offloader = off
    off.base = base


class _FakeMoE(nn.Module):
    """Duck-typed FusedMoE: the attributes _install_cache reads."""

    def __init__(self, global_n, local_n, expert_map=None):
        super().__init__()
        self.global_num_experts = global_n
        self.local_num_experts = local_n
        self.quant_method = types.SimpleNamespace()
        # per-expert rows carry the expert's local index so copies are checkable
        self.w13_weight = nn.Parameter(
            torch.arange(local_n, dtype=torch.float32).view(local_n, 1, 1).repeat(1, 2, 3),
            requires_grad=False)
        self.w2_weight = nn.Parameter(
            torch.arange(local_n, dtype=torch.float32).view(local_n, 1, 1).repeat(1, 3, 1),
            requires_grad=False)
        self.expert_map = expert_map


def _zipf_probs(E, s, rng):
    p = 1.0 / np.arange(1, E + 1) ** s
    p = p / p.sum()
    return p[rng.permutation(E)]


def _trace(kind, E, k, T_choices, steps, seed, zipf_s=1.1, rho=0.7):
    """Flat id lists per step: each token picks k distinct experts."""
    rng = np.random.default_rng(seed)
    out = []
    if kind == "uniform":
        for _ in range(steps):
            T = int(rng.choice(T_choices))
            ids = [int(v) for t in range(T) for v in rng.choice(E, size=k, replace=False)]
            out.append(ids)
        return out
    # Zipf popularity + AR(1)-correlated logit noise per token slot.
    bias = np.log(_zipf_probs(E, zipf_s, rng))
    z = rng.standard_normal((max(T_choices), E))
    for _ in range(steps):
        T = int(rng.choice(T_choices))
        z = rho * z + np.sqrt(1 - rho * rho) * rng.standard_normal(z.shape)
        logits = bias[None, :] + z[:T]
        ids = []
        for t in range(T):
            order = np.lexsort((np.arange(E), -logits[t]))
            ids += [int(v) for v in order[:k]]
        out.append(ids)
    return out


CASES = [
    # name, E, local_n, slots, frac, k, T choices, steps, trace kind, seed, ep (local_of), pins
    ("tiny_uniform", 16, 16, 6, 0.5, 2, [1, 2, 3], 120, "uniform", 11, None, None),
    ("tiny_frac0", 16, 16, 6, 0.0, 2, [1, 2, 3], 120, "uniform", 12, None, None),
    ("tiny_frac09", 16, 16, 6, 0.9, 2, [1, 2, 3], 120, "uniform", 13, None, None),
    ("v2lite_zipf", 64, 64, 48, 0.5, 6, [1, 8], 200, "zipf", 21, None, None),
    ("qwen3_s64_zipf", 128, 128, 64, 0.5, 8, [1, 8], 200, "zipf", 31, None, None),
    ("qwen3_s96_zipf", 128, 128, 96, 0.5, 8, [12], 150, "zipf", 32, None, None),
    ("stress_s32_uniform", 128, 128, 32, 0.5, 8, [4], 150, "uniform", 41, None, None),
    ("ep_half_owned", 32, 16, 8, 0.5, 4, [1, 2], 150, "uniform", 51, "even", None),
    ("pinned", 32, 32, 10, 0.5, 3, [1, 2], 150, "zipf", 61, None, [5, 7, 9]),
    ("overflow", 16, 16, 4, 0.5, 2, [1, 1, 1, 1, 2, 3], 60, "uniform", 71, None, None),
    # DeepSeek-V3 layer shape: 256 experts top-8, 64 slots, 8 tokens per step
    ("v3_s64_zipf", 256, 256, 64, 0.5, 8, [8], 120, "zipf", 81, None, None),
]


def _snapshot(cache):
    return {
        "slot_of": [cache.slot_of.get(l, -1) for l in range(cache.local_num_experts)],
        "expert_in_slot": [-1 if v is None else int(v) for v in cache.expert_in_slot],
        "probation": [int(s) for s in cache.probation.keys()],
        "protected": [int(s) for s in cache.protected.keys()],
        "free_slots": [int(s) for s in cache.free_slots],
        "map": [int(v) for v in cache.expert_map_buf.tolist()],
        "map_is_standing": bool(cache.map_is_standing),
        "protected_cap": int(cache.protected_cap),
    }


def run_case(ESO, name, E, local_n, slots, frac, k, T_choices, steps, kind, seed, ep, pins,
             fast_hit):
    os.environ["SLUICE_PROTECT_FRAC"] = str(frac)
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
    mod = _FakeMoE(E, local_n, emap)
    off._install_cache(mod)
    cache = off._caches[id(mod)]
    off._rs_caches = [cache]
    off._rs_fast_hit = fast_hit
    streams = []
    orig_stream_in = off._stream_in

    def rec_stream_in(c, local, slot, cs, on_stream=False):
        streams.append([int(local), int(slot)])
        return orig_stream_in(c, local, slot, cs, on_stream)

    off._stream_in = rec_stream_in
    trace = _trace(kind, E, k, T_choices, steps, seed)
    recs = []
    init = _snapshot(cache)
    for ids in trace:
        streams.clear()
        overflow = False
        try:
            off._router_split_gap(0, torch.tensor(ids, dtype=torch.int64).view(-1, k))
        except RuntimeError:
            overflow = True
        # slot contents must equal the streamed expert (row value == local id)
        for s, loc in enumerate(cache.expert_in_slot):
            if loc is not None:
                assert float(cache.gpu_cache["w13_weight"][s, 0, 0]) == float(loc)
        recs.append({"ids": ids, "streams": [list(x) for x in streams], "overflow": overflow,
                     "state": _snapshot(cache)})
        if overflow:
            break
    return {
        "name": name, "fast_hit": fast_hit, "E": E, "local_n": local_n, "slots": slots,
        "protect_frac": frac, "k": k, "local_of": local_of, "pins": pins,
        "counters": {"gaps": off._rs_gaps, "misses": off._rs_misses,
                     "fast_hits": off._rs_fast_hits},
        "init": init, "steps": recs,
    }


def main():
    _install_vllm_standins()
    sys.path.insert(0, REF_SRC)
    from sluice.offloader import ExpertStreamOffloader  # the reference, read from REF_SRC

    logging.getLogger("sluice").setLevel(logging.ERROR)
    cases = []
    for case in CASES:
        for fh in (False, True):
            cases.append(run_case(ExpertStreamOffloader, *case, fast_hit=fh))
    with gzip.open(OUT, "wt") as f:
        json.dump({"source": "src/sluice/offloader.py _install_cache + _router_split_gap",
                   "cases": cases}, f, separators=(",", ":"))
    print(f"wrote {OUT}: {len(cases)} traces, {sum(len(c['steps']) for c in cases)} steps")


if __name__ == "__main__":
    main()
