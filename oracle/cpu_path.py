"""The reference's per-layer router-split decode path on the host cores, in
torch fp32 -- TEST INFRASTRUCTURE: the timed CPU baseline of the benchmark
(bench.py's cpu_baseline leg) and nothing else on the product path.

One DeepSeek-V2-Lite-shaped MoE layer (hidden 2048, 64 routed SwiGLU experts
of intermediate 1408, 2 shared experts, softmax top-6 without
renormalisation, 48 slots), stepped T tokens at a time, stage by stage as
the reference's entry runs it (src/sluice/offloader.py:2578-2603):

  route    gate GEMM + Zipf router bias, softmax top-k
           (select_experts as called at 2583-2585; ties to the lower id)
  gap      the slot-cache bookkeeping of _router_split_gap (2362-2467):
           the oracle's SLRU state machine (oracle.slru.LayerCache)
  copy     _stream_in (2709-2723): host expert rows into the fp32 slot rows
  experts  fused_experts over the slot buffers (2590-2599): per resident
           expert, SwiGLU over its tokens, scaled by the routing weights
  combine  the weighted sum over k plus the shared experts (341-342, 2602)

Every stage is timed on its own (the torch CPU ops are synchronous).  The
output is checked against the float64 oracle (oracle.moe) in
tests/test_cpu_path.py.
"""

from __future__ import annotations

import os
import time
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field

import numpy as np
import torch

from oracle.slru import LayerCache

STAGES = ("route", "gap", "copy", "experts", "combine")


def zipf_bias(E: int, s: float, rng: np.random.Generator) -> np.ndarray:
    """ln p over a seeded permutation, p_r proportional to r^-s."""
    p = 1.0 / np.arange(1, E + 1) ** s
    p = p / p.sum()
    return np.log(p[rng.permutation(E)]).astype(np.float32)


@dataclass
class LayerShape:
    H: int = 2048
    E: int = 64
    I: int = 1408
    k: int = 6
    shared_I: int = 2816
    slots: int = 48
    renorm: bool = False


@dataclass
class StepTimes:
    per_stage: dict = field(default_factory=lambda: {s: [] for s in STAGES})
    misses: int = 0
    steps: int = 0

    def medians_us(self) -> dict:
        return {s: float(np.median(v)) * 1e6 if v else 0.0 for s, v in self.per_stage.items()}

    def means_us(self) -> dict:
        return {s: float(np.mean(v)) * 1e6 if v else 0.0 for s, v in self.per_stage.items()}

    def step_median_s(self) -> float:
        tot = np.sum([np.asarray(v) for v in self.per_stage.values()], axis=0)
        return float(np.median(tot))


class CpuMoELayer:
    """fp32 weights in host memory: a host store of every expert and the
    layer's S slot rows; x ~ N(0, 1), weights ~ N(0, std), Zipf router bias;
    all seeded."""

    def __init__(self, shape: LayerShape = LayerShape(), seed: int = 1, std: float = 0.02,
                 zipf_s: float = 1.1):
        sh = self.shape = shape
        rng = np.random.default_rng(seed)
        E, H, I = sh.E, sh.H, sh.I
        pool = ThreadPoolExecutor(max(1, min(16, len(os.sched_getaffinity(0)))))
        seeds = iter(np.random.SeedSequence(seed).spawn(64))

        def normal(*size):
            # rows filled in parallel chunks, each from its own seeded stream
            a = np.empty(size, dtype=np.float32)
            rows = a.reshape(size[0], -1)
            chunks = np.array_split(np.arange(size[0]), min(size[0], 32))

            def fill(idx, ss):
                g = np.random.default_rng(ss)
                blk = g.standard_normal((len(idx), rows.shape[1]), dtype=np.float32)
                blk *= std
                rows[idx[0]: idx[-1] + 1] = blk

            sub = next(seeds).spawn(len(chunks))
            list(pool.map(fill, chunks, sub))
            return torch.from_numpy(a)

        self.w13 = normal(E, 2 * I, H)   # the host store
        self.w2 = normal(E, H, I)
        self.gate = normal(E, H)
        self.shared_gu = normal(2 * sh.shared_I, H)
        self.shared_down = normal(H, sh.shared_I)
        self.bias = torch.from_numpy(zipf_bias(E, zipf_s, rng))
        S = min(sh.slots, E)
        self.slot13 = torch.zeros((S, 2 * I, H))
        self.slot2 = torch.zeros((S, H, I))
        self.cache = LayerCache(E, E, S, 0.5)
        pool.shutdown()

    # -- stages -----------------------------------------------------------------
    def route(self, x: torch.Tensor):
        sh = self.shape
        logits = x @ self.gate.T + self.bias
        # selection on the logits (softmax is monotone); a stable descending
        # sort puts equal logits in ascending id order
        order = torch.sort(logits, dim=1, descending=True, stable=True).indices[:, : sh.k]
        probs = torch.softmax(logits, dim=1)
        w = torch.gather(probs, 1, order)
        if sh.renorm:
            w = w / w.sum(dim=1, keepdim=True)
        return order.to(torch.int32), w

    def gap(self, ids: torch.Tensor):
        return self.cache.gap(ids.reshape(-1).tolist(), fast_hit=True)

    def copy(self, streams) -> None:
        for local, slot in streams:
            self.slot13[slot].copy_(self.w13[local])
            self.slot2[slot].copy_(self.w2[local])

    def experts(self, x: torch.Tensor, ids: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """Per (token, choice) pair: w * W2[s] (silu(gate) * up); pairs whose
        expert has no slot contribute zero.  Returns partials [T, k, H]."""
        T, k = ids.shape
        I = self.shape.I
        part = torch.zeros((T, k, self.shape.H))
        emap = self.cache.map
        by_slot: dict[int, list[tuple[int, int]]] = {}
        for t in range(T):
            for j in range(k):
                s = emap[int(ids[t, j])]
                if s >= 0:
                    by_slot.setdefault(s, []).append((t, j))
        for s, pairs in by_slot.items():
            tok = torch.tensor([t for t, _ in pairs])
            col = torch.tensor([j for _, j in pairs])
            h = x[tok] @ self.slot13[s].T
            act = torch.nn.functional.silu(h[:, :I]) * h[:, I:]
            part[tok, col] = (act @ self.slot2[s].T) * w[tok, col].unsqueeze(1)
        return part

    def combine(self, x: torch.Tensor, part: torch.Tensor) -> torch.Tensor:
        Is = self.shape.shared_I
        out = part.sum(dim=1)
        if Is:
            h = x @ self.shared_gu.T
            out = out + (torch.nn.functional.silu(h[:, :Is]) * h[:, Is:]) @ self.shared_down.T
        return out

    def step(self, x: torch.Tensor, times: StepTimes | None = None):
        """One decode step of the layer; returns (out [T, H], ids, weights)."""
        tick = time.perf_counter
        t0 = tick()
        ids, w = self.route(x)
        t1 = tick()
        streams = self.gap(ids)
        t2 = tick()
        self.copy(streams)
        t3 = tick()
        part = self.experts(x, ids, w)
        t4 = tick()
        out = self.combine(x, part)
        t5 = tick()
        if times is not None:
            for s, dt in zip(STAGES, (t1 - t0, t2 - t1, t3 - t2, t4 - t3, t5 - t4)):
                times.per_stage[s].append(dt)
            times.misses += len(streams)
            times.steps += 1
        return out, ids, w


def run(T: int = 8, steps: int = 64, warmup: int = 4, budget_s: float = 30.0, seed: int = 1,
        threads: int | None = None) -> dict:
    """Step the config-1 layer `warmup` untimed + up to `steps` timed steps
    (fewer if the time budget runs out) on the host cores."""
    if threads is None:
        threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    t_build = time.perf_counter()
    layer = CpuMoELayer(seed=seed)
    build_s = time.perf_counter() - t_build
    g = torch.Generator().manual_seed(5000 + seed)
    times = StepTimes()
    t0 = time.perf_counter()
    for n in range(warmup + steps):
        x = torch.randn((T, layer.shape.H), generator=g)
        layer.step(x, times if n >= warmup else None)
        if n >= warmup and time.perf_counter() - t0 > budget_s:
            break
    return {"stages_us": times.medians_us(), "stages_mean_us": times.means_us(),
            "step_median_s": times.step_median_s(),
            "steps": times.steps, "misses": times.misses, "tokens_per_step": T,
            "threads": torch.get_num_threads(), "affinity": len(os.sched_getaffinity(0)),
            "build_s": build_s, "wall_s": time.perf_counter() - t0}
