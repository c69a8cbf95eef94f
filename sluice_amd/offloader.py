"""Routing-aware MoE expert streaming offloader, router-split path, on MI355X.

Mirrors the reference's ``ExpertStreamOffloader`` (src/sluice/offloader.py)
for the router-split decode path: the same lifecycle (``wrap_modules`` ->
``post_init`` -> ``attach_model``), the same env flags, the same slot-buffer
and expert-map layout, the same ``vllm::sluice_stream_gap`` op and traced
``_forward_entry``.  Underneath, the per-layer slot cache and the gap run in
libsluice_hip.so: a device slot-lookup kernel publishes the step's selected
experts into pinned host memory, the native SLRU assigns slots exactly as the
reference's OrderedDict state machine does, missing experts stream with
hipMemcpyAsync on a dedicated copy stream, and a map kernel rewrites the
standing expert map the captured expert product reads by pointer.

Execution model per MoE layer per decode step (T <= thr tokens):

    gate + select_experts            [capturable]
    -> vllm::sluice_stream_gap       [eager gap: lookup, wait, SLRU, H2D, map]
    -> sluice::fused_experts         [capturable; slots + map by pointer]
    -> shared experts                [capturable]

Steps above the envelope (more tokens than slots // top_k: prefill chunks,
large decode batches) take the classic path instead, as in the reference
(src/sluice/offloader.py:1452-1933): the layer's ``quant_method.apply`` is
wrapped so that ``run_moe`` syncs the ids once, the native slot cache plans
the step -- one wave when the working set fits, else wave 0 (hits + fills)
and the leftover misses rotated through the probation slots in ping-pong
groups -- and the expert product runs once per wave against that wave's
map, its row copies overlapping the previous wave's product on the copy
stream; wave outputs are summed in fp32.
"""


import atexit
import ctypes
import json
import logging
import os
import time
from collections.abc import Generator
from dataclasses import dataclass, field
from typing import Optional

import torch
import torch.nn as nn

from sluice_amd import _lib, ops

logger = logging.getLogger("sluice")

# Shared/global tensors, not per-expert weights (src/sluice/offloader.py:89-96).
NON_EXPERT_WEIGHTS = frozenset(
    {"e_score_correction_bias", "w13_input_scale", "w2_input_scale", "hash_indices_table"}
)

PROTECT_FRAC_ENV = "SLUICE_PROTECT_FRAC"
ROUTER_SPLIT_ENV = "SLUICE_ROUTER_SPLIT"
PIECEWISE_ENV = "SLUICE_PIECEWISE"
GRAPH_ENV = "SLUICE_GRAPH"
FAST_HIT_ENV = "SLUICE_RS_FAST_HIT"
NOOP_ENV = "SLUICE_RS_NOOP"
# Opt-in policies (src/sluice/offloader.py:97-118): LFU-ordered protected
# victims; per-expert selection counts dumped as JSONL snapshots; a static
# pin file {"layers": {"<MoE-layer ordinal>": [global ids]}}.
LFU_ENV = "SLUICE_LFU"
COUNTS_DIR_ENV = "SLUICE_EXPERT_COUNTS"
COUNTS_EVERY_ENV = "SLUICE_EXPERT_COUNTS_EVERY"
PIN_FILE_ENV = "SLUICE_PIN_FILE"


@dataclass
class _ExpertLayerCache:
    """Per-layer streaming state (src/sluice/offloader.py:121-169).  The SLRU
    state itself lives in the native layer object; the properties below read
    it back in the reference's shapes for inspection and tests."""

    local_num_experts: int
    num_slots: int
    protected_cap: int
    device: torch.device
    param_names: list = field(default_factory=list)
    gpu_cache: dict = field(default_factory=dict)
    cpu_store: dict = field(default_factory=dict)
    host_stores: list = field(default_factory=list)
    local_of: list = field(default_factory=list)
    global_of_local: list = field(default_factory=list)
    expert_map_buf: Optional[torch.Tensor] = None
    bytes_per_expert: int = 0
    static_full: bool = False
    handle: Optional[int] = None
    pinned_slots: set = field(default_factory=set)
    ordinal: int = -1
    layer_name: str = ""
    policy_steps: int = 0  # real classic steps with selected experts, last seen

    # -- native state views ------------------------------------------------
    def _state(self):
        lib = _lib.load()
        S, L = self.num_slots, self.local_num_experts
        slot_of = (ctypes.c_int32 * L)()
        eis = (ctypes.c_int32 * S)()
        prob = (ctypes.c_int32 * S)()
        prot = (ctypes.c_int32 * S)()
        free = (ctypes.c_int32 * S)()
        n_prob, n_prot, n_free = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        ctr = (ctypes.c_int64 * 8)()
        _lib.check(lib.sluice_layer_state(self.handle, slot_of, eis, prob, ctypes.byref(n_prob),
                                          prot, ctypes.byref(n_prot), free, ctypes.byref(n_free),
                                          ctr), "sluice_layer_state")
        return {
            "slot_of": list(slot_of),
            "expert_in_slot": list(eis),
            "probation": list(prob)[: n_prob.value],
            "protected": list(prot)[: n_prot.value],
            "free_slots": list(free)[: n_free.value],
            "counters": list(ctr),
        }

    @property
    def slot_of(self) -> dict:
        return {l: s for l, s in enumerate(self._state()["slot_of"]) if s >= 0}

    @property
    def expert_in_slot(self) -> list:
        return [None if v < 0 else v for v in self._state()["expert_in_slot"]]

    @property
    def probation(self) -> list:
        return self._state()["probation"]

    @property
    def protected(self) -> list:
        return self._state()["protected"]

    @property
    def free_slots(self) -> list:
        return self._state()["free_slots"]

    @property
    def map_is_standing(self) -> bool:
        return bool(self._state()["counters"][6])

    def stats(self) -> dict:
        c = self._state()["counters"]
        return {"gaps": c[0], "misses": c[1], "fast_hits": c[2], "map_writes": c[3],
                "bytes": c[4] | (c[5] << 32)}

    def policy_state(self) -> dict:
        """LFU frequencies (local -> count, nonzero only), per-global
        decode/scan selection counts and the classic step classes."""
        lib = _lib.load()
        n, E = self.local_num_experts, len(self.local_of)
        freq = (ctypes.c_int64 * n)()
        dec = (ctypes.c_int64 * E)()
        scan = (ctypes.c_int64 * E)()
        st = (ctypes.c_int64 * 3)()
        _lib.check(lib.sluice_layer_policy_state(self.handle, freq, dec, scan, st),
                   "sluice_layer_policy_state")
        return {"freq": {l: int(f) for l, f in enumerate(freq) if f},
                "counts_decode": list(dec), "counts_scan": list(scan),
                "steps_small": int(st[0]), "steps_scan": int(st[1]), "lfu_steps": int(st[2])}

    @property
    def freq(self) -> dict:
        return self.policy_state()["freq"]


class ExpertStreamOffloader:
    """Stream routed-expert weights host->HBM per decode step, by routing.

    Args:
        expert_cache_slots: HBM-resident expert slots per MoE layer.
    """

    def __init__(self, expert_cache_slots: int):
        assert expert_cache_slots > 0
        self.expert_cache_slots = expert_cache_slots
        try:
            frac = float(os.environ.get(PROTECT_FRAC_ENV, "0.5"))
        except ValueError:
            frac = 0.5
        self.protect_frac = min(max(frac, 0.0), 0.9)
        self.piecewise = os.environ.get(PIECEWISE_ENV, "0") == "1"
        self.router_split = os.environ.get(ROUTER_SPLIT_ENV, "0") == "1"
        self.graph_mode = os.environ.get(GRAPH_ENV, "0") == "1"
        self._rs_fast_hit = os.environ.get(FAST_HIT_ENV, "0") == "1"
        self._rs_noop = os.environ.get(NOOP_ENV, "0") == "1"
        if self._rs_noop:
            logger.warning("Sluice: SLUICE_RS_NOOP=1 — the router-split gap is a NO-OP; "
                           "OUTPUTS ARE INVALID (stale expert map). Perf diagnostic only.")
        self.pin_memory = torch.cuda.is_available()
        self._caches: dict[int, _ExpertLayerCache] = {}
        self._layers: list[nn.Module] = []
        self._prepared_stores: dict[int, list] = {}  # pinned stores made before load
        self._rs_caches: list[_ExpertLayerCache] = []
        self._rs_gaps = 0
        self._rs_misses = 0
        self._rs_fast_hits = 0
        self._rs_layers = 0
        self._rs_thr: Optional[int] = None
        self._server: Optional[int] = None
        self._spec_tokens = 0
        self._signal: Optional[tuple] = None
        self._warned_waves = False
        self.lfu = os.environ.get(LFU_ENV, "0") == "1"
        # expert-count profiling (src/sluice/offloader.py:441-465, 1393-1448)
        self._counts_dir = os.environ.get(COUNTS_DIR_ENV) or None
        self._counts_every = 5000
        self._counts_calls = 0
        self._counts_snap = 0
        self._counts_file = None
        if self._counts_dir:
            try:
                self._counts_every = max(int(os.environ.get(COUNTS_EVERY_ENV, "5000")), 1)
            except ValueError:
                self._counts_every = 5000
            atexit.register(self._dump_expert_counts, True)
        # static pins (src/sluice/offloader.py:466-481): parsed here, applied
        # per layer at install; a malformed file fails loudly
        self._pin_layers: Optional[dict] = None
        self._pin_stats = [0, 0]  # experts pinned, layers with pins
        pin_path = os.environ.get(PIN_FILE_ENV)
        if pin_path:
            with open(pin_path) as f:
                raw = json.load(f)
            layers = raw.get("layers", raw)
            self._pin_layers = {int(k_): [int(g) for g in v] for k_, v in layers.items()}
            logger.info("Sluice: static pin file %s (%d layers listed).", pin_path,
                        len(self._pin_layers))
        if self.router_split:
            _register_stream_gap_op(self)
        logger.info("Sluice ExpertStreamOffloader enabled (%d cache slots per layer, "
                    "protect_frac=%.2f).", expert_cache_slots, self.protect_frac)

    # -- model construction -------------------------------------------------
    @staticmethod
    def _is_moe_layer(module: nn.Module) -> bool:
        return (hasattr(module, "local_num_experts") and hasattr(module, "global_num_experts")
                and hasattr(module, "quant_method"))

    @staticmethod
    def _per_expert_params(module: nn.Module, local_n: int) -> dict:
        return {
            name: p for name, p in module.named_parameters(recurse=False)
            if name not in NON_EXPERT_WEIGHTS and p.dim() >= 1 and p.shape[0] == local_n
        }

    def wrap_modules(self, modules_generator: Generator) -> list:
        modules = []
        for module in modules_generator:
            for sub in module.modules():
                if self._is_moe_layer(sub):
                    self._prepare_layer(sub)
            modules.append(module)
        return modules

    def _prepare_layer(self, module: nn.Module) -> None:
        """Move a layer's (still empty) per-expert params to host memory so
        the checkpoint loads there (src/sluice/offloader.py:554-571).  With a
        GPU present they become views of exact-size pinned host stores, so
        the loader writes straight into the memory the expert rows stream
        from, and _install_cache adopts it without a second host copy."""
        qm = module.quant_method
        if qm is None or getattr(qm, "is_monolithic", False):
            return
        if getattr(module, "rocm_aiter_fmoe_enabled", False):
            return
        local_n = int(module.local_num_experts)
        per_expert = self._per_expert_params(module, local_n)
        if not per_expert:
            return
        for p in per_expert.values():
            cpu = p.data if p.data.device.type == "cpu" else p.data.to("cpu")
            if self.pin_memory and ops.host_store_of(cpu) is None:
                store = ops.HostStore(tuple(cpu.shape), cpu.dtype)
                store.tensor.copy_(cpu)
                self._prepared_stores.setdefault(id(module), []).append(store)
                cpu = store.tensor
            p.data = cpu
        if all(id(module) != id(m) for m in self._layers):
            self._layers.append(module)

    # -- after load -----------------------------------------------------------
    def post_init(self, config=None) -> None:
        self._check_config(config)
        if torch.cuda.is_available():
            torch.cuda.synchronize()
        for module in self._layers:
            self._install_cache(module)
            self._wrap_apply(module)
        # SLUICE_GRAPH relaxed the eager guard on the promise that every
        # layer is static-full (a constant map is safe to capture)
        if self.graph_mode:
            streaming = [k_ for k_, c in self._caches.items() if not c.static_full]
            if streaming:
                raise RuntimeError(
                    "Sluice: SLUICE_GRAPH=1 requires every layer to be static_full (slots >= "
                    f"local experts), but {len(streaming)} layer(s) are streaming. A captured "
                    "graph would freeze a changing expert map. Raise SLUICE_SLOTS to full "
                    "residency or unset SLUICE_GRAPH.")
        if self._caches:
            host = sum(c.bytes_per_expert * c.local_num_experts for c in self._caches.values()
                       if not c.static_full)
            vram = sum(c.bytes_per_expert * c.num_slots for c in self._caches.values())
            logger.info("Sluice: %d MoE layers ready — host expert store %.1f GiB%s, HBM slot "
                        "cache %.1f GiB.", len(self._caches), host / 2**30,
                        " (pinned)" if self.pin_memory else " (pageable)", vram / 2**30)

    def _check_config(self, cfg=None) -> None:
        """The engine-configuration guards (src/sluice/offloader.py:663-851).

        With vLLM installed the config must be readable (fail closed); without
        vLLM (the standalone harness) there is nothing to check unless a
        config object is passed in.  Refuses DP > 1 and EPLB (this build
        serves one rank's experts and owns the expert map), and any CUDA-graph
        mode that would capture the streaming hook: eager is required unless
        SLUICE_PIECEWISE (the hook runs in a graph break; FULL capture is
        still refused) or SLUICE_GRAPH (every layer static-full, checked in
        post_init).  Under piecewise it makes the MoE ops and the gap op
        graph split points and enforces the router-split envelope: the whole
        batch must fit slots // top_k tokens.  Records the speculative depth
        the decode classifier needs."""
        if cfg is None:
            try:
                from vllm.config import get_current_vllm_config  # type: ignore
            except ImportError:
                return  # no engine: the standalone harness drives the offloader
            try:
                cfg = get_current_vllm_config()
            except Exception as e:
                raise RuntimeError("Sluice: could not read the vLLM config to verify it is safe "
                                   "(DP/EPLB/eager); refusing to run. This usually means an "
                                   "unexpected vLLM version.") from e
            if cfg is None:
                raise RuntimeError("Sluice: vLLM config is None; cannot verify a safe "
                                   "configuration (DP/EPLB/eager). Refusing to run.")
        pc = getattr(cfg, "parallel_config", None)
        if pc is not None:
            if (getattr(pc, "data_parallel_size", 1) or 1) > 1:
                raise RuntimeError("Sluice (MI355X build): data parallelism > 1 is not supported "
                                   "(one rank's expert shard per process; no post-dispatch "
                                   "seam).")
            if getattr(pc, "enable_eplb", False):
                raise RuntimeError("Sluice: EPLB is unsupported (it re-registers the expert map "
                                   "buffer over Sluice's slot map).")
        relax_eager = self.graph_mode or self.piecewise
        mc = getattr(cfg, "model_config", None)
        if mc is not None and not getattr(mc, "enforce_eager", False) and not relax_eager:
            raise RuntimeError(
                "Sluice: requires eager execution — run with --enforce-eager. Without it, "
                "CUDA-graph capture freezes a stale expert map (silently wrong output) and stock "
                "torch.compile skips the post_init that installs Sluice's expert cache. (Set "
                "SLUICE_GRAPH=1 only with slots >= experts / static_full.)")
        cc = getattr(cfg, "compilation_config", None)
        cg = getattr(cc, "cudagraph_mode", None) if cc is not None else None
        cg_name = getattr(cg, "name", str(cg)) if cg is not None else "NONE"
        if self.piecewise and "FULL" in cg_name:
            raise RuntimeError(
                "Sluice: SLUICE_PIECEWISE requires PIECEWISE cudagraph (the hook runs eager in a "
                f"graph break); got {cg_name}. FULL would try to capture the hook's D2H sync.")
        if cg is not None and cg_name != "NONE" and not relax_eager:
            raise RuntimeError(
                "Sluice: CUDA graphs would capture a frozen expert map and replay it with stale "
                "routing (silently wrong outputs). Run with enforce_eager (--enforce-eager).")
        if self.piecewise and cc is not None:
            # the MoE layer (whose apply runs the hook) and the gap op are
            # eager gaps between the captured pieces
            ops_ = list(getattr(cc, "splitting_ops", None) or [])
            wanted = ["vllm::moe_forward", "vllm::moe_forward_shared"]
            if self.router_split:
                wanted.append("vllm::sluice_stream_gap")
            cc.splitting_ops = ops_ + [op for op in wanted if op not in ops_]
        if self.router_split and self.piecewise:
            topk = 8
            hf = getattr(mc, "hf_config", None) if mc is not None else None
            for src in (hf, getattr(hf, "text_config", None)):
                v = getattr(src, "num_experts_per_tok", None) if src else None
                if v:
                    topk = int(v)
                    break
            thr = max(1, self.expert_cache_slots // topk)
            self._rs_thr = thr
            sched = getattr(cfg, "scheduler_config", None)
            mbt = getattr(sched, "max_num_batched_tokens", None)
            if mbt is not None and mbt > thr:
                raise RuntimeError(
                    "Sluice router-split under piecewise compiles a single trace whose size "
                    "branch is resolved at trace time; the whole batch envelope must fit it. "
                    f"Got max_num_batched_tokens={mbt} > slots//topk={thr}. Set "
                    f"--max-num-batched-tokens {thr} (prefill runs in {thr}-token chunks) or "
                    "raise SLUICE_SLOTS.")
        # A speculative-decode request verifies 1 + k tokens: its decode
        # region spans ndec * (1 + k) rows (src/sluice/offloader.py:843-851).
        sc = getattr(cfg, "speculative_config", None)
        k_spec = getattr(sc, "num_speculative_tokens", 0) if sc is not None else 0
        try:
            self._spec_tokens = max(int(k_spec or 0), 0)
        except (TypeError, ValueError):
            self._spec_tokens = 0

    @staticmethod
    def _infer_device(module: nn.Module) -> torch.device:
        for t in list(module.parameters(recurse=False)) + list(module.buffers(recurse=False)):
            if t is not None and t.device.type != "cpu":
                return t.device
        idx = torch.cuda.current_device() if torch.cuda.is_available() else 0
        return torch.device("cuda", idx)

    def _install_cache(self, module: nn.Module) -> None:
        """Slot buffers [S, ...] as the live params, a pinned host store of
        every local expert, the expert map and the native slot cache
        (src/sluice/offloader.py:895-1044)."""
        lib = _lib.load()
        local_n = int(module.local_num_experts)
        global_n = int(module.global_num_experts)
        per_expert = self._per_expert_params(module, local_n)
        if not per_expert:
            return
        device = self._infer_device(module)
        num_slots = min(self.expert_cache_slots, local_n)
        protected_cap = max(min(int(num_slots * self.protect_frac), num_slots - 1), 0)
        cache = _ExpertLayerCache(local_num_experts=local_n, num_slots=num_slots,
                                  protected_cap=protected_cap, device=device,
                                  param_names=list(per_expert.keys()))
        cache.static_full = num_slots >= local_n
        for name, p in per_expert.items():
            cpu = p.data if p.data.device.type == "cpu" else p.data.to("cpu")
            slot = torch.empty((num_slots, *p.shape[1:]), dtype=p.dtype, device=device)
            if cache.static_full:
                slot.copy_(cpu)
            else:
                store = ops.host_store_of(cpu)
                if store is not None:
                    # already pinned (e.g. one host pool shared by several
                    # layers): adopt it as the host store, no copy
                    cache.cpu_store[name] = cpu
                else:
                    store = ops.HostStore(tuple(cpu.shape), cpu.dtype)
                    store.tensor.copy_(cpu)
                    cache.cpu_store[name] = store.tensor
                cache.host_stores.append(store)
            cache.gpu_cache[name] = slot
            p.data = slot
            cache.bytes_per_expert += cpu[0].nbytes
        # adopted stores now live in cache.host_stores; a static-full layer's
        # rows are all in HBM, so its prepared stores are released here
        self._prepared_stores.pop(id(module), None)
        orig_map = getattr(module, "expert_map", None)
        if orig_map is not None:
            cache.local_of = [int(v) for v in orig_map.to("cpu").tolist()]
        else:
            cache.local_of = list(range(global_n))
        cache.global_of_local = [-1] * local_n
        for g, loc in enumerate(cache.local_of):
            if 0 <= loc < local_n:
                cache.global_of_local[loc] = g
        cache.expert_map_buf = torch.full((global_n,), -1, dtype=torch.int32, device=device)
        if cache.static_full:
            for g, loc in enumerate(cache.local_of):
                if loc >= 0:
                    cache.expert_map_buf[g] = loc
        module.register_buffer("_expert_map", cache.expert_map_buf, persistent=False)

        h = ctypes.c_void_p()
        _lib.check(lib.sluice_layer_create(global_n, local_n, num_slots, protected_cap,
                                           _lib.int32_array(cache.local_of),
                                           cache.expert_map_buf.data_ptr(), ctypes.byref(h)),
                   "sluice_layer_create")
        cache.handle = h.value
        cache.ordinal = len(self._caches)
        cache.layer_name = getattr(module, "layer_name", "") or ""
        if not cache.static_full:
            for name in cache.param_names:
                slot_t = cache.gpu_cache[name]
                host_t = cache.cpu_store[name]
                _lib.check(lib.sluice_layer_add_param(cache.handle, slot_t.data_ptr(),
                                                      host_t.data_ptr(), host_t[0].nbytes),
                           "sluice_layer_add_param")
            if self.lfu or self._counts_dir:
                _lib.check(lib.sluice_layer_set_policy(cache.handle, int(self.lfu),
                                                       int(bool(self._counts_dir))),
                           "sluice_layer_set_policy")
            if self._pin_layers is not None:
                self._apply_pins(cache, cache.ordinal)
        self._caches[id(module)] = cache
        logger.info("Sluice: %d local experts -> %d HBM slots (%d protected), %d params/expert, "
                    "%.1f MiB/expert.", local_n, num_slots, protected_cap, len(per_expert),
                    cache.bytes_per_expert / 2**20)

    def _apply_pins(self, cache: _ExpertLayerCache, ordinal: int) -> None:
        """Fill this layer's pinned slots from the pin file, one row copy per
        expert at init (src/sluice/offloader.py:1046-1083): pins live outside
        both segments and the free list, so nothing evicts them, and each one
        is debited from protected_cap so probation keeps its size."""
        wanted = self._pin_layers.get(ordinal, []) if self._pin_layers else []
        if not wanted:
            return
        lib = _lib.load()
        budget = cache.protected_cap
        n = 0
        resident = set(cache.slot_of)
        for g in wanted:
            if n >= budget:
                logger.warning("Sluice: layer %d pin list (%d ids) exceeds the protected budget "
                               "(%d); pinning the first %d only.", ordinal, len(wanted), budget,
                               n)
                break
            if not (0 <= g < len(cache.local_of)):
                continue
            local = cache.local_of[g]
            if local < 0 or local in resident:
                continue
            slot = ctypes.c_int()
            if lib.sluice_layer_pin(cache.handle, local, 1, ctypes.byref(slot)) != _lib.SLUICE_OK:
                continue  # no free slot left
            for name, gpu in cache.gpu_cache.items():
                gpu[slot.value].copy_(cache.cpu_store[name][local])
            resident.add(local)
            cache.pinned_slots.add(slot.value)
            n += 1
        if n:
            cache.protected_cap -= n
            self._pin_stats[0] += n
            self._pin_stats[1] += 1

    # -- expert-count profiling ---------------------------------------------------
    def _counts_tick(self) -> None:
        self._counts_calls += 1
        if self._counts_calls % self._counts_every == 0:
            self._dump_expert_counts(False)

    def _dump_expert_counts(self, final: bool) -> None:
        """Append one cumulative JSONL snapshot per streaming layer (nonzero
        counts only, keyed by global expert id) to
        <SLUICE_EXPERT_COUNTS>/expert_counts_rank<r>.jsonl, in the
        reference's record format (src/sluice/offloader.py:1399-1448).  Never
        raises: profiling must not take serving down."""
        if not self._counts_dir:
            return
        layers = [c for c in self._caches.values() if not c.static_full and c.handle]
        if not layers:
            return
        try:
            if self._counts_file is None:
                try:
                    import torch.distributed as dist

                    rank = dist.get_rank() if dist.is_initialized() else 0
                except Exception:
                    rank = int(os.environ.get("RANK", "0") or "0")
                os.makedirs(self._counts_dir, exist_ok=True)
                self._counts_file = open(
                    os.path.join(self._counts_dir, f"expert_counts_rank{rank}.jsonl"), "a")
            self._counts_snap += 1
            pols = [c.policy_state() for c in layers]
            small = sum(p["steps_small"] for p in pols)
            scan = sum(p["steps_scan"] for p in pols)
            for c, p in zip(layers, pols):
                self._counts_file.write(json.dumps({
                    "snap": self._counts_snap, "final": final, "ts": time.time(),
                    "hook_calls": self._counts_calls, "steps_small": small, "steps_scan": scan,
                    "layer": c.ordinal, "layer_name": c.layer_name,
                    "n_global": len(p["counts_decode"]),
                    "decode": {str(g): v for g, v in enumerate(p["counts_decode"]) if v},
                    "scan": {str(g): v for g, v in enumerate(p["counts_scan"]) if v},
                }) + "\n")
            self._counts_file.flush()
        except Exception:
            logger.exception("Sluice: expert-count dump failed (non-fatal)")

    # -- classic (wave) path -------------------------------------------------
    def _wrap_apply(self, module: nn.Module) -> None:
        """Wrap the layer's ``quant_method.apply`` so steps that reach it
        (the ones the router-split entry hands to the stock path) run the
        classic hook (src/sluice/offloader.py:1085-1119)."""
        qm = module.quant_method
        if qm is None or getattr(qm, "_sluice_wrapped", False) or not hasattr(qm, "apply"):
            return
        original_apply = qm.apply
        offloader = self

        def apply(*args, **kwargs):
            layer = kwargs.get("layer", args[0] if args else None)
            topk_ids = kwargs.get("topk_ids")
            if layer is None or topk_ids is None:
                return original_apply(*args, **kwargs)
            return offloader.run_moe(original_apply, args, kwargs, layer, topk_ids)

        if self.piecewise:
            # the hook syncs the host: keep it out of any traced region
            apply = torch._dynamo.disable(apply)
        qm.apply = apply
        qm._sluice_wrapped = True

    def set_step_signal(self, nd: Optional[int], ndec: Optional[int],
                        real_step: bool = True) -> None:
        """Publish the step's decode split for engines without vLLM's forward
        context: rows [0, nd) are decode tokens of ndec requests (None: not
        published); real_step False marks a dummy run."""
        self._signal = (nd, ndec, bool(real_step))

    def clear_step_signal(self) -> None:
        self._signal = None

    def _split_signal(self) -> tuple:
        """``(num_decode_tokens, num_decodes, is_real_step)``
        (src/sluice/offloader.py:1766-1800): the signal set with
        set_step_signal, else vLLM's forward context; ``(None, None, False)``
        (a dummy run) when neither exists."""
        if self._signal is not None:
            return self._signal
        try:
            from vllm.forward_context import get_forward_context  # type: ignore

            ctx = get_forward_context()
        except Exception:
            return None, None, False
        md = getattr(ctx, "attn_metadata", None)
        if isinstance(md, dict):
            md = next(iter(md.values()), None)
        if md is None:
            return None, None, False
        nd = getattr(md, "num_decode_tokens", None)
        if nd is None:
            return None, None, True
        ndec = getattr(md, "num_decodes", None)
        try:
            return int(nd), (int(ndec) if ndec is not None else None), True
        except (TypeError, ValueError):
            return None, None, True

    def run_moe(self, original_apply, args, kwargs, module, topk_ids):
        """Classic streaming hook in place of ``quant_method.apply``
        (src/sluice/offloader.py:1452-1765, 1846-1933).

        One host sync for the ids, the native bookkeeping (decode
        classification, class-aware fills, ping-pong rotation of leftover
        misses), then the wrapped kernel once per wave: each wave's map
        write and row copies are ordered around it by the native layer, and
        the outputs of a multi-wave step are summed in fp32 (exact in math:
        an expert outside a wave's map contributes zero to it)."""
        cache = self._caches.get(id(module))
        if cache is None or cache.static_full:
            return original_apply(*args, **kwargs)
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            raise RuntimeError("Sluice: streaming hook reached under CUDA graph capture; "
                               "run with enforce_eager.")
        nd, ndec, real_step = self._split_signal()
        ids = topk_ids if topk_ids.dtype == torch.int32 else topk_ids.to(torch.int32)
        ids = ids.contiguous()
        T = int(ids.shape[0]) if ids.dim() else 0
        lib = _lib.load()
        stream = torch.cuda.current_stream(ids.device).cuda_stream
        nw = ctypes.c_int()
        _raise_gap(lib.sluice_layer_classic_plan(
            cache.handle, ids.data_ptr(), ids.numel(), T, -1 if nd is None else int(nd),
            -1 if ndec is None else int(ndec), int(bool(real_step)), int(self._spec_tokens),
            stream, ctypes.byref(nw)), "sluice_layer_classic_plan")
        n_waves = nw.value
        if self._counts_dir and real_step:
            # the reference ticks its profiling clock once per real hook call
            # that selected experts (the steps the layer classified)
            pol = cache.policy_state()
            seen = pol["steps_small"] + pol["steps_scan"]
            if seen != cache.policy_steps:
                cache.policy_steps = seen
                self._counts_tick()
        if n_waves > 1 and real_step and not self._warned_waves:
            self._warned_waves = True
            logger.warning("Sluice: a step selected more local experts than usable slots; "
                           "executing in %d waves (exact in math, not bit-identical to a "
                           "single launch). Raise SLUICE_SLOTS to avoid waves.", n_waves)
        total = out = None
        for w in range(n_waves):
            _lib.check(lib.sluice_layer_classic_wave(cache.handle, w, stream),
                       "sluice_layer_classic_wave")
            out = original_apply(*args, **kwargs)
            _lib.check(lib.sluice_layer_classic_wave_done(cache.handle, w, stream),
                       "sluice_layer_classic_wave_done")
            if n_waves == 1:
                return out
            total = out.to(torch.float32) if total is None else total.add_(out)
        return total.to(out.dtype)

    # -- router split -----------------------------------------------------------
    def attach_model(self, model: nn.Module) -> None:
        self.attach_router_split(model)

    def attach_router_split(self, model: nn.Module) -> None:
        """Patch each eligible layer's ``runner._forward_entry`` with the traced
        split path (src/sluice/offloader.py:2469-2635)."""
        if not self.router_split:
            return
        patched = 0
        skips: dict = {}
        seen = 0
        for module in model.modules():
            cache = self._caches.get(id(module))
            if cache is None:
                continue
            seen += 1
            runner = getattr(module, "runner", None)
            if runner is None:
                skips["no-runner"] = skips.get("no-runner", 0) + 1
                continue
            if cache.static_full:
                skips["static-full"] = skips.get("static-full", 0) + 1
                continue
            mc = getattr(runner, "moe_config", None)
            topk = getattr(mc, "experts_per_token", None) if mc else None
            if topk is None:
                topk = getattr(module, "top_k", None) or 8
            idx = len(self._rs_caches)
            self._rs_caches.append(cache)
            thr = self._rs_thr
            if thr is None:
                thr = max(1, min(16, self.expert_cache_slots // int(topk)))
            se = getattr(runner, "_shared_experts", None)
            shared_layer = getattr(se, "_layer", None) if se is not None else None
            runner._forward_entry = _make_entry(
                idx, module.w13_weight, module.w2_weight, int(module.global_num_experts),
                cache.expert_map_buf, shared_layer, runner.router.select_experts,
                runner._forward_entry, getattr(runner, "gate", None), thr,
                getattr(module, "w13_weight_scale", None), getattr(module, "w2_weight_scale", None),
                getattr(module, "block_shape", None))
            patched += 1
        self._rs_layers = patched
        logger.warning("Sluice: ROUTER-SPLIT armed on %d/%d MoE layers. skips=%s", patched, seen,
                       skips or "{}")

    def _router_split_gap(self, idx: int, topk_ids: torch.Tensor,
                          hidden_states: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
        """Body of ``vllm::sluice_stream_gap`` (src/sluice/offloader.py:2362-2467).

        Launches the layer's gap kernel on the current stream and, unless a
        gap server serves this offloader, serves its record inline (the
        reference's eager gap).  When ``hidden_states`` is given, returns the
        op's fresh copy of it, written by the gap kernel itself."""
        cache = self._rs_caches[idx]
        if self._server is None:
            self._rs_gaps += 1
            if self._rs_gaps == 1 or self._rs_gaps % 2000 == 0:
                c = self.gap_counters()
                logger.warning("Sluice DIAG[rs]: router-split layers=%d gap-calls=%d misses=%d "
                               "fast-hits=%d%s", len(self._rs_caches), self._rs_gaps,
                               c["misses"], c["fast_hits"],
                               " NOOP-GAP(OUTPUTS INVALID)" if self._rs_noop else "")
        if self._rs_noop:
            return None if hidden_states is None else hidden_states.clone()
        ids = topk_ids if topk_ids.dtype == torch.int32 else topk_ids.to(torch.int32)
        ids = ids.contiguous()
        lib = _lib.load()
        stream = torch.cuda.current_stream(ids.device).cuda_stream
        out = None
        src = dst = None
        nbytes = 0
        if hidden_states is not None:
            out = torch.empty_like(hidden_states)
            nb = hidden_states.numel() * hidden_states.element_size()
            if (hidden_states.is_contiguous() and nb % 16 == 0
                    and hidden_states.data_ptr() % 16 == 0 and out.data_ptr() % 16 == 0):
                src, dst, nbytes = hidden_states.data_ptr(), out.data_ptr(), nb
            else:
                out.copy_(hidden_states)
        rc = lib.sluice_layer_gap_launch(cache.handle, ids.data_ptr(), ids.numel(), src, dst,
                                         nbytes, stream)
        _lib.check(rc, "sluice_layer_gap_launch")
        if self._server is None:
            rc = lib.sluice_layer_gap_serve(cache.handle, int(self._rs_fast_hit), stream)
            _raise_gap(rc, "sluice_layer_gap_serve")
        return out

    # -- gap server ---------------------------------------------------------------
    def start_gap_server(self) -> None:
        """Serve every router-split layer's gap records on a native thread:
        the gap op becomes a pure device launch (capturable), so a whole
        decode step, gaps included, can replay as one hipGraph.  Slot
        assignment and maps are the same as with inline gaps."""
        if self._server is not None or not self._rs_caches:
            return
        lib = _lib.load()
        handles = (ctypes.c_void_p * len(self._rs_caches))(*[c.handle for c in self._rs_caches])
        srv = ctypes.c_void_p()
        _lib.check(lib.sluice_gap_server_create(handles, len(self._rs_caches),
                                                int(self._rs_fast_hit), ctypes.byref(srv)),
                   "sluice_gap_server_create")
        self._server = srv.value

    def drain(self, timeout_s: float = 60.0) -> None:
        """Synchronise the device and wait until every gap record it posted
        has been served; raises what the gap raised (e.g. the overflow
        RuntimeError)."""
        torch.cuda.synchronize()
        if self._server is None:
            return
        rc = _lib.load().sluice_gap_server_drain(self._server, float(timeout_s))
        _raise_gap(rc, "sluice_gap_server_drain")

    def stop_gap_server(self) -> None:
        if self._server is None:
            return
        self.drain()
        srv, self._server = self._server, None
        _raise_gap(_lib.load().sluice_gap_server_destroy(srv), "sluice_gap_server_destroy")

    def gap_counters(self) -> dict:
        tot = {"gaps": 0, "misses": 0, "fast_hits": 0, "map_writes": 0, "bytes": 0}
        for c in self._rs_caches:
            for k_, v in c.stats().items():
                tot[k_] += v
        return tot

    def classic_counters(self) -> dict:
        """Classic steps and waves run over every streaming layer."""
        lib = _lib.load()
        tot = {"steps": 0, "waves": 0}
        ctr = (ctypes.c_int64 * 2)()
        n = ctypes.c_int()
        for c in self._caches.values():
            if c.handle and not c.static_full:
                _lib.check(lib.sluice_layer_classic_plan_read(c.handle, None, 0, ctypes.byref(n),
                                                              ctr), "classic_plan_read")
                tot["steps"] += ctr[0]
                tot["waves"] += ctr[1]
        return tot

    def get_stats(self) -> dict:
        c = self.gap_counters()
        cl = self.classic_counters()
        return {"rs": {"steps": c["gaps"], "hits": None, "misses": c["misses"],
                       "bytes": c["bytes"], "waves": c["gaps"], "fast_hits": c["fast_hits"]},
                "classic": {"steps": cl["steps"], "waves": cl["waves"]}}

    def close(self) -> None:
        lib = _lib.load()
        if self._server is not None:
            srv, self._server = self._server, None
            torch.cuda.synchronize()
            lib.sluice_gap_server_drain(srv, 60.0)
            lib.sluice_gap_server_destroy(srv)
        for c in self._caches.values():
            if c.handle:
                lib.sluice_layer_destroy(c.handle)
                c.handle = None


def _raise_gap(rc: int, what: str) -> None:
    if rc == _lib.SLUICE_E_OVERFLOW:
        raise RuntimeError("Sluice router-split: working set exceeds slots on a "
                           "decode-sized step; raise SLUICE_SLOTS.")
    _lib.check(rc, what)


def _make_entry(idx, w13, w2, gne, emap, shared_layer, sel, orig, gate, thr, w13_scale, w2_scale,
                block_shape):
    """Bind one layer's tensors into a fresh traced entry; weights and map are
    captured BY POINTER, the gap rewrites their contents
    (src/sluice/offloader.py:2562-2603)."""

    def _forward_entry(hs, rl, sei, iid, lname, unpad):
        if hs.shape[0] > thr:
            return orig(hs, rl, sei, iid, lname, unpad)
        if gate is not None:
            rl, _ = gate(hs)
        tw, ti = sel(hidden_states=hs, router_logits=rl, input_ids=iid)
        h = torch.ops.vllm.sluice_stream_gap(hs, ti, idx)
        kw = {}
        if w13_scale is not None:
            kw = {"w1_scale": w13_scale, "w2_scale": w2_scale,
                  "block_shape": list(block_shape or [128, 128])}
        routed = torch.ops.sluice.fused_experts(h, w13, w2, tw, ti, activation="silu",
                                                global_num_experts=gne, expert_map=emap, **kw)
        if shared_layer is None:
            return routed
        sh = shared_layer(sei if sei is not None else hs)
        return (sh, routed)

    return _forward_entry


# ---------------------------------------------------------------------------
# vllm::sluice_stream_gap
# ---------------------------------------------------------------------------
_ACTIVE_GAP: dict = {"offloader": None}


def _sluice_stream_gap_impl(hidden_states: torch.Tensor, topk_ids: torch.Tensor,
                            layer_idx: int) -> torch.Tensor:
    off = _ACTIVE_GAP["offloader"]
    if off is None:
        raise RuntimeError("vllm::sluice_stream_gap called with no active Sluice offloader")
    return off._router_split_gap(int(layer_idx), topk_ids, hidden_states)


def activate(offloader: ExpertStreamOffloader) -> None:
    """Make ``offloader`` the one ``vllm::sluice_stream_gap`` dispatches to
    (the op is process-global; the newest offloader is active by default)."""
    _ACTIVE_GAP["offloader"] = offloader


def _register_stream_gap_op(offloader: ExpertStreamOffloader) -> None:
    """Register ``vllm::sluice_stream_gap(Tensor hidden_states, Tensor topk_ids,
    int layer_idx) -> Tensor`` once per process (src/sluice/offloader.py:
    2296-2331); later offloaders rebind the implementation's target."""
    _ACTIVE_GAP["offloader"] = offloader
    if _ACTIVE_GAP.get("registered"):
        return
    try:
        from vllm.utils.torch_utils import direct_register_custom_op  # type: ignore

        def _fake(hidden_states, topk_ids, layer_idx):
            return torch.empty_like(hidden_states)

        direct_register_custom_op(op_name="sluice_stream_gap", op_func=_sluice_stream_gap_impl,
                                  mutates_args=[], fake_impl=_fake)
    except ImportError:
        if not hasattr(torch.ops.vllm, "sluice_stream_gap"):
            op = torch.library.custom_op("vllm::sluice_stream_gap", mutates_args=())(
                _sluice_stream_gap_impl)

            @op.register_fake
            def _(hidden_states, topk_ids, layer_idx):
                return torch.empty_like(hidden_states)
    _ACTIVE_GAP["registered"] = True
