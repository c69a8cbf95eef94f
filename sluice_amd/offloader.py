"""Routing-aware MoE expert streaming offloader, router-split path, on MI355X.

The drop-in for the reference's ``ExpertStreamOffloader``
(src/sluice/offloader.py:186-2814) on the router-split decode path: the same
lifecycle (``wrap_modules`` -> ``post_init`` -> ``attach_model``), env flags,
slot-buffer and expert-map layout, ``vllm::sluice_stream_gap`` op and
patched ``runner._forward_entry``.  Underneath, the per-layer slot cache and
the gap are native (libsluice_hip.so): a device kernel publishes the step's
selected experts into pinned host memory, the native SLRU assigns slots as
the reference's OrderedDict state machine does, missing experts stream as
SDMA copies on two copy engines, and the device installs the standing
expert map that the captured expert product reads by pointer.

Execution model per MoE layer per decode step (T <= thr tokens):

    gate + sluice::select_experts     [capturable; wave64 top-k kernel]
    -> vllm::sluice_stream_gap        [gap: lookup, SLRU, H2D, map]
    -> sluice::fused_experts          [capturable; slots + map by pointer]
    -> shared experts                 [capturable]

Steps above the envelope (more tokens than slots // top_k: prefill chunks,
large decode batches) take the stock path, whose ``quant_method.apply`` the
offloader wraps (src/sluice/offloader.py:1085-1122, 1452-1933): the native
planner syncs the ids once, plans one wave when the working set fits, else
wave 0 (hits + fills) and the leftover misses rotated through the probation
slots in ping-pong groups, and the expert product runs once per wave
against that wave's map; wave outputs are summed in fp32.
"""

import atexit
import ctypes
import json
import logging
import os
import time
from collections.abc import Generator
from dataclasses import dataclass, field
from typing import Any, Optional

import torch
import torch.nn as nn

from sluice_amd import _lib, ops

logger = logging.getLogger("sluice")

# Layer parameters with an expert dimension that are shared by every expert
# (correction bias, input scales, a hash-routing table), so never streamed
# (src/sluice/offloader.py:89-96).
NON_EXPERT_WEIGHTS = frozenset(
    {"e_score_correction_bias", "w13_input_scale", "w2_input_scale", "hash_indices_table"}
)

PROTECT_FRAC_ENV = "SLUICE_PROTECT_FRAC"
ROUTER_SPLIT_ENV = "SLUICE_ROUTER_SPLIT"
PIECEWISE_ENV = "SLUICE_PIECEWISE"
FAST_HIT_ENV = "SLUICE_RS_FAST_HIT"
NOOP_ENV = "SLUICE_RS_NOOP"
# Opt-in policies (src/sluice/offloader.py:97-118): LFU-ordered protected
# victims; per-expert selection counts dumped as JSONL snapshots; a static
# pin file {"layers": {"<MoE-layer ordinal>": [global ids]}}.
LFU_ENV = "SLUICE_LFU"
COUNTS_DIR_ENV = "SLUICE_EXPERT_COUNTS"
COUNTS_EVERY_ENV = "SLUICE_EXPERT_COUNTS_EVERY"
PIN_FILE_ENV = "SLUICE_PIN_FILE"
# Full residency with the streaming hook kept (src/sluice/offloader.py:289-293,
# 948-1012): every expert pre-filled into its own slot and pinned there.
NO_STATIC_FULL_ENV = "SLUICE_NO_STATIC_FULL"
# No counterpart in the reference: per router-split layer, how many experts
# the gap server keeps staged in HBM outside the slots (the layer's most
# selected experts it does not hold, copied while the host link idles; a
# miss on one is copied into its slot from HBM).  0 turns staging off.
STAGE_ROWS_ENV = "SLUICE_STAGE_ROWS"
STAGE_ROWS_DEFAULT = 6
# No counterpart in the reference: under the gap server, each router-split
# layer's bf16 expert rows also get a losslessly coded host store (12 bits
# per value plus rare escapes); misses copy the coded rows over the link and
# a decode kernel writes the exact rows into the slot.  0 turns it off.
CODEC_ENV = "SLUICE_CODEC"
CODEC_DEFAULT = 1
# Pinned host memory (GiB) the process may hold in host stores, uncoded and
# coded together: layers are coded in order while their coded stores fit.
# Default: a fifth of the host's memory (on MI355X boxes with 288 GiB,
# pinned allocations failed from 64-69 GiB, near a quarter of it).
CODEC_PIN_GB_ENV = "SLUICE_CODEC_PIN_GB"
CODEC_PIN_FRAC_DEFAULT = 0.2


def _codec_pin_gib() -> float:
    total = None
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemTotal:"):
                    total = int(line.split()[1]) * 1024
    except OSError:
        pass
    default = CODEC_PIN_FRAC_DEFAULT * total / 2**30 if total else 16.0
    return _env_number(CODEC_PIN_GB_ENV, default, float)

# Graph split points under piecewise capture: the MoE ops (whose apply runs
# the classic hook, which syncs the host) and the gap op.
_MOE_SPLIT_OPS = ("vllm::moe_forward", "vllm::moe_forward_shared")
_GAP_SPLIT_OP = "vllm::sluice_stream_gap"

try:  # vLLM's offloader base, when vLLM is installed (its isinstance checks)
    from vllm.model_executor.offloader.base import BaseOffloader as _OffloaderBase  # type: ignore
except Exception:  # noqa: BLE001 - vLLM absent or a different layout
    _OffloaderBase = object


def _env_flag(name: str) -> bool:
    return os.environ.get(name, "0") == "1"


def _env_number(name: str, default, cast):
    try:
        return cast(os.environ.get(name, default))
    except (TypeError, ValueError):
        return default


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
    # router-split layers: the expert product's plan, filled by each gap
    # kernel for ids of up to num_slots pairs (int32, device)
    plan: Optional[torch.Tensor] = None

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

    def step_stats(self) -> dict:
        """Real classic steps of this layer by class ("small" = pure decode,
        "scan"): steps, hit and missed local experts, waves."""
        out = (ctypes.c_int64 * 8)()
        _lib.check(_lib.load().sluice_layer_step_stats(self.handle, out),
                   "sluice_layer_step_stats")
        keys = ("steps", "hits", "misses", "waves")
        return {kind: {k: int(out[4 * i + j]) for j, k in enumerate(keys)}
                for i, kind in enumerate(("small", "scan"))}

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


# ---------------------------------------------------------------------------
# What the offloader reads from a layer and from the engine
# ---------------------------------------------------------------------------
def _expert_counts(module: nn.Module) -> Optional[tuple[int, int]]:
    """(global, local) expert counts of a FusedMoE-like layer (it carries
    both counts and a quant method), else None."""
    if not hasattr(module, "quant_method"):
        return None
    g = getattr(module, "global_num_experts", None)
    l = getattr(module, "local_num_experts", None)
    if g is None or l is None:
        return None
    return int(g), int(l)


def _streamed_params(module: nn.Module, local_n: int) -> dict:
    """The layer's own parameters with one row per local expert, except the
    ones every expert shares: what streams per expert."""
    out = {}
    for name, p in module.named_parameters(recurse=False):
        per_expert = p.dim() > 0 and p.shape[0] == local_n
        if per_expert and name not in NON_EXPERT_WEIGHTS:
            out[name] = p
    return out


def _module_device(module: nn.Module) -> torch.device:
    """Where the layer's resident tensors live (the current GPU when all of
    them are still on the host)."""
    tensors = [*module.parameters(recurse=False), *module.buffers(recurse=False)]
    devices = {t.device for t in tensors if t is not None and t.device.type != "cpu"}
    if devices:
        return next(iter(devices))
    return torch.device("cuda", torch.cuda.current_device() if torch.cuda.is_available() else 0)


@dataclass
class _EngineView:
    """The parts of a vLLM engine config the offloader acts on."""

    top_k: Optional[int] = None            # hf num_experts_per_tok
    max_batched_tokens: Optional[int] = None
    spec_tokens: int = 0                   # speculative draft depth
    compilation: Any = None                # compilation_config (splitting_ops)


def _engine_view(cfg) -> _EngineView:
    view = _EngineView()
    model = getattr(cfg, "model_config", None)
    hf = getattr(model, "hf_config", None)
    # multimodal checkpoints keep the language model's fields in text_config
    for src in (hf, getattr(hf, "text_config", None)):
        k = getattr(src, "num_experts_per_tok", None) if src is not None else None
        if k:
            view.top_k = int(k)
            break
    sched = getattr(cfg, "scheduler_config", None)
    mbt = getattr(sched, "max_num_batched_tokens", None)
    view.max_batched_tokens = int(mbt) if mbt is not None else None
    spec = getattr(cfg, "speculative_config", None)
    try:
        view.spec_tokens = max(int(getattr(spec, "num_speculative_tokens", 0) or 0), 0)
    except (TypeError, ValueError):
        view.spec_tokens = 0
    view.compilation = getattr(cfg, "compilation_config", None)
    return view


def _current_engine_config():
    """vLLM's current config; None when vLLM is not installed (the standalone
    harness drives the offloader).  An installed vLLM whose config cannot be
    read is an error: the router-split envelope could not be checked."""
    try:
        from vllm.config import get_current_vllm_config  # type: ignore
    except ImportError:
        return None
    try:
        cfg = get_current_vllm_config()
    except Exception as e:  # noqa: BLE001
        raise RuntimeError("Sluice: reading the vLLM engine config failed, so the expert-cache "
                           "settings cannot be checked; not starting.") from e
    if cfg is None:
        raise RuntimeError("Sluice: the vLLM engine config is None, so the expert-cache settings "
                           "cannot be checked; not starting.")
    return cfg


def _engine_step_signal() -> tuple:
    """(decode tokens, decode requests, real step) of the running step from
    vLLM's forward context (src/sluice/offloader.py:1766-1800): (None, None,
    False) for a dummy or profiling run without attention metadata; decode
    counts None when the backend publishes none."""
    try:
        from vllm.forward_context import get_forward_context  # type: ignore

        meta = getattr(get_forward_context(), "attn_metadata", None)
    except Exception:  # noqa: BLE001 - no engine, or no context set
        return None, None, False
    if isinstance(meta, dict):  # per-layer metadata: every layer agrees
        meta = next(iter(meta.values()), None)
    if meta is None:
        return None, None, False

    def as_int(v):
        try:
            return None if v is None else int(v)
        except (TypeError, ValueError):
            return None

    nd = as_int(getattr(meta, "num_decode_tokens", None))
    if nd is None:
        return None, None, True
    return nd, as_int(getattr(meta, "num_decodes", None)), True


def _process_rank() -> int:
    try:
        import torch.distributed as dist

        if dist.is_available() and dist.is_initialized():
            return dist.get_rank()
    except Exception:  # noqa: BLE001
        pass
    return _env_number("RANK", 0, int)


class _CountsJournal:
    """Per-expert selection counts of real classic steps, appended as one
    JSONL record per streaming layer every ``every`` hook ticks and at exit,
    to <directory>/expert_counts_rank<r>.jsonl.  The record keys are the
    reference's format (src/sluice/offloader.py:1399-1448).  Writing never
    raises: profiling must not take serving down."""

    def __init__(self, directory: str, every: int):
        self.directory = directory
        self.every = max(every, 1)
        self.ticks = 0
        self.snapshots = 0
        self._file = None

    def tick(self, layers) -> None:
        self.ticks += 1
        if self.ticks % self.every == 0:
            self.write(layers, final=False)

    def write(self, layers, final: bool) -> None:
        layers = [c for c in layers if not c.static_full and c.handle]
        if not layers:
            return
        try:
            if self._file is None:
                os.makedirs(self.directory, exist_ok=True)
                path = os.path.join(self.directory, f"expert_counts_rank{_process_rank()}.jsonl")
                self._file = open(path, "a")
            self.snapshots += 1
            states = [c.policy_state() for c in layers]
            totals = {"steps_small": sum(p["steps_small"] for p in states),
                      "steps_scan": sum(p["steps_scan"] for p in states)}
            for cache, pol in zip(layers, states):
                record = {
                    "snap": self.snapshots, "final": final, "ts": time.time(),
                    "hook_calls": self.ticks, **totals,
                    "layer": cache.ordinal, "layer_name": cache.layer_name,
                    "n_global": len(pol["counts_decode"]),
                    "decode": {str(g): n for g, n in enumerate(pol["counts_decode"]) if n},
                    "scan": {str(g): n for g, n in enumerate(pol["counts_scan"]) if n},
                }
                self._file.write(json.dumps(record) + "\n")
            self._file.flush()
        except Exception:  # noqa: BLE001
            logger.exception("Sluice: writing the expert-count snapshot failed; serving goes on.")


class _ClassicHook:
    """Takes the place of a layer's ``quant_method.apply``: calls that carry
    the step's routing (``layer`` and ``topk_ids``) go through the
    offloader's classic step; anything else goes straight to the original."""

    def __init__(self, offloader: "ExpertStreamOffloader", original):
        self.offloader = offloader
        self.original = original

    def __call__(self, *args, **kwargs):
        layer = kwargs["layer"] if "layer" in kwargs else (args[0] if args else None)
        topk_ids = kwargs.get("topk_ids")
        if layer is None or topk_ids is None:
            return self.original(*args, **kwargs)
        return self.offloader.run_moe(self.original, args, kwargs, layer, topk_ids)


# ---------------------------------------------------------------------------
# Routing settings of a layer -> the wave64 top-k kernel
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class RouteSpec:
    """Arguments of ``sluice::select_experts`` equivalent to a layer's router."""

    top_k: int
    scoring: str = "softmax"
    renormalize: bool = False
    scale: float = 1.0
    n_group: int = 1
    topk_group: int = 1
    bias: Optional[torch.Tensor] = None


def route_spec(module: nn.Module, runner=None) -> tuple[Optional[RouteSpec], str]:
    """Map a layer's router settings, read under vLLM's FusedMoE attribute
    names (on ``runner.router`` first, then on the layer), onto the routing
    kernel.  Returns (spec, "") or (None, reason) when the kernel cannot
    express the router exactly; such layers keep vLLM's select_experts.

    vLLM's select_experts (called at src/sluice/offloader.py:2583-2585) runs
    softmax top-k (``fused_topk``: selection on the logits, optional
    renormalisation, no scaling) or, with ``use_grouped_topk``,
    ``grouped_topk``: softmax or sigmoid scores, a group score that is the
    group's largest score without a correction bias and the sum of its two
    largest biased scores with one, the ``topk_group`` best groups eligible,
    renormalisation, then ``routed_scaling_factor``.  The kernel fixes the
    group score by the scoring (softmax: max; sigmoid + bias: top-2 sum), so
    the combinations it computes exactly are the ones accepted below."""
    router = getattr(runner, "router", None) if runner is not None else None

    def attr(name, default=None):
        for src in (router, module):
            if src is not None and hasattr(src, name):
                v = getattr(src, name)
                if v is not None:
                    return v
        return default

    top_k = attr("top_k")
    if top_k is None:
        mc = getattr(runner, "moe_config", None) if runner is not None else None
        top_k = getattr(mc, "experts_per_token", None)
    if top_k is None:
        return None, "router:no-top_k"
    top_k = int(top_k)
    n_experts = int(attr("global_num_experts", 0) or 0)
    if not 0 < top_k <= _lib.MAX_TOPK or not 0 < n_experts <= _lib.MAX_EXPERTS:
        return None, "router:shape"
    if attr("custom_routing_function") is not None:
        return None, "router:custom"
    if attr("apply_router_weight_on_input", False):
        return None, "router:weight-on-input"
    if getattr(module, "hash_indices_table", None) is not None:
        return None, "router:hash"
    scoring = str(attr("scoring_func", "softmax"))
    if scoring not in ("softmax", "sigmoid"):
        return None, f"router:scoring-{scoring}"
    bias = attr("e_score_correction_bias")
    renorm = bool(attr("renormalize", False))
    if not attr("use_grouped_topk", False):
        if scoring != "softmax" or bias is not None:
            return None, "router:ungrouped-sigmoid-or-bias"
        return RouteSpec(top_k, "softmax", renorm), ""
    n_group = int(attr("num_expert_group", 1) or 1)
    topk_group = int(attr("topk_group", 1) or 1)
    if n_group < 1 or n_experts % n_group or not 1 <= topk_group <= n_group:
        return None, "router:groups"
    scale = float(attr("routed_scaling_factor", 1.0) or 1.0)
    if scoring == "softmax" and bias is not None:
        return None, "router:softmax-bias"
    if scoring == "sigmoid" and bias is None and n_group > 1:
        return None, "router:sigmoid-no-bias"
    return RouteSpec(top_k, scoring, renorm, scale, n_group, topk_group, bias), ""


# ---------------------------------------------------------------------------
# The offloader
# ---------------------------------------------------------------------------
class ExpertStreamOffloader(_OffloaderBase):
    """Stream routed-expert weights host->HBM per decode step, by routing.

    Args:
        expert_cache_slots: HBM-resident expert slots per MoE layer.
    """

    def __init__(self, expert_cache_slots: int):
        if expert_cache_slots <= 0:
            raise ValueError("expert_cache_slots must be positive")
        self.expert_cache_slots = expert_cache_slots
        frac = _env_number(PROTECT_FRAC_ENV, 0.5, float)
        self.protect_frac = min(max(frac, 0.0), 0.9)
        self.piecewise = _env_flag(PIECEWISE_ENV)
        self.router_split = _env_flag(ROUTER_SPLIT_ENV)
        self._rs_fast_hit = _env_flag(FAST_HIT_ENV)
        self._rs_noop = _env_flag(NOOP_ENV)
        if self._rs_noop:
            logger.warning("Sluice: %s=1 turns the gap into a no-op for timing; the expert map "
                           "goes stale and layer outputs are WRONG.", NOOP_ENV)
        self.pin_memory = torch.cuda.is_available()
        self.lfu = _env_flag(LFU_ENV)
        self.no_static_full = _env_flag(NO_STATIC_FULL_ENV)
        self.stage_rows = min(max(_env_number(STAGE_ROWS_ENV, STAGE_ROWS_DEFAULT, int), 0), 8)
        self.codec = _env_number(CODEC_ENV, CODEC_DEFAULT, int) != 0
        self._caches: dict[int, _ExpertLayerCache] = {}
        self._layers: list[nn.Module] = []
        self._prepared_stores: dict[int, list] = {}  # pinned stores made before load
        self._rs_caches: list[_ExpertLayerCache] = []
        self._rs_gaps = 0
        self._rs_layers = 0
        self._rs_thr: Optional[int] = None
        self._rs_routes: list = []  # per armed layer: RouteSpec or None (vLLM routes)
        self._server: Optional[int] = None
        self._spec_tokens = 0
        self._signal: Optional[tuple] = None
        self._warned_waves = False
        self._counts_dir = os.environ.get(COUNTS_DIR_ENV) or None
        self._counts: Optional[_CountsJournal] = None
        if self._counts_dir:
            self._counts = _CountsJournal(self._counts_dir,
                                          _env_number(COUNTS_EVERY_ENV, 5000, int))
            atexit.register(self._dump_expert_counts, True)
        self._pin_layers: Optional[dict] = None
        self._pin_stats = [0, 0]  # experts pinned, layers with pins
        pin_path = os.environ.get(PIN_FILE_ENV)
        if pin_path:
            self._pin_layers = _read_pin_file(pin_path)
        if self.router_split:
            _register_stream_gap_op(self)
        logger.info("Sluice: offloader on, %d HBM expert slots per MoE layer "
                    "(protect_frac %.2f).", expert_cache_slots, self.protect_frac)

    # -- model construction -------------------------------------------------
    def wrap_modules(self, modules_generator: Generator) -> list:
        """Pass the model's modules through, moving every MoE layer's
        per-expert params to host memory before the checkpoint loads."""
        modules = []
        for module in modules_generator:
            for sub in module.modules():
                if _expert_counts(sub) is not None:
                    self._prepare_layer(sub)
            modules.append(module)
        return modules

    def _prepare_layer(self, module: nn.Module) -> None:
        """A layer's (still empty) per-expert params become host tensors
        before the checkpoint loads (src/sluice/offloader.py:554-571).  With a
        GPU present they are views of exact-size pinned host stores, so the
        loader writes straight into the memory the expert rows stream from,
        and _install_cache adopts it without a second host copy.  Layers whose
        kernel does not read the expert map (monolithic quant methods, the
        ROCm AITER fused MoE) stay as they are."""
        qm = module.quant_method
        if qm is None or getattr(qm, "is_monolithic", False) or getattr(
                module, "rocm_aiter_fmoe_enabled", False):
            return
        _, local_n = _expert_counts(module)
        params = _streamed_params(module, local_n)
        if not params:
            return
        for p in params.values():
            host = p.data.to("cpu") if p.data.device.type != "cpu" else p.data
            if self.pin_memory and ops.host_store_of(host) is None:
                store = ops.HostStore(tuple(host.shape), host.dtype)
                store.tensor.copy_(host)
                self._prepared_stores.setdefault(id(module), []).append(store)
                host = store.tensor
            p.data = host
        if not any(m is module for m in self._layers):
            self._layers.append(module)

    # -- after load -----------------------------------------------------------
    def post_init(self, config=None) -> None:
        """Apply the engine settings, then install every prepared layer's slot
        cache and classic hook (src/sluice/offloader.py:575-657)."""
        cfg = config if config is not None else _current_engine_config()
        if cfg is not None:
            self._apply_engine(_engine_view(cfg))
        if torch.cuda.is_available():
            torch.cuda.synchronize()
        for module in self._layers:
            self._install_cache(module)
            self._install_classic_hook(module)
        streaming = [c for c in self._caches.values() if not c.static_full]
        if self._caches:
            host = sum(c.bytes_per_expert * c.local_num_experts for c in streaming)
            hbm = sum(c.bytes_per_expert * c.num_slots for c in self._caches.values())
            logger.info("Sluice: %d MoE layers (%d streaming); %.1f GiB of experts in %s host "
                        "memory, %.1f GiB of HBM slots.", len(self._caches), len(streaming),
                        host / 2**30, "pinned" if self.pin_memory else "pageable", hbm / 2**30)

    def _apply_engine(self, view: _EngineView) -> None:
        """What the engine config decides (src/sluice/offloader.py:786-851):
        the speculative depth the decode classifier needs; under piecewise
        capture, the split points that keep the hooks eager; and under
        router-split, the token threshold slots // top_k, which must bound
        every batch, since the traced entry's size branch is fixed at trace
        time."""
        self._spec_tokens = view.spec_tokens
        if not self.piecewise:
            return
        cc = view.compilation
        if cc is not None:
            wanted = list(_MOE_SPLIT_OPS) + ([_GAP_SPLIT_OP] if self.router_split else [])
            have = list(getattr(cc, "splitting_ops", None) or [])
            cc.splitting_ops = have + [op for op in wanted if op not in have]
        if not self.router_split:
            return
        thr = max(1, self.expert_cache_slots // (view.top_k or 8))
        self._rs_thr = thr
        mbt = view.max_batched_tokens
        if mbt is not None and mbt > thr:
            # the message is a contract: operators act on it
            raise RuntimeError(
                "Sluice router-split under piecewise compiles a single trace whose size "
                "branch is resolved at trace time; the whole batch envelope must fit it. "
                f"Got max_num_batched_tokens={mbt} > slots//topk={thr}. Set "
                f"--max-num-batched-tokens {thr} (prefill runs in {thr}-token chunks) or "
                "raise SLUICE_SLOTS.")

    def _install_cache(self, module: nn.Module) -> None:
        """Slot buffers [S, ...] as the live params, a pinned host store of
        every local expert, the expert map and the native slot cache
        (src/sluice/offloader.py:895-1044)."""
        lib = _lib.load()
        global_n, local_n = _expert_counts(module)
        per_expert = _streamed_params(module, local_n)
        if not per_expert:
            return
        device = _module_device(module)
        num_slots = min(self.expert_cache_slots, local_n)
        protected_cap = max(min(int(num_slots * self.protect_frac), num_slots - 1), 0)
        cache = _ExpertLayerCache(local_num_experts=local_n, num_slots=num_slots,
                                  protected_cap=protected_cap, device=device,
                                  param_names=list(per_expert.keys()))
        cache.static_full = num_slots >= local_n and not self.no_static_full
        # capacity for every expert but the hook kept on: all of them are
        # loaded once here and pinned, so nothing ever streams
        prefill_resident = num_slots >= local_n and not cache.static_full
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
            if self.lfu or self._counts is not None:
                _lib.check(lib.sluice_layer_set_policy(cache.handle, int(self.lfu),
                                                       int(self._counts is not None)),
                           "sluice_layer_set_policy")
            if prefill_resident:
                slot = ctypes.c_int()
                for local in range(local_n):
                    _lib.check(lib.sluice_layer_pin(cache.handle, local, 0, ctypes.byref(slot)),
                               "sluice_layer_pin")
                    if slot.value != local:
                        raise RuntimeError(f"Sluice: full-residency pre-fill put expert {local} "
                                           f"in slot {slot.value}")
                for name in cache.param_names:
                    cache.gpu_cache[name][:local_n].copy_(cache.cpu_store[name])
                cache.pinned_slots.update(range(local_n))
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
                logger.warning("Sluice: MoE layer %d lists %d pins but its protected budget is "
                               "%d; the first %d are pinned.", ordinal, len(wanted), budget, n)
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
    def _dump_expert_counts(self, final: bool) -> None:
        if self._counts is not None:
            self._counts.write(list(self._caches.values()), final)

    # -- classic (wave) path -------------------------------------------------
    def _install_classic_hook(self, module: nn.Module) -> None:
        """Route the layer's ``quant_method.apply`` (the stock path that
        steps above the router-split envelope take) through the classic hook
        (src/sluice/offloader.py:1085-1122).  Under piecewise capture the hook
        runs outside any traced region, since it syncs the host."""
        qm = getattr(module, "quant_method", None)
        if qm is None or getattr(qm, "_sluice_hook", None) is not None:
            return
        original = getattr(qm, "apply", None)
        if original is None:
            return
        hook = _ClassicHook(self, original)
        qm._sluice_hook = hook
        qm.apply = torch._dynamo.disable(hook) if self.piecewise else hook

    def set_step_signal(self, nd: Optional[int], ndec: Optional[int],
                        real_step: bool = True) -> None:
        """Publish the step's decode split for engines without vLLM's forward
        context: rows [0, nd) are decode tokens of ndec requests (None: not
        published); real_step False marks a dummy run."""
        self._signal = (nd, ndec, bool(real_step))

    def clear_step_signal(self) -> None:
        self._signal = None

    def _split_signal(self) -> tuple:
        """``(num_decode_tokens, num_decodes, is_real_step)``: the signal set
        with set_step_signal, else vLLM's forward context."""
        return self._signal if self._signal is not None else _engine_step_signal()

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
            raise RuntimeError("Sluice: the classic streaming hook syncs the host and cannot run "
                               "inside a captured graph; capture piecewise (SLUICE_PIECEWISE=1) "
                               "or run eagerly.")
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
        if self._counts is not None and real_step:
            # the profiling clock ticks once per real hook call that selected
            # experts (the steps the layer classified)
            pol = cache.policy_state()
            seen = pol["steps_small"] + pol["steps_scan"]
            if seen != cache.policy_steps:
                cache.policy_steps = seen
                self._counts.tick(list(self._caches.values()))
        if n_waves > 1 and real_step and not self._warned_waves:
            self._warned_waves = True
            logger.warning("Sluice: a step needs more local experts than the %d usable slots; "
                           "it runs in %d waves, summed in fp32 (exact in math, not the bits of "
                           "one launch). More SLUICE_SLOTS avoids waves.", cache.num_slots,
                           n_waves)
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
        """Called by the plugin once the model is loaded."""
        self.attach_router_split(model)

    def attach_router_split(self, model: nn.Module) -> None:
        """Patch every eligible layer's ``runner._forward_entry`` with the
        traced split path (src/sluice/offloader.py:2469-2635).  Layers
        without the needed seams keep the stock path (counted in the skip
        census); layers whose router the routing kernel cannot express keep
        vLLM's select_experts inside the split path (counted as well)."""
        if not self.router_split:
            return
        skips: dict = {}
        seen = 0
        for module in model.modules():
            cache = self._caches.get(id(module))
            if cache is None:
                continue
            seen += 1
            runner = getattr(module, "runner", None)
            reason = _split_ineligible(runner, cache)
            if reason is not None:
                skips[reason] = skips.get(reason, 0) + 1
                continue
            spec, why = route_spec(module, runner)
            if spec is None:
                skips[why] = skips.get(why, 0) + 1  # armed, routed by vLLM
            idx = len(self._rs_caches)
            self._rs_caches.append(cache)
            self._rs_routes.append(spec)
            if cache.plan is None and not self._rs_noop:
                cache.plan = torch.zeros(_lib.load().sluice_moe_plan_ints(1, cache.num_slots),
                                         dtype=torch.int32, device=cache.device)
            top_k = spec.top_k if spec is not None else _runner_top_k(module, runner)
            thr = self._rs_thr
            if thr is None:  # eager: a per-step branch, capped at 16 tokens
                thr = max(1, min(16, self.expert_cache_slots // top_k))
            runner._forward_entry = _split_entry(_LayerBinding(
                idx=idx, thr=thr, w13=module.w13_weight, w2=module.w2_weight,
                global_n=_expert_counts(module)[0], expert_map=cache.expert_map_buf,
                gate=getattr(runner, "gate", None), route=spec,
                vllm_select=runner.router.select_experts if spec is None else None,
                stock=runner._forward_entry, shared=_shared_layer(runner),
                quant=_quant_kwargs(module), plan=cache.plan, plan_pairs=cache.num_slots))
        self._rs_layers = len(self._rs_caches)
        kernel = sum(1 for r in self._rs_routes if r is not None)
        logger.warning("Sluice: ROUTER-SPLIT armed on %d/%d MoE layers (%d routed by the wave64 "
                       "top-k kernel). skips=%s", self._rs_layers, seen, kernel, skips or "{}")

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
                logger.warning("Sluice gap: %d router-split layers, %d gaps, %d misses, %d "
                               "fast hits%s", len(self._rs_caches), self._rs_gaps, c["misses"],
                               c["fast_hits"], " [no-op gap: outputs invalid]"
                               if self._rs_noop else "")
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
        plan = self.gap_plan(idx, ids.numel())
        rc = lib.sluice_layer_gap_launch(cache.handle, ids.data_ptr(), ids.numel(), src, dst,
                                         nbytes, None if plan is None else plan.data_ptr(),
                                         stream)
        _lib.check(rc, "sluice_layer_gap_launch")
        if self._server is None:
            rc = lib.sluice_layer_gap_serve(cache.handle, int(self._rs_fast_hit), stream)
            _raise_gap(rc, "sluice_layer_gap_serve")
        return out

    def gap_plan(self, idx: int, n_pairs: int) -> Optional[torch.Tensor]:
        """The buffer router-split layer ``idx``'s gap fills with the expert
        product's plan for ids of ``n_pairs`` pairs (the product then needs
        no align launch), or None when its gap builds none."""
        cache = self._rs_caches[idx]
        if cache.plan is None or n_pairs > cache.num_slots:
            return None
        return cache.plan

    # -- gap server ---------------------------------------------------------------
    def start_gap_server(self) -> None:
        """Serve every router-split layer's gap records on a native thread:
        the gap op becomes a pure device launch (capturable), so a whole
        decode step, gaps included, can replay as one hipGraph.  Slot
        assignment and maps are the same as with inline gaps."""
        if self._server is not None or not self._rs_caches:
            return
        lib = _lib.load()
        coding = self.codec
        if coding:
            # what coded stores may still take of the pinned budget
            room = (_codec_pin_gib() * 2**30 - ops.pinned_store_bytes()
                    - sum(self._layer_codec(c)["coded_bytes"] for c in self._rs_caches))
        for c in self._rs_caches:
            # the coded store and staging only speed the path up: without
            # them (no pinned memory left, no copy engines free, no HBM left)
            # the layer streams as before
            if coding and self._layer_codec(c)["params"] == 0:
                bf16 = [i for i, n in enumerate(c.param_names)
                        if c.gpu_cache[n].dtype == torch.bfloat16]
                # coded rows take ~0.75 of the rows (12 bits per value)
                need = 0.76 * c.local_num_experts * sum(
                    c.gpu_cache[c.param_names[i]][0].nbytes for i in bf16)
                rc = (lib.sluice_layer_set_codec(c.handle, sum(1 << i for i in bf16))
                      if need <= room else _lib.SLUICE_E_NOMEM)
                if rc != 0:
                    coding = False  # this layer and the ones after it stream uncoded rows
                    logger.warning("Sluice: layer %s and later ones stream uncoded rows (%s=1, "
                                   "%s=%.1f): %s", c.layer_name or c.ordinal, CODEC_ENV,
                                   CODEC_PIN_GB_ENV, _codec_pin_gib(), _lib.strerror(rc))
                else:
                    room -= self._layer_codec(c)["coded_bytes"]
            rc = lib.sluice_layer_set_staging(c.handle, self.stage_rows)
            if rc != 0:
                logger.warning("Sluice: layer %s runs without staging rows (%s=%d): %s",
                               c.layer_name or c.ordinal, STAGE_ROWS_ENV, self.stage_rows,
                               _lib.strerror(rc))
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

    def reset_gaps(self) -> None:
        """After a gap raised (overflow, a timed-out or aborted wait) and the
        caller has handled it: synchronise the device, stop the gap server
        (dropping the error it kept), clear the abort flag and line every
        router-split layer's host stamps up with the device's, then restart
        the server if one was running.  Slot state is what the served records
        left; the outputs of the failed steps are invalid.  No counterpart in
        the reference, whose gap errors end the engine."""
        torch.cuda.synchronize()
        lib = _lib.load()
        restart = self._server is not None
        if restart:
            srv, self._server = self._server, None
            lib.sluice_gap_server_destroy(srv)  # returns the error already raised
        _lib.check(lib.sluice_gap_abort(0), "sluice_gap_abort")
        for c in self._rs_caches:
            _lib.check(lib.sluice_layer_gap_resync(c.handle), "sluice_layer_gap_resync")
        if restart:
            self.start_gap_server()

    # -- stats ----------------------------------------------------------------
    def gap_counters(self) -> dict:
        """Router-split gap counters summed over the armed layers."""
        tot = {"gaps": 0, "misses": 0, "fast_hits": 0, "map_writes": 0, "bytes": 0}
        for c in self._rs_caches:
            for k_, v in c.stats().items():
                tot[k_] += v
        return tot

    def stage_counters(self) -> dict:
        """Staging rows summed over the armed layers: rows, rows holding an
        expert whole, rows filled, host-to-device bytes of staging copies,
        misses copied into their slots from a staged row, and their bytes."""
        lib = _lib.load()
        keys = ("rows", "ready", "filled", "h2d_bytes", "hits", "hit_bytes")
        tot = dict.fromkeys(keys, 0)
        ctr = (ctypes.c_int64 * 6)()
        for c in self._rs_caches:
            _lib.check(lib.sluice_layer_stage_counters(c.handle, ctr), "sluice_layer_stage_counters")
            for i, k_ in enumerate(keys):
                tot[k_] += ctr[i]
        return tot

    @staticmethod
    def _layer_codec(c) -> dict:
        """One layer's coded store: params coded and bytes of its coded rows."""
        ctr = (ctypes.c_int64 * 6)()
        _lib.check(_lib.load().sluice_layer_codec_counters(c.handle, ctr),
                   "sluice_layer_codec_counters")
        return {"params": ctr[0], "coded_bytes": ctr[2]}

    def codec_counters(self) -> dict:
        """Coded host stores summed over the armed layers: params coded,
        bytes of one expert's coded params as rows (summed over layers),
        bytes of every local expert's coded rows and (store_bytes) of the
        same rows uncoded, bytes of the slot fills' copies over the link
        (coded or not), decode jobs, and those that decoded a staging row."""
        lib = _lib.load()
        keys = ("params", "row_bytes", "coded_bytes", "link_bytes", "decodes", "decodes_staged")
        tot = dict.fromkeys(keys, 0)
        tot["store_bytes"] = 0  # the coded params' rows of every local expert, uncoded
        tot["layers"] = 0  # layers with a coded store
        ctr = (ctypes.c_int64 * 6)()
        for c in self._rs_caches:
            _lib.check(lib.sluice_layer_codec_counters(c.handle, ctr), "sluice_layer_codec_counters")
            for i, k_ in enumerate(keys):
                tot[k_] += ctr[i]
            tot["store_bytes"] += ctr[1] * c.local_num_experts
            tot["layers"] += ctr[0] > 0
        return tot

    def get_gap_stats(self) -> dict:
        """The router-split gap's own counters (the reference keeps them
        outside get_stats: src/sluice/offloader.py:349-351, 2456)."""
        return {"layers": len(self._rs_caches), **self.gap_counters()}

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
        """Classic-step stats per class, in the reference's schema
        (src/sluice/offloader.py:2804-2814): {"small": {...}, "scan": {...}},
        each {steps, hits, misses, bytes, waves} summed over the streaming
        layers ("small" = pure decode steps)."""
        out = {kind: {"steps": 0, "hits": 0, "misses": 0, "bytes": 0, "waves": 0}
               for kind in ("small", "scan")}
        for c in self._caches.values():
            if not c.handle or c.static_full:
                continue
            for kind, st in c.step_stats().items():
                acc = out[kind]
                for key in ("steps", "hits", "misses", "waves"):
                    acc[key] += st[key]
                acc["bytes"] += st["misses"] * c.bytes_per_expert
        return out

    def close(self) -> None:
        """Stop the gap server, destroy the native layers and drop this
        offloader's references to host stores and layers (the slot buffers
        live on as the layers' params while the model does); the gap op no
        longer dispatches here."""
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
            c.cpu_store.clear()
            c.host_stores.clear()
        self._prepared_stores.clear()
        self._layers.clear()
        if _ACTIVE_GAP.get("offloader") is self:
            _ACTIVE_GAP["offloader"] = None


def _read_pin_file(path: str) -> dict:
    """{MoE-layer ordinal: [global expert ids]} from a pin file (the ids
    under "layers", or at the top level); a malformed file fails loudly."""
    with open(path) as f:
        raw = json.load(f)
    layers = raw.get("layers", raw)
    pins = {int(k_): [int(g) for g in v] for k_, v in layers.items()}
    logger.info("Sluice: pin file %s lists experts for %d layers.", path, len(pins))
    return pins


def _raise_gap(rc: int, what: str) -> None:
    if rc == _lib.SLUICE_E_OVERFLOW:
        # the message is a contract: callers match on it
        raise RuntimeError("Sluice router-split: working set exceeds slots on a "
                           "decode-sized step; raise SLUICE_SLOTS.")
    _lib.check(rc, what)


# ---------------------------------------------------------------------------
# The router-split entry
# ---------------------------------------------------------------------------
# Runner seams whose absence (or whose variants) the split entry cannot take;
# such layers keep the stock path (src/sluice/offloader.py:2499-2538).
def _split_ineligible(runner, cache: _ExpertLayerCache) -> Optional[str]:
    if runner is None:
        return "no-runner"
    if cache.static_full:
        return "static-full"
    checks = (
        ("monolithic", lambda r: getattr(getattr(r, "_quant_method", None), "is_monolithic",
                                         False)),
        ("fused-gate", lambda r: getattr(r, "gate", None) is not None
         and getattr(r, "_fse_fuse_gate", False)),
        ("naive-dispatch", lambda r: getattr(r, "do_naive_dispatch_combine", False)),
        ("pcp", lambda r: (getattr(getattr(r, "moe_config", None), "pcp_size", 1) or 1) > 1),
        ("no-router", lambda r: getattr(getattr(r, "router", None), "select_experts",
                                        None) is None),
        ("no-entry", lambda r: getattr(r, "_forward_entry", None) is None),
    )
    for reason, bad in checks:
        if bad(runner):
            return reason
    return None


def _runner_top_k(module, runner) -> int:
    mc = getattr(runner, "moe_config", None)
    k = getattr(mc, "experts_per_token", None) or getattr(module, "top_k", None)
    return int(k or 8)


def _shared_layer(runner):
    se = getattr(runner, "_shared_experts", None)
    return getattr(se, "_layer", None) if se is not None else None


def _quant_kwargs(module) -> dict:
    """fused_experts keywords of a block-quantised (fp8) layer."""
    s13 = getattr(module, "w13_weight_scale", None)
    if s13 is None:
        return {}
    return {"w1_scale": s13, "w2_scale": getattr(module, "w2_weight_scale", None),
            "block_shape": list(getattr(module, "block_shape", None) or [128, 128])}


@dataclass
class _LayerBinding:
    """One layer's tensors and callables, bound into its entry.  The weights
    and the map are held BY POINTER: the gap rewrites their contents."""

    idx: int
    thr: int
    w13: torch.Tensor
    w2: torch.Tensor
    global_n: int
    expert_map: torch.Tensor
    gate: Any
    route: Optional[RouteSpec]
    vllm_select: Any
    stock: Any
    shared: Any
    quant: dict
    plan: Optional[torch.Tensor] = None  # filled by the layer's gap (ids of <= plan_pairs)
    plan_pairs: int = 0


def _split_entry(b: _LayerBinding):
    """The traced ``runner._forward_entry`` of one layer
    (src/sluice/offloader.py:2578-2603): batches above the threshold take the
    stock entry; others run gate -> routing -> gap op -> expert product ->
    shared experts, returning (shared, routed) or routed."""
    idx, thr, gate, route = b.idx, b.thr, b.gate, b.route
    w13, w2, emap, gne, quant = b.w13, b.w2, b.expert_map, b.global_n, b.quant
    stock, select, shared = b.stock, b.vllm_select, b.shared
    plan, plan_pairs = b.plan, b.plan_pairs

    def _forward_entry(hs, rl, sei, iid, lname, unpad):
        if hs.shape[0] > thr:
            return stock(hs, rl, sei, iid, lname, unpad)
        if gate is not None:
            rl, _ = gate(hs)
        if route is not None:
            tw, ti = torch.ops.sluice.select_experts(
                rl, route.top_k, route.scoring, route.renormalize, route.scale, route.bias,
                route.n_group, route.topk_group)
        else:
            tw, ti = select(hidden_states=hs, router_logits=rl, input_ids=iid)
        h = torch.ops.vllm.sluice_stream_gap(hs, ti, idx)
        # the gap op built the product's plan of ti over the map it left
        # (its output h orders the product after it)
        p = plan if plan is not None and ti.numel() <= plan_pairs else None
        routed = torch.ops.sluice.fused_experts(h, w13, w2, tw, ti, activation="silu",
                                                global_num_experts=gne, expert_map=emap,
                                                plan=p, **quant)
        if shared is None:
            return routed
        return (shared(sei if sei is not None else hs), routed)

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
