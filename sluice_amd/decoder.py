"""Synthetic decode harness around the router-split path.

``SyntheticMoELayer`` has the module surface the offloader works on in vLLM
(src/sluice/offloader.py:491-505, 2495-2540): ``local_num_experts`` /
``global_num_experts`` / ``quant_method``, per-expert params ``w13_weight``
[E, 2I, H] (gate rows then up rows) and ``w2_weight`` [E, H, I], an
``expert_map`` property over the ``_expert_map`` buffer, and a ``runner``
with ``gate``, ``router.select_experts``, ``_shared_experts._layer``,
``moe_config.experts_per_token`` and a patchable ``_forward_entry``.  The
layer's forward is the runner's traced tail: shared + routed.

``build_offloaded`` runs the offloader lifecycle over such layers exactly as
vLLM would (wrap_modules -> post_init -> attach_model) with router-split on.

Weights are random (N(0, 0.02)); routing is the gate GEMM plus an optional
synthetic per-expert bias: log-Zipf(s) popularity over a seeded permutation
and, per step, rho-correlated AR(1) noise.
"""

import contextlib
import os
import types
from typing import Optional

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from sluice_amd import ops


class _QuantMethod:
    """Unquantized-method stand-in (not monolithic, applies expert_map)."""

    is_monolithic = False


class _SharedMLP(nn.Module):
    """Dense SwiGLU MLP (shared experts fused into one, intermediate I_s)."""

    def __init__(self, H: int, I_s: int, device, dtype, gen: torch.Generator):
        super().__init__()
        self.gate_up = nn.Parameter(
            (torch.randn((2 * I_s, H), generator=gen) * 0.02).to(dtype).to(device),
            requires_grad=False)
        self.down = nn.Parameter(
            (torch.randn((H, I_s), generator=gen) * 0.02).to(dtype).to(device),
            requires_grad=False)
        self.I_s = I_s

    def forward(self, x):
        gu = F.linear(x, self.gate_up)
        g, u = gu[:, : self.I_s], gu[:, self.I_s:]
        return F.linear(F.silu(g) * u, self.down)


class RoutingBias:
    """Per-layer synthetic router bias: log-Zipf popularity + AR(1) noise.

    The noise for every step is precomputed on the CPU from a seeded
    generator and uploaded once, so a captured graph reads step ``i``'s row
    through a device index."""

    def __init__(self, E: int, rows: int, steps: int, zipf_s: float, rho: float, sigma: float,
                 seed: int, device):
        rng = np.random.default_rng(seed)
        p = 1.0 / np.arange(1, E + 1) ** zipf_s
        p = p / p.sum()
        zipf = np.log(p[rng.permutation(E)]).astype(np.float32)
        z = np.zeros((steps, rows, E), np.float32)
        cur = rng.standard_normal((rows, E)).astype(np.float32)
        for t in range(steps):
            cur = rho * cur + np.sqrt(1 - rho * rho) * rng.standard_normal((rows, E)).astype(
                np.float32)
            z[t] = cur
        self.table = torch.from_numpy(zipf[None, None, :] + sigma * z).to(device)  # [steps,rows,E]
        self.step = torch.zeros((), dtype=torch.long, device=device)

    def __call__(self, T: int) -> torch.Tensor:
        return self.table.index_select(0, self.step.view(1))[0, :T]


class SyntheticMoELayer(nn.Module):
    def __init__(self, H: int, I: int, E: int, k: int, *, scoring: str = "softmax",
                 renorm: bool = False, routed_scale: float = 1.0, n_group: int = 1,
                 topk_group: int = 1, shared_I: int = 0, seed: int = 0,
                 device: Optional[torch.device] = None, dtype: torch.dtype = torch.bfloat16,
                 e_bias: bool = False, routing_bias: Optional[RoutingBias] = None,
                 weight_std: float = 0.02, name: str = "moe"):
        super().__init__()
        dev = device or torch.device("cuda", torch.cuda.current_device())
        gen = torch.Generator().manual_seed(1000 + seed)
        self.H, self.I, self.E, self.top_k = H, I, E, k
        self.layer_name = name
        self.global_num_experts = E
        self.local_num_experts = E
        self.quant_method = _QuantMethod()
        # Per-expert params are built on the CPU: the offloader keeps them in
        # the pinned host store and installs HBM slot buffers in their place.
        w13 = (torch.randn((E, 2 * I, H), generator=gen) * weight_std).to(dtype)
        w2 = (torch.randn((E, H, I), generator=gen) * weight_std).to(dtype)
        self.host_w13, self.host_w2 = w13, w2
        self.w13_weight = nn.Parameter(w13.clone(), requires_grad=False)
        self.w2_weight = nn.Parameter(w2.clone(), requires_grad=False)
        # the gate lives in a submodule, as in vLLM (it is not a per-expert param)
        self.gate = nn.Module()
        self.gate.weight = nn.Parameter(
            (torch.randn((E, H), generator=gen) * weight_std).to(dtype).to(dev),
            requires_grad=False)
        self.e_score_correction_bias = (
            nn.Parameter((torch.randn(E, generator=gen) * 0.01).to(dev), requires_grad=False)
            if e_bias else None)
        self.routing_bias = routing_bias
        self.scoring, self.renorm, self.routed_scale = scoring, renorm, routed_scale
        self.n_group, self.topk_group = n_group, topk_group
        self.shared = _SharedMLP(H, shared_I, dev, dtype, gen) if shared_I else None
        self.last_logits = self.last_ids = self.last_weights = None

        layer = self

        def gate(hs):
            logits = F.linear(hs, layer.gate.weight).float()
            if layer.routing_bias is not None:
                logits = logits + layer.routing_bias(hs.shape[0])
            return logits, None

        def select_experts(hidden_states, router_logits, input_ids=None):
            w, ids = ops.select_experts(
                router_logits, layer.top_k, scoring=layer.scoring, renormalize=layer.renorm,
                routed_scaling_factor=layer.routed_scale,
                e_score_correction_bias=layer.e_score_correction_bias,
                num_expert_group=layer.n_group, topk_group=layer.topk_group)
            layer.last_logits, layer.last_ids, layer.last_weights = router_logits, ids, w
            return w, ids

        def stock_entry(hs, rl, sei, iid, lname, unpad):
            raise RuntimeError(
                f"{lname}: {hs.shape[0]} tokens exceed the router-split envelope; larger steps "
                "need the classic wave path, which this build does not include")

        self.runner = types.SimpleNamespace(
            gate=gate,
            router=types.SimpleNamespace(select_experts=select_experts),
            _shared_experts=(types.SimpleNamespace(_layer=self.shared) if self.shared else None),
            moe_config=types.SimpleNamespace(experts_per_token=k, pcp_size=1),
            _forward_entry=stock_entry,
        )

    @property
    def expert_map(self):
        return self._buffers.get("_expert_map")

    def forward(self, hs: torch.Tensor) -> torch.Tensor:
        r = self.runner._forward_entry(hs, None, None, None, self.layer_name, False)
        if isinstance(r, tuple):
            sh, routed = r
            return routed + sh
        return r


@contextlib.contextmanager
def _env(**kv):
    old = {k: os.environ.get(k) for k in kv}
    try:
        for k, v in kv.items():
            os.environ[k] = str(v)
        yield
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def build_offloaded(layers, slots: int, device=None, fast_hit: bool = True,
                    protect_frac: float = 0.5, config=None):
    """Offload ``layers`` (SyntheticMoELayer) with router-split armed."""
    from sluice_amd.offloader import ExpertStreamOffloader

    dev = device or torch.device("cuda", torch.cuda.current_device())
    with _env(SLUICE_ROUTER_SPLIT=1, SLUICE_PIECEWISE=1, SLUICE_RS_FAST_HIT=int(fast_hit),
              SLUICE_PROTECT_FRAC=protect_frac):
        off = ExpertStreamOffloader(expert_cache_slots=slots)
    off.wrap_modules(iter(layers))
    with torch.cuda.device(dev):
        off.post_init(config)
    off.attach_model(nn.ModuleList(layers))
    return off
