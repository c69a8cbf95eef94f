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
    """Unquantized-method stand-in (not monolithic, applies expert_map): its
    ``apply`` is the fused-MoE kernel call of vLLM's stock path, which the
    offloader wraps with the classic hook."""

    is_monolithic = False

    def apply(self, layer, x, topk_weights, topk_ids, **kw):
        scale = getattr(layer, "w13_weight_scale", None)
        extra = {}
        if scale is not None:
            extra = dict(w1_scale=scale, w2_scale=layer.w2_weight_scale,
                         block_shape=list(getattr(layer, "block_shape", None) or [128, 128]))
        return ops.fused_experts(x, layer.w13_weight, layer.w2_weight, topk_weights, topk_ids,
                                 global_num_experts=layer.global_num_experts,
                                 expert_map=layer.expert_map, **extra)


def _stock_entry(layer, gate, select_experts):
    """vLLM's stock MoE entry as a runner's ``_forward_entry``: gate, top-k,
    ``quant_method.apply`` (the classic hook once offloaded), then shared."""

    def stock_entry(hs, rl, sei, iid, lname, unpad):
        if gate is not None:
            rl, _ = gate(hs)
        tw, ti = select_experts(hidden_states=hs, router_logits=rl, input_ids=iid)
        routed = layer.quant_method.apply(layer=layer, x=hs, topk_weights=tw, topk_ids=ti)
        if layer.shared is None:
            return routed
        return (layer.shared(sei if sei is not None else hs), routed)

    return stock_entry


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

    table[t, r, e] = ln p(e) + sigma * z_t[r, e]: p a Zipf(zipf_s)
    popularity over a seeded permutation of the experts, z_t per row
    (sequence) an AR(1) process z_t = rho z_{t-1} + sqrt(1 - rho^2) eps_t
    with unit variance.  Every step's row is precomputed on the CPU from a
    seeded generator and uploaded once, so a captured graph reads step
    ``i``'s row through a device index; ``refill`` rewrites the table in
    place (captured graphs keep reading it)."""

    def __init__(self, E: int, rows: int, steps: int, zipf_s: float, rho: float, sigma: float,
                 seed: int, device, step: Optional[torch.Tensor] = None):
        self.table = torch.empty((steps, rows, E), dtype=torch.float32, device=device)
        self.step = step if step is not None else torch.zeros((), dtype=torch.long, device=device)
        self.refill(zipf_s, rho, sigma, seed)

    def refill(self, zipf_s: float, rho: float, sigma: float, seed: int) -> None:
        steps, rows, E = self.table.shape
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
        self.table.copy_(torch.from_numpy(zipf[None, None, :] + sigma * z))
        self.knobs = {"zipf_s": zipf_s, "rho": rho, "sigma": sigma, "seed": seed}

    def fill_uniform(self, gen: torch.Generator, scale: float = 10.0) -> None:
        """Large i.i.d. noise in every entry: uniform top-k routing."""
        self.table.normal_(generator=gen)
        self.table.mul_(scale)
        self.knobs = {"uniform": True, "scale": scale}

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
        _router_attrs(self, scoring, renorm, routed_scale, n_group, topk_group)
        self.shared = _SharedMLP(H, shared_I, dev, dtype, gen) if shared_I else None
        # the last router logits (the gate records them); ids and weights when
        # vLLM's select_experts stand-in routed the step (the stock path)
        self.last_logits = self.last_ids = self.last_weights = None

        layer = self

        def gate(hs):
            logits = F.linear(hs, layer.gate.weight).float()
            if layer.routing_bias is not None:
                logits = logits + layer.routing_bias(hs.shape[0])
            layer.last_logits, layer.last_ids, layer.last_weights = logits, None, None
            return logits, None

        def select_experts(hidden_states, router_logits, input_ids=None):
            w, ids = ops.select_experts(
                router_logits, layer.top_k, scoring=layer.scoring, renormalize=layer.renorm,
                routed_scaling_factor=layer.routed_scale,
                e_score_correction_bias=layer.e_score_correction_bias,
                num_expert_group=layer.n_group, topk_group=layer.topk_group)
            layer.last_logits, layer.last_ids, layer.last_weights = router_logits, ids, w
            return w, ids

        self.runner = types.SimpleNamespace(
            gate=gate,
            router=types.SimpleNamespace(select_experts=select_experts),
            _shared_experts=(types.SimpleNamespace(_layer=self.shared) if self.shared else None),
            moe_config=types.SimpleNamespace(experts_per_token=k, pcp_size=1),
            _forward_entry=_stock_entry(self, gate, select_experts),
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


def _router_attrs(layer, scoring, renorm, routed_scale, n_group, topk_group):
    """The router settings under vLLM's FusedMoE attribute names, which the
    offloader maps onto the routing kernel (grouped top-k when the experts
    are split into groups; the correction bias is the layer's
    e_score_correction_bias)."""
    layer.scoring_func = scoring
    layer.renormalize = renorm
    layer.use_grouped_topk = n_group > 1
    layer.num_expert_group = n_group
    layer.topk_group = topk_group
    layer.routed_scaling_factor = routed_scale
    layer.custom_routing_function = None


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


# ---------------------------------------------------------------------------
# Synthetic decoder: model shapes, attention, graph pieces around the gap.
# ---------------------------------------------------------------------------
SPECS = {
    # DeepSeek-V2-Lite: 27 layers (layer 0 dense), MLA attention, 64 routed
    # experts top-6 (softmax greedy, no renorm) + 2 shared experts.
    "v2lite": dict(vocab=102400, H=2048, layers=27, first_dense=1, dense_I=10944, E=64, k=6,
                   I=1408, shared_I=2816, scoring="softmax", renorm=False, routed_scale=1.0,
                   n_group=1, topk_group=1, e_bias=False, attn="mla", heads=16, kv_lora=512,
                   qk_nope=128, qk_rope=64, v_head=128, rope_theta=10000.0, fp8=False),
    # Qwen3-30B-A3B: 48 MoE layers, GQA 32/4 heads of 128 with q/k norm,
    # 128 experts top-8 (softmax + renorm), no shared expert.
    "qwen3": dict(vocab=151936, H=2048, layers=48, first_dense=0, dense_I=0, E=128, k=8, I=768,
                  shared_I=0, scoring="softmax", renorm=True, routed_scale=1.0, n_group=1,
                  topk_group=1, e_bias=False, attn="gqa", heads=32, kv_heads=4, head_dim=128,
                  rope_theta=1e6, fp8=False),
    # DeepSeek-V3 MoE stack (no attention): 8 layers, 256 experts top-8,
    # sigmoid + bias group-limited (8 groups, top-4), scale 2.5, 1 shared
    # expert, fp8 e4m3fn weights with 128x128 block scales.
    "v3": dict(vocab=0, H=7168, layers=8, first_dense=0, dense_I=0, E=256, k=8, I=2048,
               shared_I=2048, scoring="sigmoid", renorm=True, routed_scale=2.5, n_group=8,
               topk_group=4, e_bias=True, attn=None, fp8=True),
}


_EPS = 1e-6


def _k():
    from sluice_amd import _lib

    return _lib.load(), _lib.check


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def add_rmsnorm(x, delta, w, out=None, eps=_EPS):
    """x += delta (bf16, in place; skipped when delta is None), then
    out = rmsnorm(x) * w.  One kernel."""
    lib, check = _k()
    if out is None:
        out = torch.empty_like(x)
    check(lib.sluice_dec_add_rmsnorm(x.data_ptr(), None if delta is None else delta.data_ptr(),
                                     w.data_ptr(), out.data_ptr(), x.shape[0], x.shape[1],
                                     float(eps), _stream(x)), "sluice_dec_add_rmsnorm")
    return out


# One zero-filled workspace per device for the skinny GEMMs' split-K hand-off
# (its size does not depend on the shape; the calls of a step run one after
# another on one stream).
_LIN_WS = ops._Workspace(zero=True)  # split-K counters start (and end) at zero


def _linear_ws(dev):
    lib, _ = _k()
    return _LIN_WS.get(dev, int(lib.sluice_dec_linear_workspace()))


def linear(x, w):
    """y = x . w^T for decode batches (T <= 16): one streaming MFMA kernel."""
    lib, check = _k()
    T, K = x.shape
    N = w.shape[0]
    if T > 16:
        raise ValueError(f"decode linear supports at most 16 rows, got {T}")
    y = torch.empty((T, N), dtype=x.dtype, device=x.device)
    check(lib.sluice_dec_linear(x.data_ptr(), w.data_ptr(), T, N, K, y.data_ptr(),
                                _linear_ws(x.device).data_ptr(), _stream(x)),
          "sluice_dec_linear")
    return y


def linear_split(x, w):
    """x . w^T left as its K parts [ks, T, N] fp32 (T <= 16): their in-order
    sum rounded to bf16 is the projection; the next kernel sums them, so no
    workgroup waits for another's part."""
    lib, check = _k()
    T, K = x.shape
    N = w.shape[0]
    ks = lib.sluice_dec_linear_split_parts(T, N, K)
    if ks < 1:
        raise ValueError(f"linear_split does not take T={T}, N={N}, K={K}")
    parts = torch.empty((ks, T, N), dtype=torch.float32, device=x.device)
    check(lib.sluice_dec_linear_split(x.data_ptr(), w.data_ptr(), T, N, K, parts.data_ptr(),
                                      _stream(x)), "sluice_dec_linear_split")
    return parts


def linear_glu(x, w):
    """silu(x . w[:N/2]^T) * (x . w[N/2:]^T) for decode batches (T <= 16):
    the gate/up projection with the activation in its epilogue."""
    lib, check = _k()
    T, K = x.shape
    N = w.shape[0]
    if T > 16:
        raise ValueError(f"decode linear supports at most 16 rows, got {T}")
    y = torch.empty((T, N // 2), dtype=x.dtype, device=x.device)
    check(lib.sluice_dec_linear_glu(x.data_ptr(), w.data_ptr(), T, N, K, y.data_ptr(),
                                    _linear_ws(x.device).data_ptr(), _stream(x)),
          "sluice_dec_linear_glu")
    return y


def argmax_rows(x, out):
    """out[t] = argmax x[t] (int64, first index on ties) without library
    reductions, which record memsets that replayed graphs do not honour."""
    lib, check = _k()
    check(lib.sluice_dec_argmax(x.data_ptr(), x.shape[0], x.shape[1], out.data_ptr(), _stream(x)),
          "sluice_dec_argmax")
    return out


def silu_mul(gu):
    lib, check = _k()
    rows, two_i = gu.shape
    out = torch.empty((rows, two_i // 2), dtype=gu.dtype, device=gu.device)
    check(lib.sluice_dec_silu_mul(gu.data_ptr(), out.data_ptr(), rows, two_i // 2, _stream(gu)),
          "sluice_dec_silu_mul")
    return out


def _randn(shape, gen, std, dev, dtype=torch.bfloat16):
    return (torch.randn(shape, generator=gen, device=dev) * std).to(dtype)


def _mla_kslot(dev):
    """Slot of row r of a 32-row block in the transposed latent cache (the
    K order of the kernels' P . ckv product)."""
    return torch.tensor([8 * ((r & 15) >> 2) + 4 * (r >> 4) + (r & 3) for r in range(32)],
                        device=dev)


class _MLA(nn.Module):
    """Multi-head latent attention (DeepSeek-V2), decode form with the
    up-projections absorbed: one GEMM for [q ; kv latent + rope key], then
    sluice_dec_mla_decode (q absorption into the latent space and the new
    cache rows; scores, softmax and the weighted latent sum over row splits
    on the matrix cores; merge and value up-projection) and the output
    GEMM.  The latent cache is kept row-major and, for the P . ckv product,
    transposed in 32-row blocks (ckvt)."""

    def __init__(self, sp, batch, max_len, dev, gen):
        super().__init__()
        H, nh, lora = sp["H"], sp["heads"], sp["kv_lora"]
        nope, rope, vh = sp["qk_nope"], sp["qk_rope"], sp["v_head"]
        self.nh, self.lora, self.nope, self.rope, self.vh = nh, lora, nope, rope, vh
        self.nq = nh * (nope + rope)
        self.w_qkva = _randn((self.nq + lora + rope, H), gen, 0.02, dev)
        self.kv_norm = torch.ones(lora, device=dev, dtype=torch.bfloat16)
        self.w_uk = _randn((nh, nope, lora), gen, 0.02, dev)
        self.w_ukt = self.w_uk.transpose(1, 2).contiguous()
        self.w_uv = _randn((nh, lora, vh), gen, 0.02, dev)
        self.wo = _randn((H, nh * vh), gen, 0.02, dev)
        if max_len % 32:
            raise ValueError(f"MLA cache length {max_len} is not a multiple of 32")
        self.ckv = torch.zeros((batch, max_len, lora), device=dev, dtype=torch.bfloat16)
        self.ckvt = torch.zeros((batch, max_len // 32, lora, 32), device=dev, dtype=torch.bfloat16)
        self.kpe = torch.zeros((batch, max_len, rope), device=dev, dtype=torch.bfloat16)
        self.scale = (nope + rope) ** -0.5
        self.L = max_len
        self._work = {}

    def fill_prompt(self, n, gen):
        b, L, lora = self.ckv.shape
        self.ckv[:, :n] = _randn((b, n, lora), gen, 1.0, self.ckv.device)
        self.kpe[:, :n] = _randn((b, n, self.rope), gen, 1.0, self.ckv.device)
        self.ckvt[..., _mla_kslot(self.ckv.device)] = self.ckv.view(b, L // 32, 32, lora).transpose(2, 3)

    # the output projection can hand its K parts to the next (fused) norm
    splits_output = True

    def forward(self, hn, pos, cos_t, sin_t, split=False):
        """Attention output [c, H] bf16, or with split=True the output
        projection's K parts [ks, c, H] fp32."""
        lib, check = _k()
        c = hn.shape[0]
        qkva = linear(hn, self.w_qkva)
        work = self._work.get(c)
        if work is None:  # fixed per batch size, so captured graphs keep it
            work = self._work[c] = torch.empty(
                int(lib.sluice_dec_mla_workspace(c, self.nh)), dtype=torch.uint8,
                device=hn.device)
        row = qkva.shape[1]
        o = torch.empty((c, self.nh * self.vh), dtype=hn.dtype, device=hn.device)
        check(lib.sluice_dec_mla_decode(
            qkva.data_ptr(), row, qkva.data_ptr() + self.nq * 2, row, self.kv_norm.data_ptr(),
            self.w_ukt.data_ptr(), self.w_uv.data_ptr(), cos_t.data_ptr(), sin_t.data_ptr(),
            pos.data_ptr(), c, self.nh, self.nope, self.rope, self.lora, self.vh, self.L, _EPS,
            float(self.scale), self.ckv.data_ptr(), self.ckvt.data_ptr(), self.kpe.data_ptr(),
            work.data_ptr(), o.data_ptr(), _stream(hn)), "sluice_dec_mla_decode")
        return linear_split(o, self.wo) if split else linear(o, self.wo)


class _GQA(nn.Module):
    """Grouped-query attention with per-head q/k RMSNorm (Qwen3): one QKV
    GEMM, one attention kernel (norms, RoPE, cache write, attention) and the
    output GEMM."""

    def __init__(self, sp, batch, max_len, dev, gen):
        super().__init__()
        H, nh, kvh, hd = sp["H"], sp["heads"], sp["kv_heads"], sp["head_dim"]
        self.nh, self.kvh, self.hd = nh, kvh, hd
        self.wqkv = _randn(((nh + 2 * kvh) * hd, H), gen, 0.02, dev)
        self.q_norm = torch.ones(hd, device=dev, dtype=torch.bfloat16)
        self.k_norm = torch.ones(hd, device=dev, dtype=torch.bfloat16)
        self.wo = _randn((H, nh * hd), gen, 0.02, dev)
        self.k = torch.zeros((batch, kvh, max_len, hd), device=dev, dtype=torch.bfloat16)
        self.v = torch.zeros((batch, kvh, max_len, hd), device=dev, dtype=torch.bfloat16)
        self.scale = hd ** -0.5
        self.L = max_len

    def fill_prompt(self, n, gen):
        b = self.v.shape[0]
        self.k[:, :, :n] = _randn((b, self.kvh, n, self.hd), gen, 1.0, self.v.device)
        self.v[:, :, :n] = _randn((b, self.kvh, n, self.hd), gen, 1.0, self.v.device)

    # the output projection can hand its K parts to the next (fused) norm
    splits_output = True

    def forward(self, hn, pos, cos_t, sin_t, split=False):
        """Attention output [c, H] bf16, or with split=True the output
        projection's K parts [ks, c, H] fp32 (their in-order sum, rounded to
        bf16, is the bf16 output)."""
        lib, check = _k()
        c = hn.shape[0]
        # (the QKV projection stays whole: every 16-lane group of the attention
        # kernel reads the head's q, k and v, and reading K parts instead cost
        # the kernel more than splitting saved the projection)
        qkv = linear(hn, self.wqkv)
        o = torch.empty((c, self.nh * self.hd), dtype=hn.dtype, device=hn.device)
        check(lib.sluice_dec_gqa_decode(
            qkv.data_ptr(), None, 0, self.q_norm.data_ptr(),
            self.k_norm.data_ptr(), cos_t.data_ptr(), sin_t.data_ptr(), pos.data_ptr(), c,
            self.nh, self.kvh, self.hd, self.L, _EPS, float(self.scale), self.k.data_ptr(),
            self.v.data_ptr(), o.data_ptr(), _stream(hn)), "sluice_dec_gqa_decode")
        return linear_split(o, self.wo) if split else linear(o, self.wo)


class _DenseMLP(nn.Module):
    """SwiGLU MLP: the gate/up GEMM with the activation in its epilogue, then
    the down GEMM."""

    def __init__(self, H, I, dev, gen):
        super().__init__()
        self.gate_up = _randn((2 * I, H), gen, 0.02, dev)
        self.down = _randn((H, I), gen, 0.02, dev)
        self.I = I

    def forward(self, x):
        return linear(linear_glu(x, self.gate_up), self.down)


class _Fp8SharedMLP(nn.Module):
    """A SwiGLU shared expert in e4m3fn codes with 128x128 fp32 block scales
    (gate rows then up rows in gate_up [2*I, H], down [H, I]), like the
    routed experts of an fp8 layer.  Alone it runs as a one-expert product;
    inside the routed product it rides along as fused_experts' shared
    weights."""

    def __init__(self, H, I, dev, gen):
        super().__init__()
        self.gate_up = (torch.randn((2 * I, H), generator=gen, device=dev) * 0.5).to(
            torch.float8_e4m3fn).view(torch.uint8)
        self.down = (torch.randn((H, I), generator=gen, device=dev) * 0.5).to(
            torch.float8_e4m3fn).view(torch.uint8)
        self.gate_up_scale = torch.rand((2 * I // 128, H // 128), generator=gen,
                                        device=dev) * 0.02 + 0.01
        self.down_scale = torch.rand((H // 128, I // 128), generator=gen, device=dev) * 0.02 + 0.01
        self.I = I

    def forward(self, x):
        T = x.shape[0]
        ids = torch.zeros((T, 1), dtype=torch.int32, device=x.device)
        w = torch.ones((T, 1), dtype=torch.float32, device=x.device)
        return ops.fused_experts(x, self.gate_up[None], self.down[None], w, ids,
                                 global_num_experts=1, w1_scale=self.gate_up_scale[None],
                                 w2_scale=self.down_scale[None], block_shape=[128, 128])


def _expert_store(sp, gen_seed, dev, fp8):
    """One pinned host store of every expert of a layer ([E, ...] per param),
    filled from device-generated random values (N(0, 0.02) for bf16; for fp8,
    e4m3fn codes of N(0, 0.5) with block scales in [0.01, 0.03)), generated
    and copied down in chunks of experts (about 1 GB each)."""
    E, H, I = sp["E"], sp["H"], sp["I"]
    g = torch.Generator(device=dev).manual_seed(gen_seed)
    out = {}
    shapes = {"w13_weight": (E, 2 * I, H), "w2_weight": (E, H, I)}
    for name, shp in shapes.items():
        dt = torch.uint8 if fp8 else torch.bfloat16
        st = ops.HostStore(shp, dt)
        row_bytes = st.nbytes // E
        n = max(1, (1 << 30) // max(row_bytes, 1))
        for e0 in range(0, E, n):
            e1 = min(E, e0 + n)
            v = torch.randn((e1 - e0, *shp[1:]), generator=g, device=dev)
            if fp8:
                v = v.mul_(0.5).to(torch.float8_e4m3fn).view(torch.uint8)
            else:
                v = v.mul_(0.02).to(torch.bfloat16)
            st.tensor[e0:e1].copy_(v)
            del v
        out[name] = st
    if fp8:
        for name, shp in (("w13_weight_scale", (E, 2 * I // 128, H // 128)),
                          ("w2_weight_scale", (E, H // 128, I // 128))):
            st = ops.HostStore(shp, torch.float32)
            st.tensor.copy_(torch.rand(shp, generator=g, device=dev) * 0.02 + 0.01)
            out[name] = st
    return out


def expert_store_bytes(sp) -> int:
    """Host bytes of one layer's expert store."""
    E, H, I = sp["E"], sp["H"], sp["I"]
    if sp["fp8"]:
        return E * (3 * I * H + ((2 * I // 128) * (H // 128) + (H // 128) * (I // 128)) * 4)
    return E * 3 * I * H * 2


def host_memory_available() -> Optional[int]:
    """MemAvailable of this host (bytes), bounded by the cgroup limit if one
    is set; None if unknown."""
    avail = None
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemAvailable:"):
                    avail = int(line.split()[1]) * 1024
    except OSError:
        return None
    for path in ("/sys/fs/cgroup/memory.max", "/sys/fs/cgroup/memory/memory.limit_in_bytes"):
        try:
            with open(path) as f:
                raw = f.read().strip()
            if raw and raw != "max" and int(raw) < (1 << 60):
                used = 0
                for upath in ("/sys/fs/cgroup/memory.current",
                              "/sys/fs/cgroup/memory/memory.usage_in_bytes"):
                    try:
                        with open(upath) as uf:
                            used = int(uf.read().strip())
                        break
                    except OSError:
                        continue
                lim = int(raw) - used
                avail = lim if avail is None else min(avail, lim)
            break
        except (OSError, ValueError):
            continue
    return avail


class _StoreMoELayer(nn.Module):
    """FusedMoE-shaped layer whose per-expert params ARE pinned host stores
    (possibly shared between layers), adopted by the offloader without a copy."""

    def __init__(self, sp, store, seed, dev, routing_bias, name, gate_std=0.02):
        super().__init__()
        E, H = sp["E"], sp["H"]
        g = torch.Generator(device=dev).manual_seed(5000 + seed)
        self.H, self.I, self.E, self.top_k = H, sp["I"], E, sp["k"]
        self.layer_name = name
        self.global_num_experts = E
        self.local_num_experts = E
        self.quant_method = _QuantMethod()
        for pname, st in store.items():
            setattr(self, pname, nn.Parameter(st.tensor, requires_grad=False))
        self.block_shape = [128, 128] if sp["fp8"] else None
        self.gate = nn.Module()
        self.gate.weight = nn.Parameter(_randn((E, H), g, gate_std, dev), requires_grad=False)
        self.e_score_correction_bias = (
            nn.Parameter(torch.randn(E, generator=g, device=dev) * 0.01, requires_grad=False)
            if sp["e_bias"] else None)
        self.shared = None
        if sp["shared_I"]:
            self.shared = (_Fp8SharedMLP(H, sp["shared_I"], dev, g) if sp["fp8"]
                           else _DenseMLP(H, sp["shared_I"], dev, g))
        self.routing_bias = routing_bias
        self.sp = sp
        _router_attrs(self, sp["scoring"], sp["renorm"], sp["routed_scale"], sp["n_group"],
                      sp["topk_group"])

        # vLLM runner surface, so attach_router_split arms this layer
        layer = self

        def gate(hs):
            return layer.logits(hs), None

        def select_experts(hidden_states, router_logits, input_ids=None):
            return layer.select(router_logits)

        self.runner = types.SimpleNamespace(
            gate=gate, router=types.SimpleNamespace(select_experts=select_experts),
            _shared_experts=(types.SimpleNamespace(_layer=self.shared) if self.shared else None),
            moe_config=types.SimpleNamespace(experts_per_token=self.top_k, pcp_size=1),
            _forward_entry=_stock_entry(self, gate, select_experts))

    @property
    def expert_map(self):
        return self._buffers.get("_expert_map")

    def forward(self, hs: torch.Tensor) -> torch.Tensor:
        r = self.runner._forward_entry(hs, None, None, None, self.layer_name, False)
        if isinstance(r, tuple):
            sh, routed = r
            return routed + sh
        return r

    def logits(self, hn):
        """Router logits (fp32) = gate GEMV + this step's synthetic bias, one kernel."""
        lib, check = _k()
        T = hn.shape[0]
        out = torch.empty((T, self.E), dtype=torch.float32, device=hn.device)
        rb = self.routing_bias
        check(lib.sluice_dec_gate_logits(
            hn.data_ptr(), self.gate.weight.data_ptr(),
            None if rb is None else rb.table.data_ptr(), None if rb is None else rb.step.data_ptr(),
            0 if rb is None else rb.table.shape[0], 0 if rb is None else rb.table.shape[1], T,
            self.H, self.E, out.data_ptr(), _stream(hn)), "sluice_dec_gate_logits")
        return out

    def norm_logits(self, x, delta, w):
        """(x_out, hn, logits): the residual add, the RMSNorm before this layer
        and its router logits in one kernel (x_out = x + delta, hn =
        rmsnorm(x_out) * w, as add_rmsnorm computes them), or None when the
        batch shape is one the fused kernel does not take.  delta may be a
        projection's fp32 K parts [ks, T, H] (their in-order sum rounded to
        bf16 is the delta)."""
        lib, check = _k()
        T = x.shape[0]
        if not lib.sluice_dec_add_rmsnorm_gate_ok(T, self.H):
            return None
        parts = delta is not None and delta.dtype == torch.float32
        x_out, hn = torch.empty_like(x), torch.empty_like(x)
        out = torch.empty((T, self.E), dtype=torch.float32, device=x.device)
        rb = self.routing_bias
        check(lib.sluice_dec_add_rmsnorm_gate(
            x.data_ptr(), None if delta is None or parts else delta.data_ptr(),
            delta.data_ptr() if parts else None, delta.shape[0] if parts else 0, w.data_ptr(),
            x_out.data_ptr(), hn.data_ptr(), self.gate.weight.data_ptr(),
            None if rb is None else rb.table.data_ptr(), None if rb is None else rb.step.data_ptr(),
            0 if rb is None else rb.table.shape[0], 0 if rb is None else rb.table.shape[1], T,
            self.H, self.E, _EPS, out.data_ptr(), _stream(x)), "sluice_dec_add_rmsnorm_gate")
        return x_out, hn, out

    def select(self, lg):
        sp = self.sp
        return ops.select_experts(lg, sp["k"], scoring=sp["scoring"], renormalize=sp["renorm"],
                                  routed_scaling_factor=sp["routed_scale"],
                                  e_score_correction_bias=self.e_score_correction_bias,
                                  num_expert_group=sp["n_group"], topk_group=sp["topk_group"])

    def select_out(self, lg, ids_out):
        """select() writing the ids into ids_out (for timing the router alone)."""
        sp = self.sp
        return ops.select_experts(lg, sp["k"], scoring=sp["scoring"], renormalize=sp["renorm"],
                                  routed_scaling_factor=sp["routed_scale"],
                                  e_score_correction_bias=self.e_score_correction_bias,
                                  num_expert_group=sp["n_group"], topk_group=sp["topk_group"],
                                  ids_out=ids_out)

    def shared_foldable(self) -> bool:
        """The shared experts can run inside the routed product: their
        intermediate is a multiple (<= 4) of the routed experts'."""
        sh = self.shared
        return sh is not None and sh.I % self.I == 0 and sh.I // self.I <= 4

    def experts(self, hn, tw, ti, shared_output=None, fold_shared=False, plan=None):
        """Routed experts (+ shared_output), or with fold_shared the routed
        and the shared experts in one grouped product.  plan: the product's
        plan the layer's gap built for ti (None: the product plans itself)."""
        kw = {} if plan is None else {"plan": plan}
        if self.sp["fp8"]:
            kw.update(w1_scale=self.w13_weight_scale, w2_scale=self.w2_weight_scale,
                      block_shape=[128, 128])
        if fold_shared:
            sh = self.shared
            kw.update(shared_w1=sh.gate_up, shared_w2=sh.down)
            if self.sp["fp8"]:
                kw.update(shared_w1_scale=sh.gate_up_scale, shared_w2_scale=sh.down_scale)
        return ops.fused_experts(hn, self.w13_weight, self.w2_weight, tw, ti,
                                 global_num_experts=self.E, expert_map=self._expert_map,
                                 shared_output=shared_output, **kw)


class SyntheticDecoder:
    """Random-init decoder of a SPECS shape, decoded with hipGraphs.

    Piece p holds everything between MoE layer p-1's gap and MoE layer p's
    gap: MoE layer p-1's expert product + shared experts + residual, every
    dense/attention block up to MoE layer p, and MoE layer p's norm, gate and
    top-k routing.  The last piece ends with the final norm, the LM head and
    the greedy next-token write.  With the gap server (default) the gap op
    is a device launch and the whole step -- pieces and gaps -- is captured
    as one graph; with ``gap_server=False`` each piece is a graph and the
    reference's eager gap runs between them.
    Prompts are synthetic: until ``prefill`` runs, the first ``prompt_len``
    KV positions hold random latents/keys/values; ``prefill(c)`` decodes a
    seeded random prompt through the model position by position instead
    (every prompt token routed through every MoE layer).  Decoding starts at
    position ``prompt_len``; the caches hold prompt_len + gen_len positions.

    ``expert_checkpoint`` (a safetensors file or directory, Hugging Face
    expert naming) loads every MoE layer's routed experts from a checkpoint
    instead of random values; the other weights stay random.

    Routing: router logits = gate GEMM (weights N(0, gate_std)) + log-Zipf
    (zipf_s) popularity over a seeded permutation + sigma * z_t, z_t a
    unit-variance AR(1) process (rho) per sequence and layer.  The defaults
    (zipf_s 1.1, rho 0.7, sigma 1.2, gate_std 0.004: a gate term of standard
    deviation ~0.18 at hidden 2048) give selections whose top-k experts take
    the share Zipf(1.1) popularity gives them (55-57% at 64 experts top-6
    and 128 top-8) and logits whose step-to-step correlation is ~0.68;
    ``RoutingBias.refill`` changes the knobs in place.
    ``uniform_routing`` replaces the bias with large i.i.d. noise (uniform
    top-k, the miss-dominated stress case).

    Host stores: ``host_pool`` "shared" (one store of the layer shape, every
    MoE layer streams from it), "per-layer", or "auto" (per-layer when they
    fit in half of the host memory available, else shared); ``stores``
    adopts the per-layer stores of another decoder of the same shape."""

    def __init__(self, spec: str, max_batch: int, slots: int, prompt_len: int = 128,
                 gen_len: int = 256, seed: int = 0, device=None, host_pool: str = "shared",
                 zipf_s: float = 1.1, rho: float = 0.7, sigma: float = 1.2,
                 gate_std: float = 0.004, uniform_routing: bool = False, fast_hit: bool = True,
                 layers: int = None, gap_server: bool = True, expert_checkpoint=None,
                 stores=None, progress=None):
        self.sp = sp = dict(SPECS[spec])
        if layers is not None:
            sp["layers"] = layers
        self.name = spec
        dev = self.dev = device or torch.device("cuda", torch.cuda.current_device())
        # (a multiple of 32: the MLA latent cache is also kept in 32-row blocks)
        self.max_batch, self.max_len = max_batch, (prompt_len + gen_len + 8 + 31) // 32 * 32
        self.prompt_len = prompt_len
        self.gen_len = gen_len
        g = torch.Generator(device=dev).manual_seed(seed)
        H = sp["H"]
        steps_tbl = prompt_len + gen_len + 64
        n_moe = sp["layers"] - sp["first_dense"]
        self.host_store_bytes = expert_store_bytes(sp)
        if stores is not None:
            host_pool = "adopted"
        elif host_pool == "auto":
            avail = host_memory_available()
            fits = avail is not None and n_moe * self.host_store_bytes <= avail // 2
            host_pool = "per-layer" if fits else "shared"
        if host_pool not in ("shared", "per-layer", "adopted"):
            raise ValueError(f"host_pool {host_pool!r}")
        self.host_pool = host_pool
        self.host_pool_note = None
        self.stores = []
        self.routing_knobs = ({"uniform": True} if uniform_routing else
                              {"zipf_s": zipf_s, "rho": rho, "sigma": sigma})
        self.routing_knobs["gate_std"] = gate_std
        self.has_attn = sp["attn"] is not None
        self.embed = _randn((sp["vocab"], H), g, 0.02, dev) if self.has_attn else None
        self.lm_head = _randn((sp["vocab"], H), g, 0.02, dev) if self.has_attn else None
        self.final_norm = torch.ones(H, device=dev, dtype=torch.bfloat16)
        self.blocks = []
        self.moe_layers = []
        self.bias_tables = []
        self.step = torch.zeros((), dtype=torch.long, device=dev)  # routing-bias row, all layers
        store = None
        for li in range(sp["layers"]):
            blk = types.SimpleNamespace(attn=None, mlp=None, moe=None,
                                        n1=torch.ones(H, device=dev, dtype=torch.bfloat16),
                                        n2=torch.ones(H, device=dev, dtype=torch.bfloat16))
            if sp["attn"] == "mla":
                blk.attn = _MLA(sp, max_batch, self.max_len, dev, g)
            elif sp["attn"] == "gqa":
                blk.attn = _GQA(sp, max_batch, self.max_len, dev, g)
            if blk.attn is not None:
                blk.attn.fill_prompt(prompt_len, g)
            if li < sp["first_dense"]:
                blk.mlp = _DenseMLP(H, sp["dense_I"], dev, g)
            else:
                if expert_checkpoint is not None:
                    # the layer's real expert rows (Hugging Face safetensors
                    # naming), straight into pinned stores in the slot layout
                    from sluice_amd import loader

                    store = loader.expert_stores_from_checkpoint(expert_checkpoint, li)
                    shp = tuple(store["w13_weight"].tensor.shape)
                    if shp != (sp["E"], 2 * sp["I"], sp["H"]):
                        raise ValueError(f"checkpoint layer {li}: experts {shp} do not match the "
                                         f"{spec} shape")
                elif stores is not None:
                    store = stores[len(self.moe_layers)]
                elif store is None or host_pool == "per-layer":
                    try:
                        store = _expert_store(sp, 7000 + li, dev, sp["fp8"])
                    except RuntimeError as e:
                        if store is None or host_pool != "per-layer":
                            raise
                        # pinned memory ran out: the remaining layers share
                        # the last store made
                        self.host_pool = host_pool = "per-layer, then shared"
                        self.host_pool_note = (f"pinned allocation failed at MoE layer "
                                               f"{len(self.moe_layers)}: {e}")
                        if progress is not None:
                            progress(self.host_pool_note)
                    if progress is not None:
                        progress(f"host store of layer {li} ready")
                self.stores.append(store)
                rb = None
                if uniform_routing:
                    rb = RoutingBias(sp["E"], max_batch, steps_tbl, 0.0, 0.0, 0.0, 8000 + li, dev,
                                     step=self.step)
                    # sigmoid scores saturate to 1.0 in fp32 past |x| ~ 17, which
                    # would tie many experts (the lowest ids win): smaller noise
                    rb.fill_uniform(g, scale=3.0 if sp["scoring"] == "sigmoid" else 10.0)
                else:
                    rb = RoutingBias(sp["E"], max_batch, steps_tbl, zipf_s, rho, sigma, 8000 + li,
                                     dev, step=self.step)
                self.bias_tables.append(rb)
                blk.moe = _StoreMoELayer(sp, store, li, dev, rb, f"layers.{li}.mlp",
                                         gate_std=gate_std)
                self.moe_layers.append(blk.moe)
            self.blocks.append(blk)
        self.off = build_offloaded([m for m in self.moe_layers], slots, dev, fast_hit=fast_hit)
        if gap_server:
            self.off.start_gap_server()
        self.caches = [self.off._caches[id(m)] for m in self.moe_layers]
        # batches above the router-split envelope take the classic path
        self.thr = self.off._rs_thr or max(1, min(16, slots // sp["k"]))
        assert [id(c) for c in self.off._rs_caches] == [id(c) for c in self.caches]
        for m in self.moe_layers:
            ops.reserve_workspace(dev, max_batch, H, sp["I"], sp["k"], sp["shared_I"])
        _linear_ws(dev)  # before any capture: graphs bake its address
        rope_d = (sp["qk_rope"] if sp["attn"] == "mla" else sp.get("head_dim", 128))
        inv = 1.0 / (sp.get("rope_theta", 1e4) ** (torch.arange(0, rope_d, 2, device=dev).float()
                                                     / rope_d))
        ang = torch.arange(self.max_len, device=dev).float()[:, None] * inv[None, :]
        self.cos_tbl, self.sin_tbl = ang.cos(), ang.sin()
        # per-batch-size static state
        self.state = {}
        self.graphs = {}
        self.layer_io = {}
        self.pool = None

    # -- state -----------------------------------------------------------------
    def _state(self, c):
        st = self.state.get(c)
        if st is None:
            dev = self.dev
            g = torch.Generator(device=dev).manual_seed(99 + c)
            st = types.SimpleNamespace()
            st.c = c
            st.pos = torch.full((c,), self.prompt_len, dtype=torch.long, device=dev)
            st.bidx = torch.arange(c, device=dev)
            st.tokens = (torch.randint(0, max(self.sp["vocab"], 1), (c,), generator=g, device=dev)
                         if self.has_attn else None)
            st.prompt = (torch.randint(0, max(self.sp["vocab"], 1), (c, self.prompt_len),
                                       generator=g, device=dev) if self.has_attn else None)
            st.x = _randn((c, self.sp["H"]), g, 1.0, dev)  # MoE-stack input
            st.out_tokens = []
            self.state[c] = st
        return st

    def reset(self, c):
        st = self._state(c)
        st.pos.fill_(self.prompt_len)
        self.step.zero_()

    def prefill(self, c, graphs: bool = True) -> None:
        """Process batch c's synthetic prompts, untimed: position by position
        through the decode step (the captured one when ``graphs``), each
        step's input token the prompt's next one, so every prompt token is
        routed through every MoE layer -- the slot caches warm up on the
        prompts' routing -- and the KV caches hold the prompts' keys and
        values.  Ends at position prompt_len with the first generated token
        as the next input.  (A MoE stack without attention steps its hidden
        state prompt_len times.)"""
        st = self._state(c)
        st.pos.zero_()
        self.step.zero_()
        for p in range(self.prompt_len):
            if st.prompt is not None:
                st.tokens.copy_(st.prompt[:, p])
            if graphs:
                self.step_graphs(c)
            else:
                self.step_eager(c)

    # -- pieces ----------------------------------------------------------------
    def _block_front(self, i, io, st):
        """Block i up to its MLP input: the residual add of the pending
        delta fused into the attention norm, attention, then the MLP norm
        (which adds the attention output).  Leaves io["hn"] = MLP input."""
        blk = self.blocks[i]
        x = io["x"]
        lib, _ = _k()
        fuse = blk.moe is not None and lib.sluice_dec_add_rmsnorm_gate_ok(x.shape[0], x.shape[1])
        if blk.attn is not None:
            hn = add_rmsnorm(x, io["delta"], blk.n1)
            if fuse and getattr(blk.attn, "splits_output", False):
                # the output projection's K parts go straight into the fused norm
                io["delta"] = blk.attn(hn, st.pos, self.cos_tbl, self.sin_tbl, split=True)
            else:
                io["delta"] = blk.attn(hn, st.pos, self.cos_tbl, self.sin_tbl)
        fused = blk.moe.norm_logits(x, io["delta"], blk.n2) if fuse else None
        if fused is not None:
            # a MoE layer's norm and router logits in one kernel
            io["x"], io["hn"], io["lg"] = fused
        else:
            io["hn"] = add_rmsnorm(x, io["delta"], blk.n2)
        io["delta"] = None

    def _to_next_gap(self, i, io, st):
        """From block i on: run dense blocks; at the next MoE block compute
        its norm, router logits and top-k, and return its index (None if
        the model ends first, after the final norm, LM head and next token)."""
        while i < len(self.blocks):
            blk = self.blocks[i]
            self._block_front(i, io, st)
            if blk.moe is None:
                io["delta"] = blk.mlp(io["hn"])
                i += 1
                continue
            lg = io.pop("lg", None)
            tw, ti = blk.moe.select(lg if lg is not None else blk.moe.logits(io["hn"]))
            io.update(tw=tw, ti=ti, i=i)
            return i
        hf = add_rmsnorm(io["x"], io["delta"], self.final_norm)
        if self.has_attn:
            argmax_rows(linear(hf, self.lm_head), st.tokens)
            st.pos.add_(1)
        else:
            st.x.copy_(hf)
        self.step.add_(1)
        return None

    def classic(self, c) -> bool:
        """Batch size c runs the classic (wave) path: more tokens than the
        router-split envelope (slots // top_k)."""
        return c > self.thr

    def pieces(self, c):
        """List of (piece_fn, gap_layer_index or None); piece_fn(io) mutates
        io.  Piece 0 embeds and runs up to the first MoE routing; piece p runs
        MoE layer p-1's experts (shared expert folded into the combine) and
        on to MoE layer p's routing; the last piece ends the step.  On the
        classic path MoE layer p-1's routed output is computed between the
        pieces (io["routed"]) and piece p adds the shared expert to it."""
        st = self._state(c)
        classic = self.classic(c)
        moe_pos = [i for i, b in enumerate(self.blocks) if b.moe is not None]

        def first(io):
            x = self.embed.index_select(0, st.tokens) if self.has_attn else st.x.clone()
            io.update(x=x, delta=None)
            self._to_next_gap(0, io, st)

        out = [(first, 0)]
        for n, i in enumerate(moe_pos):
            last = n == len(moe_pos) - 1

            def mid(io, i=i, n=n):
                moe = self.blocks[i].moe
                # the plan this layer's gap op built for its ids
                plan = None if classic else self.off.gap_plan(n, io["ti"].numel())
                if not classic and moe.shared_foldable():
                    # routed and shared experts in one grouped product
                    io["delta"] = moe.experts(io["hn"], io["tw"], io["ti"], fold_shared=True,
                                              plan=plan)
                else:
                    sh = moe.shared(io["hn"]) if moe.shared is not None else None
                    if classic:
                        io["delta"] = io["routed"] if sh is None else io["routed"] + sh
                    else:
                        io["delta"] = moe.experts(io["hn"], io["tw"], io["ti"], shared_output=sh,
                                                  plan=plan)
                self._to_next_gap(i + 1, io, st)

            out.append((mid, n + 1 if not last else None))
        return out

    # -- execution ---------------------------------------------------------------
    def gap(self, n, ti):
        self.off._router_split_gap(n, ti)

    def classic_moe(self, n, io, out=None):
        """MoE layer n's routed output on the classic path: the layer's
        ``quant_method.apply``, which the offloader's hook runs once per wave
        (eager: it syncs the host for the ids).  Written into ``out`` when
        given (the static buffer captured pieces read)."""
        moe = self.moe_layers[n]
        routed = moe.quant_method.apply(layer=moe, x=io["hn"], topk_weights=io["tw"],
                                        topk_ids=io["ti"])
        if out is None:
            io["routed"] = routed
        else:
            out.copy_(routed)

    def _step_fn(self, c):
        """The whole step: every piece, with the ``vllm::sluice_stream_gap``
        op between a MoE layer's routing and its expert product (the op's
        output feeds the experts, as in the router-split entry) -- or, above
        the envelope, the classic hook.  Records each MoE layer's
        routing/activation tensors in ``self.layer_io[c]``."""
        ps = self.pieces(c)
        rec = []
        classic = self.classic(c)

        def run(io):
            rec.clear()
            if classic:
                self.off.set_step_signal(c, c, True)  # every row a one-token decode
            for fn, gap_idx in ps:
                fn(io)
                if gap_idx is None:
                    continue
                if classic:
                    self.classic_moe(gap_idx, io)
                else:
                    io["hn"] = torch.ops.vllm.sluice_stream_gap(io["hn"], io["ti"], gap_idx)
                rec.append({"hn": io["hn"], "ti": io["ti"], "tw": io["tw"]})
            self.layer_io[c] = list(rec)

        return run

    def step_eager(self, c):
        """One eager step through the registered ops."""
        from sluice_amd.offloader import activate

        activate(self.off)
        io = {}
        self._step_fn(c)(io)
        return io

    def capture(self, c, warmup: int = 2):
        """Capture batch size c after eager warm-up steps.  With the gap
        server the whole step (gap launches included) is ONE graph; with
        inline gaps every piece between two gaps is a graph and the gaps run
        eagerly in between."""
        from sluice_amd.offloader import activate

        activate(self.off)
        st = self._state(c)
        for _ in range(warmup):
            self.step_eager(c)
        self.sync()
        if self.pool is None:
            self.pool = torch.cuda.graph_pool_handle()
        s = torch.cuda.Stream(device=self.dev)
        s.wait_stream(torch.cuda.current_stream())
        graphs = []
        classic = self.classic(c)
        if classic:
            self.routed_buf = getattr(self, "routed_buf", {})
            self.routed_buf[c] = torch.zeros((c, self.sp["H"]), dtype=torch.bfloat16,
                                             device=self.dev)
        if self.off._server is not None and not classic:
            io = {}
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=self.pool, stream=s):
                self._step_fn(c)(io)
            graphs.append((g, None, io))
        else:
            ps = self.pieces(c)
            io = {"routed": self.routed_buf[c]} if classic else {}
            rec = []
            for fn, gap_idx in ps:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, pool=self.pool, stream=s):
                    fn(io)
                graphs.append((g, gap_idx, dict(io)))
                if gap_idx is not None:
                    rec.append({"hn": io["hn"], "ti": io["ti"], "tw": io["tw"]})
            self.layer_io[c] = rec
        torch.cuda.current_stream().wait_stream(s)
        self.sync()
        self.graphs[c] = graphs
        self.reset(c)
        del st
        return graphs

    def step_graphs(self, c):
        if self.classic(c):
            self.off.set_step_signal(c, c, True)
            out = self.routed_buf[c]
            for g, gap_idx, io in self.graphs[c]:
                g.replay()
                if gap_idx is not None:
                    self.classic_moe(gap_idx, io, out=out)
            return
        for g, gap_idx, io in self.graphs[c]:
            g.replay()
            if gap_idx is not None:
                self.gap(gap_idx, io["ti"])

    def sync(self):
        """Device synchronise + every gap record served (raises gap errors)."""
        self.off.drain()

    def set_gap_mode(self, server: bool, pipelined: bool) -> None:
        """How the gaps of later steps run.  server: served by the native
        thread, the whole step one captured graph; else inline, the host
        waiting for each MoE layer's ids between captured pieces (the
        reference's eager gap op, src/sluice/offloader.py:2311-2331, 2406).
        pipelined: a missing gap is answered before its rows land and the
        expert product waits per filled slot; else only after every row
        landed (the reference's copy-then-compute order, 2464).  Drops the
        captured graphs: the next run of a batch size recaptures."""
        from sluice_amd import _lib

        self.sync()
        self.graphs = {}
        self.pool = None  # the dropped graphs' pool is released with them
        if server:
            self.off.start_gap_server()
        else:
            self.off.stop_gap_server()
        _lib.check(_lib.load().sluice_gap_set_pipelined(int(pipelined)),
                   "sluice_gap_set_pipelined")

    def gap_counters(self):
        return self.off.gap_counters()

    def close(self):
        self.off.close()
