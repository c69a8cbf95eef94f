"""Device ops of the decode hot path, over the C ABI of libsluice_hip.so.

  select_experts   top-k routing (replaces vLLM's runner.router.select_experts,
                   called at src/sluice/offloader.py:2583-2585)
  fused_experts    grouped SwiGLU product over slot buffers + weighted
                   combine (replaces torch.ops.vllm.fused_experts as called at
                   src/sluice/offloader.py:2590-2599)
  HostStore        exact-size pinned host memory for the expert store

Every call enqueues on torch's current stream and never synchronises.  The
ops are registered with torch.library as ``sluice::fused_experts`` (and as
``vllm::fused_experts`` when vLLM is not installed, so code written against
the vLLM op name runs unchanged); their fake implementations make them
traceable.
"""


import ctypes
import weakref
from typing import Optional

import numpy as np
import torch

from sluice_amd import _lib

_SCORING = {"softmax": 0, "sigmoid": 1}
_MAX_PAIRS = 4096  # SLUICE_MAX_PAIRS: (token, expert) pairs per fused_experts launch


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------------------
# Routing
# ---------------------------------------------------------------------------
def select_experts(router_logits: torch.Tensor, top_k: int, *, scoring: str = "softmax",
                   renormalize: bool = False, routed_scaling_factor: float = 1.0,
                   e_score_correction_bias: Optional[torch.Tensor] = None, num_expert_group: int = 1,
                   topk_group: int = 1, ids_out: Optional[torch.Tensor] = None,
                   weights_out: Optional[torch.Tensor] = None):
    """router_logits [T,E] fp32/bf16 on the GPU -> (topk_weights [T,k] fp32,
    topk_ids [T,k] int32)."""
    lib = _lib.load()
    if router_logits.dim() != 2:
        raise ValueError("router_logits must be [T, E]")
    if router_logits.dtype not in (torch.float32, torch.bfloat16):
        router_logits = router_logits.float()
    logits = router_logits.contiguous()
    T, E = logits.shape
    dev = logits.device
    ids = ids_out if ids_out is not None else torch.empty((T, top_k), dtype=torch.int32, device=dev)
    w = weights_out if weights_out is not None else torch.empty((T, top_k), dtype=torch.float32,
                                                                device=dev)
    bias = e_score_correction_bias
    if bias is not None:
        bias = bias.to(device=dev, dtype=torch.float32).contiguous()
    rc = lib.sluice_route_topk(
        logits.data_ptr(), 1 if logits.dtype == torch.bfloat16 else 0, T, E, top_k,
        _SCORING[scoring], int(bool(renormalize)), float(routed_scaling_factor), _ptr(bias),
        int(num_expert_group), int(topk_group), ids.data_ptr(), w.data_ptr(), _stream(dev))
    _lib.check(rc, "sluice_route_topk")
    return w, ids


@torch.library.custom_op("sluice::select_experts", mutates_args=())
def select_experts_op(router_logits: torch.Tensor, top_k: int, scoring: str = "softmax",
                      renormalize: bool = False, routed_scaling_factor: float = 1.0,
                      e_score_correction_bias: Optional[torch.Tensor] = None,
                      num_expert_group: int = 1,
                      topk_group: int = 1) -> tuple[torch.Tensor, torch.Tensor]:
    """select_experts as a registered op, so a traced entry (torch.compile,
    graph capture) calls the routing kernel as one node."""
    return select_experts(router_logits, top_k, scoring=scoring, renormalize=renormalize,
                          routed_scaling_factor=routed_scaling_factor,
                          e_score_correction_bias=e_score_correction_bias,
                          num_expert_group=num_expert_group, topk_group=topk_group)


@select_experts_op.register_fake
def _(router_logits, top_k, scoring="softmax", renormalize=False, routed_scaling_factor=1.0,
      e_score_correction_bias=None, num_expert_group=1, topk_group=1):
    T = router_logits.shape[0]
    return (router_logits.new_empty((T, top_k), dtype=torch.float32),
            router_logits.new_empty((T, top_k), dtype=torch.int32))


# ---------------------------------------------------------------------------
# Expert product
# ---------------------------------------------------------------------------
class _Workspace:
    """One grow-only device workspace per device, shared by every layer (the
    layers run one after another on one stream).  reserve() sizes it ahead of
    graph capture so captured launches bake a pointer that never moves.
    ``zero``: the buffer is zero-filled when (re)allocated, for kernels that
    keep counters in it; the expert product's workspace needs no initial
    contents."""

    def __init__(self, zero: bool = False):
        self.buf: dict[int, torch.Tensor] = {}
        self.zero = zero

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        cur = self.buf.get(idx)
        if cur is None or cur.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "sluice fused_experts workspace too small during graph capture; call "
                    "sluice_amd.ops.reserve_workspace(...) before capturing")
            alloc = torch.zeros if self.zero else torch.empty
            cur = alloc(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            self.buf[idx] = cur
        return cur


_WS = _Workspace()


def workspace_bytes(T: int, H: int, I: int, k: int, shared_I: int = 0) -> int:
    return int(_lib.load().sluice_fused_experts_workspace(T, H, I, k, shared_I))


def reserve_workspace(device, max_tokens: int, H: int, I: int, k: int,
                      shared_I: int = 0) -> None:
    _WS.get(torch.device(device), workspace_bytes(max_tokens, H, I, k, shared_I))


def _fused_experts_impl(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                        topk_weights: torch.Tensor, topk_ids: torch.Tensor, activation: str,
                        global_num_experts: int, expert_map: Optional[torch.Tensor],
                        w1_scale: Optional[torch.Tensor], w2_scale: Optional[torch.Tensor],
                        block_shape: Optional[list[int]], routed_scaling_factor: float,
                        shared_output: Optional[torch.Tensor],
                        shared_w1: Optional[torch.Tensor] = None,
                        shared_w2: Optional[torch.Tensor] = None,
                        shared_w1_scale: Optional[torch.Tensor] = None,
                        shared_w2_scale: Optional[torch.Tensor] = None,
                        plan: Optional[torch.Tensor] = None) -> torch.Tensor:
    """shared_w1 [2*Is, H] / shared_w2 [H, Is] (Is a multiple of I): the
    layer's shared experts, computed inside the grouped product and added
    unscaled (fp8 with their own block scales when the experts are fp8).
    plan: int32 device buffer holding the plan of these ids over this map,
    built on the stream before the call by the layer's gap; the product then
    launches no align kernel of its own."""
    if activation != "silu":
        raise NotImplementedError(f"activation {activation!r}: only 'silu' is on the path")
    lib = _lib.load()
    x = hidden_states
    if x.dtype != torch.bfloat16:
        raise TypeError("hidden_states must be bf16")
    x = x.contiguous()
    T, H = x.shape
    S = w1.shape[0]
    I = w2.shape[2]
    if w1.shape[1] != 2 * I or w1.shape[2] != H or w2.shape[1] != H:
        raise ValueError(f"bad expert shapes w13 {tuple(w1.shape)} w2 {tuple(w2.shape)}")
    k = topk_ids.shape[1]
    ids = topk_ids if topk_ids.dtype == torch.int32 else topk_ids.to(torch.int32)
    ids = ids.contiguous()
    tw = topk_weights if topk_weights.dtype == torch.float32 else topk_weights.float()
    tw = tw.contiguous()
    if expert_map is not None:
        E = expert_map.shape[0]
        emap = expert_map if expert_map.dtype == torch.int32 else expert_map.to(torch.int32)
        emap_ptr = emap.data_ptr()
    else:
        E = global_num_experts if global_num_experts > 0 else S
        emap_ptr = None
    Is = 0
    if shared_w1 is not None or shared_w2 is not None:
        if shared_w1 is None or shared_w2 is None:
            raise ValueError("shared experts need shared_w1 and shared_w2")
        Is = shared_w2.shape[1]
        if (shared_w1.shape != (2 * Is, H) or shared_w2.shape != (H, Is) or Is % I != 0
                or shared_w1.dtype != w1.dtype or shared_w2.dtype != w2.dtype):
            raise ValueError(f"bad shared expert shapes w13 {tuple(shared_w1.shape)} "
                             f"w2 {tuple(shared_w2.shape)} for I={I}, H={H}")
        shared_w1, shared_w2 = shared_w1.contiguous(), shared_w2.contiguous()
    out = torch.empty_like(x)
    if T == 0:
        return out
    chunk = _MAX_PAIRS // (k + Is // I)
    if plan is not None:
        if (plan.dtype != torch.int32 or plan.device != x.device or not plan.is_contiguous()
                or plan.numel() < lib.sluice_moe_plan_ints(T, k) or T > chunk):
            raise ValueError(f"plan must be a contiguous int32 buffer of >= "
                             f"{lib.sluice_moe_plan_ints(T, k)} ints on {x.device} "
                             f"(T={T}, k={k}, at most {chunk} tokens)")
    if T > chunk:
        # more (token, expert) pairs than one launch takes (a prefill chunk on
        # the classic path): tokens are independent, so run slices of them
        for t0 in range(0, T, chunk):
            t1 = min(T, t0 + chunk)
            out[t0:t1] = _fused_experts_impl(
                x[t0:t1], w1, w2, tw[t0:t1], ids[t0:t1], activation, global_num_experts,
                expert_map, w1_scale, w2_scale, block_shape, routed_scaling_factor,
                None if shared_output is None else shared_output[t0:t1], shared_w1, shared_w2,
                shared_w1_scale, shared_w2_scale)
        return out
    nbytes = workspace_bytes(T, H, I, k, Is)
    ws = _WS.get(x.device, nbytes)
    sh = None
    if shared_output is not None:
        sh = shared_output.contiguous()
        if sh.dtype != torch.bfloat16 or sh.shape != x.shape:
            raise ValueError("shared_output must be bf16 [T, H]")
    stream = _stream(x.device)
    if w1.dtype == torch.bfloat16:
        rc = lib.sluice_fused_experts_bf16(
            x.data_ptr(), w1.data_ptr(), w2.data_ptr(), tw.data_ptr(), ids.data_ptr(), emap_ptr,
            T, H, I, k, E, S, float(routed_scaling_factor), _ptr(shared_w1), _ptr(shared_w2), Is,
            _ptr(sh), ws.data_ptr(), ws.numel(), out.data_ptr(), _ptr(plan), stream)
        _lib.check(rc, "sluice_fused_experts_bf16")
    elif w1.dtype in (torch.uint8, torch.float8_e4m3fn):
        if w1_scale is None or w2_scale is None:
            raise ValueError("fp8 experts need w1_scale and w2_scale")
        bn, bk = (block_shape or [128, 128])[:2]
        if Is and (shared_w1_scale is None or shared_w2_scale is None):
            raise ValueError("fp8 shared experts need shared_w1_scale and shared_w2_scale")
        rc = lib.sluice_fused_experts_fp8(
            x.data_ptr(), w1.data_ptr(), w1_scale.data_ptr(), w2.data_ptr(), w2_scale.data_ptr(),
            int(bn), int(bk), tw.data_ptr(), ids.data_ptr(), emap_ptr, T, H, I, k, E, S,
            float(routed_scaling_factor), _ptr(shared_w1), _ptr(shared_w1_scale),
            _ptr(shared_w2), _ptr(shared_w2_scale), Is, _ptr(sh), ws.data_ptr(), ws.numel(),
            out.data_ptr(), _ptr(plan), stream)
        _lib.check(rc, "sluice_fused_experts_fp8")
    else:
        raise TypeError(f"unsupported expert dtype {w1.dtype}")
    return out


@torch.library.custom_op("sluice::fused_experts", mutates_args=())
def fused_experts_op(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                     topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                     activation: str = "silu", global_num_experts: int = -1,
                     expert_map: Optional[torch.Tensor] = None,
                     w1_scale: Optional[torch.Tensor] = None,
                     w2_scale: Optional[torch.Tensor] = None,
                     block_shape: Optional[list[int]] = None,
                     routed_scaling_factor: float = 1.0,
                     shared_output: Optional[torch.Tensor] = None,
                     shared_w1: Optional[torch.Tensor] = None,
                     shared_w2: Optional[torch.Tensor] = None,
                     shared_w1_scale: Optional[torch.Tensor] = None,
                     shared_w2_scale: Optional[torch.Tensor] = None,
                     plan: Optional[torch.Tensor] = None) -> torch.Tensor:
    return _fused_experts_impl(hidden_states, w1, w2, topk_weights, topk_ids, activation,
                               global_num_experts, expert_map, w1_scale, w2_scale, block_shape,
                               routed_scaling_factor, shared_output, shared_w1, shared_w2,
                               shared_w1_scale, shared_w2_scale, plan)


@fused_experts_op.register_fake
def _(hidden_states, w1, w2, topk_weights, topk_ids, activation="silu", global_num_experts=-1,
      expert_map=None, w1_scale=None, w2_scale=None, block_shape=None,
      routed_scaling_factor=1.0, shared_output=None, shared_w1=None, shared_w2=None,
      shared_w1_scale=None, shared_w2_scale=None, plan=None):
    return torch.empty_like(hidden_states)


def fused_experts(hidden_states, w1, w2, topk_weights, topk_ids, activation="silu",
                  global_num_experts=-1, expert_map=None, **kw):
    """Keyword surface of vLLM's fused_experts as the router-split entry uses it."""
    return torch.ops.sluice.fused_experts(hidden_states, w1, w2, topk_weights, topk_ids,
                                          activation=activation,
                                          global_num_experts=global_num_experts,
                                          expert_map=expert_map, **kw)


def _vllm_present() -> bool:
    try:
        import vllm  # noqa: F401

        return True
    except Exception:
        return False


if not _vllm_present() and not hasattr(torch.ops.vllm, "fused_experts"):
    @torch.library.custom_op("vllm::fused_experts", mutates_args=())
    def _vllm_fused_experts(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                            topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                            activation: str = "silu", global_num_experts: int = -1,
                            expert_map: Optional[torch.Tensor] = None,
                            w1_scale: Optional[torch.Tensor] = None,
                            w2_scale: Optional[torch.Tensor] = None,
                            block_shape: Optional[list[int]] = None,
                            routed_scaling_factor: float = 1.0,
                            shared_output: Optional[torch.Tensor] = None,
                            shared_w1: Optional[torch.Tensor] = None,
                            shared_w2: Optional[torch.Tensor] = None,
                            shared_w1_scale: Optional[torch.Tensor] = None,
                            shared_w2_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
        return _fused_experts_impl(hidden_states, w1, w2, topk_weights, topk_ids, activation,
                                   global_num_experts, expert_map, w1_scale, w2_scale,
                                   block_shape, routed_scaling_factor, shared_output, shared_w1,
                                   shared_w2, shared_w1_scale, shared_w2_scale)

    @_vllm_fused_experts.register_fake
    def _(hidden_states, w1, w2, topk_weights, topk_ids, activation="silu",
          global_num_experts=-1, expert_map=None, w1_scale=None, w2_scale=None,
          block_shape=None, routed_scaling_factor=1.0, shared_output=None, shared_w1=None,
          shared_w2=None, shared_w1_scale=None, shared_w2_scale=None):
        return torch.empty_like(hidden_states)


# ---------------------------------------------------------------------------
# Pinned host store
# ---------------------------------------------------------------------------
# base address -> HostStore of every live store (weak: the registry keeps
# nothing alive).
_HOST_STORES: "weakref.WeakValueDictionary" = weakref.WeakValueDictionary()


def pinned_store_bytes() -> int:
    """Bytes of every live HostStore of the process."""
    return sum(st.nbytes for st in list(_HOST_STORES.values()))


def host_store_of(t: torch.Tensor):
    """The HostStore whose allocation holds all of tensor ``t`` (a CPU
    tensor), or None."""
    if t.device.type != "cpu":
        return None
    lo = t.data_ptr()
    hi = lo + t.numel() * t.element_size()
    for base, st in list(_HOST_STORES.items()):
        if base <= lo and hi <= base + st.nbytes:
            return st
    return None


def _free_host(ptr: int) -> None:
    lib = _lib._lib
    if lib is not None:
        lib.sluice_host_free(ptr)


class HostStore:
    """Exact-size pinned host buffer (hipHostMalloc) viewed as a CPU tensor.

    The memory lives as long as any tensor viewing it: the tensor keeps the
    buffer object it was made from, and the buffer's finalizer frees the
    allocation when the last view goes (no reference cycle, so nothing
    waits for the cycle collector).  Memory still held at interpreter exit is
    left to the process teardown."""

    def __init__(self, shape, dtype: torch.dtype):
        lib = _lib.load()
        n = int(np.prod(shape))
        esz = torch.empty((), dtype=dtype).element_size()
        self.nbytes = n * esz
        p = ctypes.c_void_p()
        _lib.check(lib.sluice_host_alloc(max(self.nbytes, 1), ctypes.byref(p)), "sluice_host_alloc")
        self._ptr = p.value
        raw = (ctypes.c_uint8 * max(self.nbytes, 1)).from_address(self._ptr)
        fin = weakref.finalize(raw, _free_host, self._ptr)
        fin.atexit = False
        arr = np.frombuffer(raw, dtype=np.uint8, count=self.nbytes)
        self.tensor = torch.from_numpy(arr).view(dtype).view(*shape)
        _HOST_STORES[self._ptr] = self

    def data_ptr(self) -> int:
        return self._ptr
