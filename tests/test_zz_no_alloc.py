"""The no-allocation expert product (sluice_fused_experts_bf16_noalloc): its
results equal the bits of sluice_fused_experts_bf16 with a caller workspace,
on two calls in a row (the second smaller, so it runs over the first call's
leftover scratch contents), both called through the C ABI; calls too large
for the fixed scratch are refused before any device work."""

import ctypes

import numpy as np
import pytest
import torch

from sluice_amd import _lib

DEV = torch.device("cuda:0")


def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)


def _case(T, H, I, E, S, k, shared_I, rng):
    x = _bf16(rng.standard_normal((T, H))).to(DEV)
    w13 = _bf16(rng.standard_normal((S, 2 * I, H)) * 0.02).to(DEV)
    w2 = _bf16(rng.standard_normal((S, H, I)) * 0.02).to(DEV)
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    emap = np.full(E, -1, np.int32)
    emap[rng.choice(E, size=S, replace=False)] = np.arange(S, dtype=np.int32)
    emap[rng.choice(E, size=E // 8, replace=False)] = -1  # some selected experts miss
    tw = torch.from_numpy(rng.random((T, k), dtype=np.float32)).to(DEV)
    sw13 = sw2 = None
    if shared_I:
        sw13 = _bf16(rng.standard_normal((2 * shared_I, H)) * 0.02).to(DEV)
        sw2 = _bf16(rng.standard_normal((H, shared_I)) * 0.02).to(DEV)
    return dict(x=x, w13=w13, w2=w2, ids=torch.from_numpy(ids).to(DEV),
                emap=torch.from_numpy(emap).to(DEV), tw=tw, sw13=sw13, sw2=sw2, T=T, H=H, I=I,
                E=E, S=S, k=k, shared_I=shared_I)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _run(lib, c, noalloc, plan=None):
    out = torch.full((c["T"], c["H"]), float("nan"), dtype=torch.bfloat16, device=DEV)
    st = torch.cuda.current_stream(DEV).cuda_stream
    common = (c["x"].data_ptr(), c["w13"].data_ptr(), c["w2"].data_ptr(), c["tw"].data_ptr(),
              c["ids"].data_ptr(), c["emap"].data_ptr(), c["T"], c["H"], c["I"], c["k"], c["E"],
              c["S"], 1.0, _ptr(c["sw13"]), _ptr(c["sw2"]), c["shared_I"], None)
    if noalloc:
        rc = lib.sluice_fused_experts_bf16_noalloc(*common, out.data_ptr(), _ptr(plan), st)
        _lib.check(rc, "sluice_fused_experts_bf16_noalloc")
    else:
        nb = lib.sluice_fused_experts_workspace(c["T"], c["H"], c["I"], c["k"], c["shared_I"])
        ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
        rc = lib.sluice_fused_experts_bf16(*common, ws.data_ptr(), ws.numel(), out.data_ptr(),
                                           _ptr(plan), st)
        _lib.check(rc, "sluice_fused_experts_bf16")
    return out


def test_oversize_call_refused_without_device_work(lib):
    """A call whose workspace exceeds the fixed scratch returns
    SLUICE_E_SCRATCH before anything is looked up or launched (the pointers
    are aligned stand-ins that nothing may dereference)."""
    fake = 1 << 20
    T, H, I, k = 512, 7168, 2048, 8
    assert lib.sluice_fused_experts_workspace(T, H, I, k, 0) > _lib.NOALLOC_SCRATCH_BYTES
    rc = lib.sluice_fused_experts_bf16_noalloc(fake, fake, fake, fake, fake, fake, T, H, I, k, 256,
                                               64, 1.0, None, None, 0, None, fake, None, None)
    assert rc == _lib.SLUICE_E_SCRATCH
    assert "scratch" in _lib.strerror(rc)


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_on_two_calls():
    lib = _lib.load()
    torch.cuda.set_device(DEV)
    rng = np.random.default_rng(7)
    # a DeepSeek-V2-Lite-shaped layer step with its two shared experts, then a
    # smaller Qwen3-shaped step without them
    cases = [_case(8, 2048, 1408, 64, 48, 6, 2816, rng), _case(3, 2048, 768, 128, 64, 8, 0, rng)]
    for n, c in enumerate(cases):
        print(f"noalloc call {n}: T={c['T']} H={c['H']} I={c['I']} k={c['k']} "
              f"shared_I={c['shared_I']}", flush=True)
        assert (lib.sluice_fused_experts_workspace(c["T"], c["H"], c["I"], c["k"], c["shared_I"])
                <= _lib.NOALLOC_SCRATCH_BYTES)
        got = _run(lib, c, noalloc=True)
        want = _run(lib, c, noalloc=False)
        torch.cuda.synchronize()
        assert not torch.isnan(want.float()).any()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), n


@pytest.mark.gpu
def test_noalloc_over_a_gap_plan_with_streaming_slots_matches_workspace_entry(monkeypatch):
    """The no-allocation entry on the router-split path: a layer's gap with
    misses (answered before its rows land, so the product's plan flags the
    filled slots pending and the split launch runs, its hand-off counters in
    the fixed scratch) builds the plan in the layer's plan buffer; the
    no-allocation entry over that plan and the layer's registered map gives
    the bits of the workspace entry over the same plan, on two gaps in a row
    (the second smaller)."""
    import types

    import torch.nn as nn

    from sluice_amd.offloader import ExpertStreamOffloader

    class _Layer(nn.Module):
        def __init__(self, E, H, I):
            super().__init__()
            self.global_num_experts = self.local_num_experts = E
            self.quant_method = types.SimpleNamespace()
            g = torch.Generator().manual_seed(E)
            self.w13_weight = nn.Parameter(
                (torch.randn((E, 2 * I, H), generator=g) * 0.02).to(torch.bfloat16),
                requires_grad=False)
            self.w2_weight = nn.Parameter(
                (torch.randn((E, H, I), generator=g) * 0.02).to(torch.bfloat16),
                requires_grad=False)

    lib = _lib.load()
    torch.cuda.set_device(DEV)
    E, S, k, H, I = 64, 32, 4, 1024, 512
    monkeypatch.setenv("SLUICE_ROUTER_SPLIT", "1")
    monkeypatch.setenv("SLUICE_RS_FAST_HIT", "0")
    layer = _Layer(E, H, I)
    off = ExpertStreamOffloader(expert_cache_slots=S)
    off.wrap_modules(iter([layer]))
    with torch.cuda.device(DEV):
        off.post_init()
    cache = off._caches[id(layer)]
    off._rs_caches.append(cache)
    cache.plan = torch.zeros(lib.sluice_moe_plan_ints(S // k, k), dtype=torch.int32, device=DEV)
    rng = np.random.default_rng(11)
    for n, T in enumerate((8, 5)):
        m = cache.expert_map_buf.cpu().numpy()
        absent = np.flatnonzero(m < 0)
        ids_np = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
        if not np.isin(ids_np, absent).any():  # at least one selected expert misses
            ids_np[0, 0] = next(a for a in absent if a not in ids_np[0])
        ids = torch.from_numpy(ids_np).to(DEV)
        x = _bf16(rng.standard_normal((T, H))).to(DEV)
        torch.ops.vllm.sluice_stream_gap(x, ids, 0)  # inline gap: misses, plan built
        c = dict(x=x, w13=cache.gpu_cache["w13_weight"], w2=cache.gpu_cache["w2_weight"],
                 ids=ids, emap=cache.expert_map_buf,
                 tw=torch.from_numpy(rng.random((T, k), dtype=np.float32)).to(DEV),
                 sw13=None, sw2=None, T=T, H=H, I=I, E=E, S=S, k=k, shared_I=0)
        pend = int(cache.plan[2].item())  # resident blocks; pending ones follow
        print(f"noalloc over a gap plan {n}: T={T}, {int(cache.plan[0].item())} blocks, "
              f"{pend} resident", flush=True)
        assert int(cache.plan[0].item()) > pend  # the plan has pending (streaming) blocks
        got = _run(lib, c, noalloc=True, plan=cache.plan)
        want = _run(lib, c, noalloc=False, plan=cache.plan)
        torch.cuda.synchronize()
        assert not torch.isnan(want.float()).any()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), n
    off.close()
