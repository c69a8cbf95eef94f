"""Kernels of the synthetic decoders (include/sluice_decoder.h) against plain
float32 torch references of the same math, computed on the CPU from the same
bf16 inputs: residual add + RMSNorm, SwiGLU activation, router logits, MLA
and GQA decode attention (with their cache layouts)."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 1e-2


def _lib():
    from sluice_amd import _lib

    return _lib.load(), _lib.check


def _st():
    return torch.cuda.current_stream().cuda_stream


def _rel(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / max(b.norm(), 1e-30))


def _rope(x, cos, sin):
    d = x.shape[-1] // 2
    x1, x2 = x[..., :d], x[..., d:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)


def _rms(x, w, eps=1e-6):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


@pytest.mark.parametrize("rows,H,with_delta", [(8, 2048, True), (1, 7168, False), (12, 2048, True)])
def test_add_rmsnorm(rows, H, with_delta):
    from sluice_amd.decoder import add_rmsnorm

    g = torch.Generator().manual_seed(rows + H)
    x = torch.randn((rows, H), generator=g).bfloat16()
    d = torch.randn((rows, H), generator=g).bfloat16() if with_delta else None
    w = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16()
    xd = x.to(DEV)
    out = add_rmsnorm(xd, None if d is None else d.to(DEV), w.to(DEV))
    torch.cuda.synchronize()
    xs = (x.float() + d.float()).bfloat16() if with_delta else x
    assert torch.equal(xd.cpu(), xs)  # the residual stream is the bf16 sum, in place
    ref = _rms(xs.float(), w.float())
    assert _rel(out, ref) <= TOL


def test_silu_mul():
    from sluice_amd.decoder import silu_mul

    g = torch.Generator().manual_seed(3)
    gu = torch.randn((8, 2 * 2816), generator=g).bfloat16()
    out = silu_mul(gu.to(DEV))
    torch.cuda.synchronize()
    gf, uf = gu.float()[:, :2816], gu.float()[:, 2816:]
    assert _rel(out, gf * torch.sigmoid(gf) * uf) <= TOL


@pytest.mark.parametrize("rows,H,E,bias", [(8, 2048, 64, True), (1, 2048, 128, False),
                                           (12, 7168, 256, True)])
def test_gate_logits(rows, H, E, bias):
    lib, check = _lib()
    g = torch.Generator().manual_seed(E + rows)
    hn = torch.randn((rows, H), generator=g).bfloat16()
    wg = (0.02 * torch.randn((E, H), generator=g)).bfloat16()
    steps, brow = 5, 16
    table = torch.randn((steps, brow, E), generator=g)
    step = torch.tensor(7, dtype=torch.long)  # wraps to row 7 % 5 = 2
    out = torch.empty((rows, E), dtype=torch.float32, device=DEV)
    d = {k: v.to(DEV) for k, v in dict(hn=hn, wg=wg, table=table, step=step).items()}
    check(lib.sluice_dec_gate_logits(d["hn"].data_ptr(), d["wg"].data_ptr(),
                                     d["table"].data_ptr() if bias else None,
                                     d["step"].data_ptr() if bias else None, steps if bias else 0,
                                     brow if bias else 0, rows, H, E, out.data_ptr(), _st()),
          "gate_logits")
    torch.cuda.synchronize()
    ref = hn.float() @ wg.float().T
    if bias:
        ref = ref + table[2, :rows]
    assert torch.allclose(out.cpu(), ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("rows,H,E,delta,bias", [(8, 2048, 128, True, True),
                                                 (1, 2048, 64, True, False),
                                                 (12, 2048, 128, False, True),
                                                 (16, 2048, 60, True, True),
                                                 (8, 4096, 256, True, True),
                                                 (12, 7168, 256, True, True),
                                                 (3, 2560, 7, True, False)])
def test_add_rmsnorm_gate_matches_the_two_kernels(rows, H, E, delta, bias):
    """The fused norm + router logits against add_rmsnorm then gate_logits:
    hn and the residual bit for bit; logits bit for bit at H == 2048 (same
    element order), to fp32 rounding otherwise."""
    from sluice_amd.decoder import add_rmsnorm

    lib, check = _lib()
    assert lib.sluice_dec_add_rmsnorm_gate_ok(rows, H)
    g = torch.Generator().manual_seed(rows * 7 + H + E)
    x = torch.randn((rows, H), generator=g).bfloat16()
    dl = torch.randn((rows, H), generator=g).bfloat16() if delta else None
    w = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16()
    wg = (0.02 * torch.randn((E, H), generator=g)).bfloat16()
    steps, brow = 5, 16
    table = torch.randn((steps, brow, E), generator=g)
    step = torch.tensor(7, dtype=torch.long)
    d = {k: v.to(DEV) for k, v in dict(x=x, w=w, wg=wg, table=table, step=step).items()}
    dd = dl.to(DEV) if delta else None
    x_out, hn = torch.empty_like(d["x"]), torch.empty_like(d["x"])
    lg = torch.empty((rows, E), dtype=torch.float32, device=DEV)
    bargs = ((d["table"].data_ptr(), d["step"].data_ptr(), steps, brow) if bias
             else (None, None, 0, 0))
    check(lib.sluice_dec_add_rmsnorm_gate(
        d["x"].data_ptr(), dd.data_ptr() if delta else None, None, 0, d["w"].data_ptr(),
        x_out.data_ptr(), hn.data_ptr(), d["wg"].data_ptr(), *bargs, rows, H, E, 1e-6,
        lg.data_ptr(), _st()), "add_rmsnorm_gate")
    # the two-kernel path on a copy of x
    x2 = d["x"].clone()
    hn2 = add_rmsnorm(x2, dd, d["w"])
    lg2 = torch.empty_like(lg)
    check(lib.sluice_dec_gate_logits(hn2.data_ptr(), d["wg"].data_ptr(), *bargs, rows, H, E,
                                     lg2.data_ptr(), _st()), "gate_logits")
    torch.cuda.synchronize()
    assert torch.equal(d["x"].cpu(), x)  # x itself is not written
    assert torch.equal(x_out.cpu(), x2.cpu())
    assert torch.equal(hn.cpu(), hn2.cpu())
    if H == 2048:
        assert torch.equal(lg.cpu(), lg2.cpu())
    else:
        assert torch.allclose(lg.cpu(), lg2.cpu(), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("T,H,K,E", [(8, 2048, 4096, 128), (1, 2048, 4096, 128),
                                     (12, 2048, 2048, 64), (16, 2048, 8192, 128),
                                     (4, 1040, 4096, 8), (8, 4096, 2048, 128),
                                     (8, 7168, 2048, 256), (3, 7168, 4096, 256)])
def test_linear_split_parts_into_the_fused_norm(T, H, K, E):
    """A projection left as its K parts and summed by the fused norm gives the
    same residual, hn and logits, bit for bit, as bf16(in-order sum of the
    parts) fed to it as a bf16 delta; that sum is the projection (to fp32
    rounding of a different K split)."""
    from sluice_amd.decoder import linear

    lib, check = _lib()
    g = torch.Generator().manual_seed(T * 31 + K)
    o = torch.randn((T, K), generator=g).bfloat16().to(DEV)
    wo = (0.02 * torch.randn((H, K), generator=g)).bfloat16().to(DEV)
    x = torch.randn((T, H), generator=g).bfloat16().to(DEV)
    w = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16().to(DEV)
    wg = (0.02 * torch.randn((E, H), generator=g)).bfloat16().to(DEV)
    ks = lib.sluice_dec_linear_split_parts(T, H, K)
    assert 1 <= ks <= 4
    parts = torch.empty((ks, T, H), dtype=torch.float32, device=DEV)
    check(lib.sluice_dec_linear_split(o.data_ptr(), wo.data_ptr(), T, H, K, parts.data_ptr(),
                                      _st()), "linear_split")
    torch.cuda.synchronize()
    s = parts[0].clone()
    for p in range(1, ks):
        s = s + parts[p]
    y = s.bfloat16()
    assert _rel(y, linear(o, wo).float()) <= 1e-2
    outs = []
    for src in ("bf16", "parts"):
        x_out, hn = torch.empty_like(x), torch.empty_like(x)
        lg = torch.empty((T, E), dtype=torch.float32, device=DEV)
        check(lib.sluice_dec_add_rmsnorm_gate(
            x.data_ptr(), y.data_ptr() if src == "bf16" else None,
            parts.data_ptr() if src == "parts" else None, ks if src == "parts" else 0,
            w.data_ptr(), x_out.data_ptr(), hn.data_ptr(), wg.data_ptr(), None, None, 0, 0, T, H,
            E, 1e-6, lg.data_ptr(), _st()), "add_rmsnorm_gate")
        outs.append((x_out, hn, lg))
    torch.cuda.synchronize()
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("T,N,K", [(8, 3648, 2048), (1, 2048, 10944), (12, 5632, 2048),
                                   (16, 160, 128), (5, 176, 192), (8, 576, 2048)])
def test_linear(T, N, K):
    from sluice_amd.decoder import linear

    g = torch.Generator().manual_seed(T * N + K)
    x = torch.randn((T, K), generator=g).bfloat16()
    w = (0.02 * torch.randn((N, K), generator=g)).bfloat16()
    y = linear(x.to(DEV), w.to(DEV))
    torch.cuda.synchronize()
    assert _rel(y, x.float() @ w.float().T) <= TOL


@pytest.mark.parametrize("T,I,K", [(8, 2816, 2048), (1, 10944, 2048), (12, 2048, 7168), (3, 16, 128)])
def test_linear_glu(T, I, K):
    """Gate/up projection with SwiGLU applied to the fp32 sums (rows 0..I-1
    gate, I..2I-1 up) against fp32 torch."""
    from sluice_amd.decoder import linear_glu

    g = torch.Generator().manual_seed(T + I + K)
    x = torch.randn((T, K), generator=g).bfloat16()
    w = (0.02 * torch.randn((2 * I, K), generator=g)).bfloat16()
    y = linear_glu(x.to(DEV), w.to(DEV))
    torch.cuda.synchronize()
    gu = x.float() @ w.float().T
    gf, uf = gu[:, :I], gu[:, I:]
    assert y.shape == (T, I)
    assert _rel(y, gf * torch.sigmoid(gf) * uf) <= TOL


def test_linear_split_k_deterministic_and_counters_back_at_zero():
    """A small matrix splits K over several workgroups (partials handed over
    through the workspace): repeated calls give identical bits, the result
    agrees with the unsplit kernel (no workspace) within rounding, and the
    workspace's counters are back at zero."""
    import ctypes

    from sluice_amd import _lib
    from sluice_amd.decoder import _linear_ws

    lib = _lib.load()
    T, N, K = 8, 2048, 2816
    g = torch.Generator().manual_seed(5)
    x = torch.randn((T, K), generator=g).bfloat16().to(DEV)
    w = (0.02 * torch.randn((N, K), generator=g)).bfloat16().to(DEV)
    ws = _linear_ws(torch.device(DEV))
    st = torch.cuda.current_stream().cuda_stream
    outs = []
    for wsp in (ws.data_ptr(), ws.data_ptr(), None):
        y = torch.empty((T, N), dtype=torch.bfloat16, device=DEV)
        _lib.check(lib.sluice_dec_linear(x.data_ptr(), w.data_ptr(), T, N, K, y.data_ptr(), wsp,
                                         st), "linear")
        outs.append(y)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert _rel(outs[0], outs[2].float()) <= TOL
    assert _rel(outs[0], x.float() @ w.float().T) <= TOL
    n_ws = int(lib.sluice_dec_linear_workspace())
    counters = ws[n_ws - 4096:n_ws].view(torch.int32)
    assert int(counters.abs().sum()) == 0


@pytest.mark.parametrize("T,N", [(1, 151936), (8, 102400), (3, 1000), (2, 1001)])
def test_argmax(T, N):
    from sluice_amd.decoder import argmax_rows

    g = torch.Generator().manual_seed(N + T)
    x = torch.randn((T, N), generator=g).bfloat16()
    x[0, N // 3] = 50.0  # a clear winner
    x[0, 3] = float("nan")  # NaN never wins
    x[-1, 7] = x[-1, N - 1] = 60.0  # a tie: the first index wins
    out = argmax_rows(x.to(DEV), torch.zeros(T, dtype=torch.long, device=DEV))
    torch.cuda.synchronize()
    ref = torch.argmax(torch.nan_to_num(x.float(), nan=-float("inf")), dim=-1)
    assert torch.equal(out.cpu(), ref)
    assert int(out[-1]) == 7


def test_argmax_replays_in_a_graph():
    """Captured once, replayed several times with new inputs in between: each
    replay's result equals the eager one."""
    from sluice_amd.decoder import argmax_rows

    x = torch.zeros((1, 151936), dtype=torch.bfloat16, device=DEV)
    out = torch.zeros(1, dtype=torch.long, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        argmax_rows(x, out)
    torch.cuda.current_stream().wait_stream(s)
    for i, pos in enumerate([5, 151935, 77777, 0, 123456]):
        x.zero_()
        x[0, pos] = 1.0 + i
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert int(out[0]) == pos


def _tables(L, d, theta):
    inv = 1.0 / (theta ** (torch.arange(0, d, 2).float() / d))
    ang = torch.arange(L).float()[:, None] * inv[None, :]
    return ang.cos().contiguous(), ang.sin().contiguous()


def _mla_kpos(r):
    return 8 * ((r & 15) >> 2) + 4 * (r >> 4) + (r & 3)


@pytest.mark.parametrize("L,positions,vh", [(64, [5, 0, 63, 31], 128),
                                            (512, [300, 1, 511, 130], 128),
                                            (256, [200, 17, 255, 64], 192),
                                            (4096, [4095, 2047, 64, 700], 128)])
def test_mla_decode(L, positions, vh):
    lib, check = _lib()
    c, nh, nope, rope, lora = 4, 16, 128, 64, 512
    g = torch.Generator().manual_seed(11 + L)
    nq = nh * (nope + rope)
    qkva = torch.randn((c, nq + lora + rope), generator=g).bfloat16()
    kv_norm = (1 + 0.1 * torch.randn(lora, generator=g)).bfloat16()
    w_uk = (0.05 * torch.randn((nh, nope, lora), generator=g)).bfloat16()
    w_uv = (0.05 * torch.randn((nh, lora, vh), generator=g)).bfloat16()
    ckv = torch.randn((c, L, lora), generator=g).bfloat16()
    kpe = torch.randn((c, L, rope), generator=g).bfloat16()
    pos = torch.tensor(positions, dtype=torch.long)
    cos_t, sin_t = _tables(L, rope, 1e4)
    scale = (nope + rope) ** -0.5
    # the transposed latent cache: [c, L/32, lora, 32]
    kslot = torch.tensor([_mla_kpos(r) for r in range(32)])
    ckvt = torch.empty((c, L // 32, lora, 32), dtype=torch.bfloat16)
    ckvt[..., kslot] = ckv.view(c, L // 32, 32, lora).transpose(2, 3)
    d = {k: v.to(DEV) for k, v in dict(qkva=qkva, kv_norm=kv_norm,
                                       w_ukt=w_uk.transpose(1, 2).contiguous(), w_uv=w_uv,
                                       ckv=ckv.clone(), ckvt=ckvt, kpe=kpe.clone(), pos=pos,
                                       cos=cos_t, sin=sin_t).items()}
    out = torch.empty((c, nh * vh), dtype=torch.bfloat16, device=DEV)
    work = torch.empty(int(lib.sluice_dec_mla_workspace(c, nh)), dtype=torch.uint8, device=DEV)
    row = qkva.shape[1]
    check(lib.sluice_dec_mla_decode(
        d["qkva"].data_ptr(), row, d["qkva"].data_ptr() + nq * 2, row, d["kv_norm"].data_ptr(),
        d["w_ukt"].data_ptr(), d["w_uv"].data_ptr(), d["cos"].data_ptr(), d["sin"].data_ptr(),
        d["pos"].data_ptr(), c, nh, nope, rope, lora, vh, L, 1e-6, scale, d["ckv"].data_ptr(),
        d["ckvt"].data_ptr(), d["kpe"].data_ptr(), work.data_ptr(), out.data_ptr(), _st()),
        "mla_decode")
    torch.cuda.synchronize()
    ck, kp = ckv.clone(), kpe.clone()
    for t in range(c):
        p = int(pos[t])
        q = qkva[t, :nq].float().view(nh, nope + rope)
        qn, qp = q[:, :nope], _rope(q[:, nope:], cos_t[p], sin_t[p])
        ql = torch.bmm(qn[:, None, :], w_uk.float())[:, 0]
        kv = qkva[t, nq:].float()
        ck[t, p] = _rms(kv[:lora], kv_norm.float()).bfloat16()
        kp[t, p] = _rope(kv[lora:], cos_t[p], sin_t[p]).bfloat16()
        assert _rel(d["ckv"][t, p], ck[t, p].float()) <= TOL
        assert _rel(d["kpe"][t, p], kp[t, p].float()) <= TOL
        cf, kf = d["ckv"][t, : p + 1].float().cpu(), d["kpe"][t, : p + 1].float().cpu()
        s = (ql @ cf.T + qp @ kf.T) * scale
        pr = torch.softmax(s, dim=-1)
        o = torch.bmm((pr @ cf)[:, None, :], w_uv.float())[:, 0]
        assert _rel(out[t].view(nh, vh), o) <= TOL, t
    # rows other than pos[t] are untouched
    mask = torch.ones((c, L), dtype=torch.bool)
    mask[torch.arange(c), pos] = False
    assert torch.equal(d["ckv"].cpu()[mask], ckv[mask])
    # the transposed copy holds exactly the row-major cache, new rows included
    got = d["ckvt"].cpu()[..., kslot].transpose(2, 3).reshape(c, L, lora)
    assert torch.equal(got, d["ckv"].cpu())


def test_mla_decode_rejects_bad_shapes():
    lib, _ = _lib()
    x = torch.zeros(1 << 16, dtype=torch.uint8, device=DEV)
    p = x.data_ptr()
    args = dict(q=p, q_stride=3648, kva=p, kva_stride=3648, kv_norm=p, w_ukt=p, w_uv=p,
                cos=p, sin=p, pos=p, c=1, nh=16, nope=128, rope=64, lora=512, vh=128, L=64,
                eps=1e-6, scale=0.1, ckv=p, ckvt=p, kpe=p, work=p, out=p)

    def call(**kw):
        a = dict(args, **kw)
        return lib.sluice_dec_mla_decode(*a.values(), _st())

    for bad in (dict(nh=8), dict(vh=100), dict(L=48), dict(c=17), dict(nope=48),
                dict(lora=256), dict(rope=32), dict(q=p + 8)):
        assert call(**bad) != 0, bad


@pytest.mark.parametrize("L,positions", [(48, [7, 47, 0]), (600, [300, 599, 129]),
                                         (4096, [4095, 2500, 1])])
def test_gqa_decode(L, positions):
    lib, check = _lib()
    c, nh, kvh, hd = 3, 32, 4, 128
    g = torch.Generator().manual_seed(12 + L)
    qkv = torch.randn((c, (nh + 2 * kvh) * hd), generator=g).bfloat16()
    q_norm = (1 + 0.1 * torch.randn(hd, generator=g)).bfloat16()
    k_norm = (1 + 0.1 * torch.randn(hd, generator=g)).bfloat16()
    k = torch.randn((c, kvh, L, hd), generator=g).bfloat16()
    v = torch.randn((c, kvh, L, hd), generator=g).bfloat16()
    pos = torch.tensor(positions, dtype=torch.long)
    cos_t, sin_t = _tables(L, hd, 1e6)
    scale = hd ** -0.5
    d = {kk: vv.to(DEV) for kk, vv in dict(qkv=qkv, qn=q_norm, kn=k_norm, k=k.clone(), v=v.clone(),
                                           pos=pos, cos=cos_t, sin=sin_t).items()}
    out = torch.empty((c, nh * hd), dtype=torch.bfloat16, device=DEV)
    check(lib.sluice_dec_gqa_decode(
        d["qkv"].data_ptr(), None, 0, d["qn"].data_ptr(), d["kn"].data_ptr(), d["cos"].data_ptr(),
        d["sin"].data_ptr(), d["pos"].data_ptr(), c, nh, kvh, hd, L, 1e-6, scale,
        d["k"].data_ptr(), d["v"].data_ptr(), out.data_ptr(), _st()), "gqa_decode")
    # the same from the projection's K parts (qkv/4 + qkv/4 + qkv/2 sums to qkv exactly):
    # bit-identical output and cache rows
    qf = d["qkv"].float()
    parts = torch.stack([qf / 4, qf / 4, qf / 2]).contiguous()
    k2, v2 = k.clone().to(DEV), v.clone().to(DEV)
    out2 = torch.empty_like(out)
    check(lib.sluice_dec_gqa_decode(
        None, parts.data_ptr(), 3, d["qn"].data_ptr(), d["kn"].data_ptr(), d["cos"].data_ptr(),
        d["sin"].data_ptr(), d["pos"].data_ptr(), c, nh, kvh, hd, L, 1e-6, scale, k2.data_ptr(),
        v2.data_ptr(), out2.data_ptr(), _st()), "gqa_decode parts")
    torch.cuda.synchronize()
    for t in range(c):
        p = int(pos[t])
        x = qkv[t].float()
        qh = x[: nh * hd].view(nh, hd)
        kh = x[nh * hd: (nh + kvh) * hd].view(kvh, hd)
        vh_ = x[(nh + kvh) * hd:].view(kvh, hd)
        qr = _rope(_rms(qh, q_norm.float()), cos_t[p], sin_t[p])
        kr = _rope(_rms(kh, k_norm.float()), cos_t[p], sin_t[p])
        assert _rel(d["k"][t, :, p], kr) <= TOL
        assert torch.equal(d["v"][t, :, p].cpu(), vh_.bfloat16())
        kc, vc = d["k"][t, :, : p + 1].float().cpu(), d["v"][t, :, : p + 1].float().cpu()
        grp = nh // kvh
        for h in range(nh):
            s = (qr[h] @ kc[h // grp].T) * scale
            o = torch.softmax(s, dim=-1) @ vc[h // grp]
            assert _rel(out[t, h * hd:(h + 1) * hd], o) <= TOL, (t, h)
    assert torch.equal(out2, out)
    assert torch.equal(k2, d["k"]) and torch.equal(v2, d["v"])
    # rows other than pos[t] are untouched
    mask = torch.ones((c, L), dtype=torch.bool)
    mask[torch.arange(c), pos] = False
    for name, ref in (("k", k), ("v", v)):
        got = d[name].cpu().permute(0, 2, 1, 3)
        assert torch.equal(got[mask], ref.permute(0, 2, 1, 3)[mask]), name
