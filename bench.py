"""Decode benchmark of the router-split MoE hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config v2lite]
                    [--batches 1,8] [--slots S] [--no-extras] [--no-cpu-baseline]

A step is one decode step of the whole synthetic decoder at batch c: every
layer's attention/dense blocks and, per MoE layer, routing -> streaming gap
-> grouped SwiGLU expert product -> combine, then the LM head and greedy
next token.  The gap op is a device launch served by the native gap server,
so a whole step (gaps included) replays as one hipGraph.  Batches above the
router-split envelope (c > slots // top_k) take the classic wave path.

Per batch size: the step is captured, then the batch's 128-token synthetic
prompts are processed position by position through the captured step
(untimed; every prompt token is routed through every MoE layer, so the slot
caches start warm and the KV caches hold the prompts), then untimed decode
steps up to the middle of a 256-token decode (the last W of them the warm-up),
then the K timed steps, centred in the decode: positions 128+(256-K)/2 ..
+K (the stress row, without prompts, times from its first steps).  The timed
region is bracketed
by device synchronisation; ``value`` is tokens/s of the headline workload
(DeepSeek-V2-Lite shape, 48 slots, c=8).

Routing: logits = gate GEMM + ln Zipf(1.1) popularity + sigma * z_t, z_t a
unit-variance AR(1) with rho = 0.7 per sequence and layer (sigma 1.2, gate
weights N(0, 0.004): the selections' top-k share is the one Zipf(1.1)
popularity gives, and the logits' lag-1 correlation ~0.7).  The knobs and the
measured top-k share, unique experts and misses per layer-step are in the
line.  Rows labelled "locality" rerun the batch with sigma 0.5, whose
fast-hit share lies in the band the reference reports for real models; the
"matched" row reruns V2-Lite c=8 with sigma 0.8, where the share of fast-hit
gaps equals the reference's (86%).  Rows "in the reference's orchestration"
rerun the headline batches with the gaps eager between captured pieces and
each missing gap answered after its rows landed.  ``vs_published`` lists
every row that has a published reference figure, with both fast-hit shares.

Also measured in the same run:
  roofline      the dominant kernel (moe_gemm1: gate/up weights stream) timed
                with HIP events on its own stream over the recorded routing
                of every layer for 8 decode steps, layers rotating so the
                256 MB last-level cache cannot serve repeats; algorithmic
                bytes = U*2*I*H*2 (unique experts' w13) + T*H*2 + P*I*2.
                gemm2, the combine and the router are timed the same way.
  h2d           peak pinned host->device GB/s (64 MiB copies) and the rate of
                expert-row stream-ins issued like the gap issues them.
  extras        the other configurations: Qwen3-30B-A3B shape (48 layers)
                at 64 slots c=1/8 (c=12 on the classic wave path) and 96
                slots c=1/8/12, the DeepSeek-V3 fp8 MoE stack (8 layers, 64
                slots) at c=8, and the miss-dominated stress (Qwen3 shape, 32
                slots, uniform routing, c=4, --stress-steps timed steps), each
                with its gemm1 roofline fraction and H2D rate.

Output: the full record (every row, kernel and baseline figure) goes to
--record and to stderr; the last stdout line is a compact headline object
(compact_line: the contract's fields, roofline, cpu_baseline, H2D rates and
one short row per measured batch), kept under LINE_LIMIT bytes.
  cpu_baseline  the path in torch fp32 on the host cores (oracle/cpu_path.py)
                on one DeepSeek-V2-Lite-shaped layer, per-stage medians.
"""

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

DEFAULT_SLOTS = {"v2lite": 48, "qwen3": 64, "v3": 64}
PUBLISHED_C8 = {"v2lite": 1062.6}  # reference, 1xH100 router-split, c=8 (tok/s)
# The reference's published router-split decode (1xH100, real-model routing):
# tok/s by slots and batch, and the share of its gaps that take the fast-hit
# path (V2-Lite: README.md:51, docs/router-split.md:324, 330; Qwen3-30B-A3B:
# README.md:66-67, docs/router-split.md:360, 375, 384).
PUBLISHED = {
    "v2lite": {"tok_per_s": {48: {1: 147.2, 8: 1062.6}}, "fast_hit_share": 0.86},
    "qwen3": {"tok_per_s": {64: {1: 121.2, 8: 864.5}, 96: {1: 122.8, 8: 883.7, 12: 1263.8}},
              "fast_hit_share": 0.99},
}
# Routing noise at which a batch's gaps take the fast-hit path as often as the
# reference's do (86% for V2-Lite; measured 86.2% at c=8 with sigma 0.8); the
# Zipf rows (sigma 1.2) are the configured workload, these rows the like-for-like one.
MATCHED_SIGMA = {"v2lite": {8: 0.8}}
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
DECODE_LEN = 256   # output tokens of the configured decode
PROMPT_LEN = 128
ROUTING = {"zipf_s": 1.1, "rho": 0.7, "sigma": 1.2, "gate_std": 0.004}
LOCALITY_SIGMA = 0.5
ORCH_GRAPH = "one graph per step, gap served by the native thread, misses pipelined"
ORCH_REFERENCE = ("reference: eager gap between captured pieces (host waits for each layer's "
                  "ids), expert product after the copies")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="v2lite", choices=sorted(DEFAULT_SLOTS))
    ap.add_argument("--batches", default=None)
    ap.add_argument("--slots", type=int, default=None)
    ap.add_argument("--uniform", action="store_true", help="i.i.d. uniform routing (stress)")
    ap.add_argument("--sigma", type=float, default=ROUTING["sigma"])
    ap.add_argument("--layers", type=int, default=None)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="only the headline configuration (no Qwen3 / V3 / stress rows)")
    ap.add_argument("--no-locality", action="store_true",
                    help="skip the sigma-0.5 locality rows")
    ap.add_argument("--no-reference", action="store_true",
                    help="skip the rows in the reference's orchestration")
    ap.add_argument("--host-pool", default="auto", choices=["auto", "shared", "per-layer"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget-s", type=float, default=20.0)
    ap.add_argument("--save-routing", default=None,
                    help="also write the routing the roofline is timed over (.npz)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="time only the kernels, over the routing of --load-routing, and print "
                         "that (no decode: the workload of the counter runs)")
    ap.add_argument("--load-routing", default=None)
    ap.add_argument("--stress-steps", type=int, default=64,
                    help="timed steps of the miss-dominated stress row (uniform i.i.d. routing "
                         "is stationary, so the per-step figure does not depend on the count)")
    ap.add_argument("--record", default="bench_record.json",
                    help="file for the full record (every row, kernel and baseline figure); "
                         "the last stdout line is the compact headline object")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def run_batch(dec, c, steps, warmup, prefill=True, label=None):
    """Capture batch c, process its prompts (untimed), decode untimed up to
    the middle of the configured decode, W warm-up steps, then time K steps
    (the window centred in the decode); counters are the timed steps' own.
    Without prompts (the uniform stress) the window starts at once."""
    import torch

    if c not in dec.graphs:
        dec.capture(c)
    t0 = time.perf_counter()
    if prefill:
        dec.prefill(c)
    else:
        dec.reset(c)
    dec.sync()
    prefill_s = time.perf_counter() - t0
    lead = max(0, (DECODE_LEN - steps) // 2 - warmup) if prefill else 0
    for _ in range(lead + warmup):
        dec.step_graphs(c)
    dec.sync()
    before = dec.gap_counters()
    stage0 = dec.off.stage_counters()
    codec0 = dec.off.codec_counters()
    cl0 = dec.off.classic_counters()
    pos0 = int(dec.state[c].pos[0]) if dec.has_attn else None
    # per-step times from events between the steps (the value is the
    # wall-clock total); they show whether a slow window is one stall or
    # every step
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        marks[i].record(stream)
        dec.step_graphs(c)
    marks[steps].record(stream)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    per_step = sorted(marks[i].elapsed_time(marks[i + 1]) for i in range(steps))
    dec.sync()
    after = dec.gap_counters()
    delta = {k: after[k] - before[k] for k in after}
    stage1 = dec.off.stage_counters()
    sdelta = {k: stage1[k] - stage0[k] for k in ("filled", "h2d_bytes", "hits", "hit_bytes")}
    codec1 = dec.off.codec_counters()
    cl1 = dec.off.classic_counters()
    n_moe = len(dec.moe_layers)
    # bytes over the host link: the slot fills' copies from the host store
    # (coded rows where the store is coded), plus the staging copies (a fill
    # from a staged row moves HBM to HBM)
    fill = delta["bytes"] / steps
    link = codec1["link_bytes"] - codec0["link_bytes"]
    h2d = (link + sdelta["h2d_bytes"]) / steps
    return {
        "c": c, "steps": steps, "path": "classic" if dec.classic(c) else "gap",
        "routing": label or "zipf",
        "orchestration": ORCH_GRAPH if dec.off._server is not None else ORCH_REFERENCE,
        "ms_per_step": dt / steps * 1e3, "tok_per_s": c * steps / dt,
        "classic_steps": cl1["steps"] - cl0["steps"],
        "waves_per_classic_step": (cl1["waves"] - cl0["waves"]) / max(cl1["steps"] - cl0["steps"],
                                                                      1),
        "gap_calls": delta["gaps"], "misses": delta["misses"],
        "fast_hits": delta["fast_hits"], "map_writes": delta["map_writes"],
        "h2d_bytes_per_step": h2d, "h2d_GBs_in_step": h2d / (dt / steps) / 1e9,
        "fill_bytes_per_step": fill, "fill_GBs_in_step": fill / (dt / steps) / 1e9,
        "staged": {"rows_per_layer": stage1["rows"] // max(n_moe, 1),
                   "hits": sdelta["hits"],
                   "hit_share_of_misses": sdelta["hits"] / max(delta["misses"], 1),
                   "rows_filled": sdelta["filled"],
                   "staging_h2d_bytes_per_step": sdelta["h2d_bytes"] / steps},
        "coded": {"layers": codec1["layers"], "of_layers": n_moe,
                  "store_ratio": codec1["coded_bytes"] / max(codec1["store_bytes"], 1),
                  "decodes": codec1["decodes"] - codec0["decodes"],
                  "fill_link_bytes_per_step": link / steps},
        "misses_per_layer_step": delta["misses"] / max(steps * n_moe, 1),
        "fast_hit_share": delta["fast_hits"] / max(delta["gaps"], 1),
        "prefill": {"tokens_per_sequence": dec.prompt_len if prefill else 0,
                    "seconds": prefill_s},
        "untimed_decode_steps": lead + warmup,
        "timed_positions": [pos0, pos0 + steps] if pos0 is not None else None,
        "step_ms_min_median_max": [per_step[0], per_step[len(per_step) // 2], per_step[-1]]
        if per_step else None,
    }


def routing_stats(dec, recorded):
    """Properties of the routing the step actually ran (recorded steps): the
    share of selections that go to each layer's k most selected experts
    (against what Zipf(zipf_s) popularity gives them), unique experts per
    layer-step, the gate term's standard deviation and the logits' lag-1
    correlation that follows from it."""
    import torch

    sp, knobs = dec.sp, dec.routing_knobs
    E, k = sp["E"], sp["k"]
    by_layer = {}
    for r in recorded:
        by_layer.setdefault(r["n"], []).append(r["ti"].cpu().numpy())
    shares, uniq = [], []
    for lst in by_layer.values():
        cnt = np.bincount(np.concatenate([a.reshape(-1) for a in lst]), minlength=E)
        shares.append(np.sort(cnt)[::-1][:k].sum() / max(cnt.sum(), 1))
        uniq += [len(np.unique(a)) for a in lst]
    out = {"top_k_share": float(np.mean(shares)), "unique_per_layer_step": float(np.mean(uniq)),
           "recorded_steps": len(recorded) // max(len(by_layer), 1)}
    if "zipf_s" in knobs:
        p = 1.0 / np.arange(1, E + 1) ** knobs["zipf_s"]
        out["zipf_top_k_share"] = float(p[:k].sum() / p.sum())
        m = dec.moe_layers[0]
        hn = torch.stack([r["hn"] for r in recorded if r["n"] == 0]).float()
        g = float((hn @ m.gate.weight.float().T).std())
        sig = knobs["sigma"]
        out["gate_logit_std"] = g
        out["lag1_logit_corr"] = knobs["rho"] * sig * sig / (sig * sig + g * g)
    return out


def record_routing(dec, c, steps):
    """Decode `steps` more steps and keep every MoE layer's routing of each,
    with the expert map the step's gap left (the tensors the captured step
    rewrites are cloned after every replay)."""
    import torch

    out = []
    for _ in range(steps):
        dec.step_graphs(c)
        torch.cuda.synchronize()
        for n, io in enumerate(dec.layer_io[c]):
            out.append({"n": n, "hn": io["hn"].clone(), "ti": io["ti"].clone(),
                        "tw": io["tw"].clone(), "map": dec.moe_layers[n]._expert_map.clone()})
    dec.sync()
    return out


def save_routing(path, recorded):
    import torch

    np.savez(path, n=np.array([r["n"] for r in recorded], np.int32),
             hn=torch.stack([r["hn"] for r in recorded]).view(torch.int16).cpu().numpy(),
             ti=torch.stack([r["ti"] for r in recorded]).cpu().numpy(),
             tw=torch.stack([r["tw"] for r in recorded]).cpu().numpy(),
             map=torch.stack([r["map"] for r in recorded]).cpu().numpy())


def load_routing(path, dev):
    import torch

    z = np.load(path)
    hn = torch.from_numpy(z["hn"]).to(dev).view(torch.bfloat16)
    return [{"n": int(z["n"][i]), "hn": hn[i], "ti": torch.from_numpy(z["ti"][i]).to(dev),
             "tw": torch.from_numpy(z["tw"][i]).to(dev),
             "map": torch.from_numpy(z["map"][i]).to(dev)} for i in range(len(z["n"]))]


def _event_loop(stream, fn, items, reps):
    import torch

    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for it in items:  # warm
            fn(it)
        e0.record(stream)
        for _ in range(reps):
            for it in items:
                fn(it)
        e1.record(stream)
    stream.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * len(items))


def _graph_loop(stream, fn, items, reps):
    """Like _event_loop for kernels shorter than a host launch: one pass over
    the items is captured as a hipGraph and replayed, as the decode step runs
    them (dispatch gaps inside the graph included, host launch cost not)."""
    import torch

    with torch.cuda.stream(stream):
        for it in items:  # warm, outside the capture
            fn(it)
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for it in items:
            fn(it)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        g.replay()
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
    stream.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * len(items))


def kernel_roofline(dec, c, recorded, reps=3):
    """Time the path's kernels with HIP events on their own stream over the
    recorded routing of every layer and step (layers rotate, so the 256 MB
    last-level cache cannot serve repeats).  Algorithmic bytes per launch:
      gemm1   U*2I*H*2 (unique experts' w13) + T*H*2 (x) + P*I*2 (act out)
      gemm2   U*H*I*2 (w2) + P*I*2 (act in) + P*H*4 (partials out)
      combine P*H*4 + T*H*2 (out) [+ T*H*2 shared]
    where U = unique resident experts of the step, P = valid pairs."""
    import torch

    from sluice_amd import _lib

    lib = _lib.load()
    sp = dec.sp
    H, I, k = sp["H"], sp["I"], sp["k"]
    stream = torch.cuda.Stream(device=dec.dev)
    nplan = lib.sluice_moe_plan_ints(c, k)
    items = []
    with torch.cuda.stream(stream):
        for r in recorded:
            n, hn, ti, tw = r["n"], r["hn"], r["ti"], r["tw"]
            m = dec.moe_layers[n]
            plan = torch.empty(nplan, dtype=torch.int32, device=dec.dev)
            _lib.check(lib.sluice_moe_align(ti.data_ptr(), c, k, r["map"].data_ptr(),
                                            sp["E"], m.w13_weight.shape[0], plan.data_ptr(),
                                            stream.cuda_stream), "align")
            act = torch.empty((c * k, I), dtype=torch.bfloat16, device=dec.dev)
            part = torch.empty((c * k, H), dtype=torch.float32, device=dec.dev)
            out = torch.empty((c, H), dtype=torch.bfloat16, device=dec.dev)
            items.append(dict(n=n, m=m, hn=hn, ti=ti, tw=tw, plan=plan, act=act, part=part,
                              out=out))
    stream.synchronize()
    b1, b2, b3, fl = [], [], [], []
    for it in items:
        p = it["plan"].cpu().numpy()
        nb = int(p[0])
        blocks = p[4: 4 + 18 * nb].reshape(nb, 18) if nb else np.zeros((0, 18), np.int64)
        U = len(set(blocks[:, 0].tolist()))
        pairs = int(blocks[:, 1].sum()) if nb else 0
        if sp["fp8"]:  # e4m3fn bytes + fp32 128x128 block scales
            b1.append(U * (2 * I * H + (2 * I // 128) * (H // 128) * 4) + c * H * 2
                      + pairs * I * 2)
            b2.append(U * (H * I + (H // 128) * (I // 128) * 4) + pairs * I * 2 + pairs * H * 4)
        else:
            b1.append(U * 2 * I * H * 2 + c * H * 2 + pairs * I * 2)
            b2.append(U * H * I * 2 + pairs * I * 2 + pairs * H * 4)
        b3.append(c * k * H * 4 + c * H * 2)
        fl.append(2 * pairs * 2 * I * H)
    st = stream.cuda_stream

    if sp["fp8"]:
        def g1(it):
            lib.sluice_moe_gemm1_fp8(it["hn"].data_ptr(), it["m"].w13_weight.data_ptr(),
                                     it["m"].w13_weight_scale.data_ptr(), it["plan"].data_ptr(),
                                     c, H, I, k, it["act"].data_ptr(), st)

        def g2(it):
            lib.sluice_moe_gemm2_fp8(it["act"].data_ptr(), it["m"].w2_weight.data_ptr(),
                                     it["m"].w2_weight_scale.data_ptr(), it["plan"].data_ptr(),
                                     it["tw"].data_ptr(), c, H, I, k, it["part"].data_ptr(), st)
    else:
        def g1(it):
            lib.sluice_moe_gemm1_bf16(it["hn"].data_ptr(), it["m"].w13_weight.data_ptr(),
                                      it["plan"].data_ptr(), c, H, I, k, it["act"].data_ptr(), st)

        def g2(it):
            lib.sluice_moe_gemm2_bf16(it["act"].data_ptr(), it["m"].w2_weight.data_ptr(),
                                      it["plan"].data_ptr(), it["tw"].data_ptr(), c, H, I, k,
                                      it["part"].data_ptr(), st)

    def cb(it):
        lib.sluice_moe_combine(it["part"].data_ptr(), it["plan"].data_ptr(), c, k, H, 1.0, None,
                               it["out"].data_ptr(), st)

    us1 = _event_loop(stream, g1, items, reps)
    us2 = _event_loop(stream, g2, items, reps)
    us3 = _graph_loop(stream, cb, items, reps)
    # routing: the decode's router kernel on fp32 logits of the step's shape
    # (the logits' values only change which ids win, not the work)
    from sluice_amd.ops import _SCORING

    bias = dec.moe_layers[0].e_score_correction_bias
    gen = torch.Generator(device=dec.dev).manual_seed(3)
    with torch.cuda.stream(stream):
        lgs = [torch.randn((c, sp["E"]), generator=gen, device=dec.dev) for _ in range(16)]
        ids_o = torch.empty((c, k), dtype=torch.int32, device=dec.dev)
        w_o = torch.empty((c, k), dtype=torch.float32, device=dec.dev)

    def rt(lg):
        lib.sluice_route_topk(lg.data_ptr(), 0, c, sp["E"], k, _SCORING[sp["scoring"]],
                              int(sp["renorm"]), float(sp["routed_scale"]),
                              bias.data_ptr() if bias is not None else None, sp["n_group"],
                              sp["topk_group"], ids_o.data_ptr(), w_o.data_ptr(), st)

    usr = _graph_loop(stream, rt, lgs, 8)
    # a plain device copy of known size: the HBM reference for counter scaling
    nb = 256 << 20
    src = torch.empty(nb, dtype=torch.uint8, device=dec.dev)
    dst = torch.empty_like(src)
    usc = _event_loop(stream, lambda _: dst.copy_(src), [0], 4)

    def res(name, us, bts):
        avg = float(np.mean(bts))
        return {"kernel": name, "avg_us": us, "algorithmic_bytes": avg,
                "achieved_GBs": avg / (us * 1e-6) / 1e9}

    def read_probe(nbytes):
        """A plain streaming-read kernel over nbytes per launch (regions
        rotating through 4x that, like the layers above), timed the same way:
        what a kernel that only reads reaches at this launch size."""
        nbytes = max(16, int(nbytes) // 16 * 16)
        buf = torch.empty(4 * nbytes, dtype=torch.uint8, device=dec.dev)
        sink = torch.zeros(1, dtype=torch.int32, device=dec.dev)
        regions = [buf.data_ptr() + i * nbytes for i in range(4)]
        us = _event_loop(stream, lambda p: _lib.check(
            lib.sluice_read_probe(p, nbytes, sink.data_ptr(), st), "read_probe"), regions,
            max(2, reps * len(items) // 4))
        del buf
        return {"bytes": nbytes, "avg_us": us, "achieved_GBs": nbytes / (us * 1e-6) / 1e9}

    kind = "fp8" if sp["fp8"] else "bf16"
    r1 = res(f"moe_gemm1_kernel<{kind}>", us1, b1)
    r1["mfma_util_pct"] = 100.0 * float(np.mean(fl)) / (us1 * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS
    r2 = res(f"moe_gemm2_kernel<{kind}>", us2, b2)
    r2["mfma_util_pct"] = 100.0 * float(np.mean(fl)) / (us2 * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS
    for r in (r1, r2):
        rp = read_probe(r["algorithmic_bytes"])
        r["read_probe_GBs"] = rp["achieved_GBs"]
        r["frac_of_read_probe"] = r["achieved_GBs"] / rp["achieved_GBs"]
    rb = c * sp["E"] * 4 + (sp["E"] * 4 if sp["e_bias"] else 0) + c * k * 8
    return {"c": c, "launches": reps * len(items), "gemm1": r1, "gemm2": r2,
            "combine": res("moe_combine_kernel", us3, b3),
            "route": res("route_topk_kernel", usr, [rb]),
            "copy_256MiB_GBs": 2 * nb / (usc * 1e-6) / 1e9}


def measured_traffic(cfg, c, slots, uniform, algorithmic_bytes, kernel="moe_gemm1"):
    """HBM bytes per launch of `kernel` for this workload, from the committed
    summary of the two counter runs (FETCH_SIZE, WRITE_SIZE), each scaled by
    what the counter reads for a 256 MiB device copy.  None when no counter
    run covers this workload: no entry, or one measured over routing whose
    algorithmic bytes per launch differ by more than 3% from this run's."""
    path = os.path.join(ROOT, "profiles", "moe_kernels_traffic.json")
    if uniform or not os.path.exists(path):
        return None
    with open(path) as f:
        table = json.load(f)
    rec = table.get(f"{cfg}/c{c}/slots{slots}", {}).get(kernel)
    if rec is None:
        return None
    if abs(rec["algorithmic_bytes_per_launch"] / algorithmic_bytes - 1.0) > 0.03:
        return None
    return {"bytes_per_launch": rec["hbm_bytes_per_launch"],
            "ratio_to_algorithmic": rec["hbm_bytes_per_launch"]
            / rec["algorithmic_bytes_per_launch"],
            "source": f"profiles/moe_kernels_traffic.json[{cfg}/c{c}/slots{slots}][{kernel}]"}


def h2d_rates(dec):
    """Pinned host->device rates: one 64 MiB copy (the link's peak), and
    expert stream-ins laid out as the gap lays them out -- one copy per
    per-expert param per missing expert, slot rows <- host rows, each param
    on its copy lane (the largest rows first, each to the lane with fewer
    bytes so far: w13 | w2 for bf16).  The lanes here are two HIP streams,
    as on the classic wave path; the gap's own lanes are SDMA engines driven
    through HSA, whose copy windows the gap timeline measures."""
    import torch

    from sluice_amd import _lib, ops

    lib = _lib.load()
    st = ops.HostStore((64 << 20,), torch.uint8)
    d = torch.empty((64 << 20,), dtype=torch.uint8, device=dec.dev)
    lanes = [torch.cuda.Stream(device=dec.dev), torch.cuda.Stream(device=dec.dev)]
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def issue(groups):
        for lane, (D, S, B, n) in zip(lanes, groups):
            if n:
                _lib.check(lib.sluice_copy_rows(D, S, B, n, lane.cuda_stream), "copy")

    def copies(dsts, srcs, sizes, lane_of, reps):
        groups = []
        for lane in range(len(lanes)):
            idx = [i for i in range(len(dsts)) if lane_of[i] == lane]
            n = len(idx)
            groups.append(((ctypes.c_void_p * n)(*[dsts[i] for i in idx]),
                           (ctypes.c_void_p * n)(*[srcs[i] for i in idx]),
                           (ctypes.c_size_t * n)(*[sizes[i] for i in idx]), n))
        issue(groups)  # warm
        torch.cuda.synchronize()
        e0.record(lanes[0])
        lanes[1].wait_event(e0)
        for _ in range(reps):
            issue(groups)
        lanes[0].wait_stream(lanes[1])
        e1.record(lanes[0])
        torch.cuda.synchronize()
        return sum(sizes) * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9

    # medians of several short timings: a single one occasionally catches a
    # stall of a few milliseconds (seen on the box: 40-45 GB/s once in six
    # back-to-back measurements, 55 GB/s the rest)
    peak = float(np.median([copies([d.data_ptr()], [st.data_ptr()], [64 << 20], [0], 8)
                            for _ in range(3)]))
    cache = dec.caches[0]
    row = {name: cache.cpu_store[name][0].nbytes for name in cache.param_names}
    load, lane_of_param = [0, 0], {}
    for name in sorted(cache.param_names, key=lambda n: -row[n]):
        lane = 0 if load[0] <= load[1] else 1
        lane_of_param[name] = lane
        load[lane] += row[name]
    dsts, srcs, sizes, lane_of = [], [], [], []
    for e in range(8):
        slot = e % cache.num_slots
        for name in cache.param_names:
            t_slot, t_host = cache.gpu_cache[name], cache.cpu_store[name]
            rb = row[name]
            dsts.append(t_slot.data_ptr() + slot * rb)
            srcs.append(t_host.data_ptr() + e * rb)
            sizes.append(rb)
            lane_of.append(lane_of_param[name])
    torch.cuda.synchronize()
    expert = float(np.median([copies(dsts, srcs, sizes, lane_of, 3) for _ in range(5)]))
    # put the touched slots back to what the cache says they hold
    for name in cache.param_names:
        for slot, loc in enumerate(cache.expert_in_slot):
            if loc is not None and slot < 8:
                cache.gpu_cache[name][slot].copy_(cache.cpu_store[name][loc])
    torch.cuda.synchronize()
    return {"peak_pinned_GBs": peak, "expert_stream_GBs": expert,
            "expert_stream_frac_of_peak": expert / peak,
            "bytes_per_expert": cache.bytes_per_expert}


def cpu_baseline(budget_s, n_moe_layers):
    """The reference's per-layer decode path in torch fp32 on the host cores
    (oracle/cpu_path.py): one DeepSeek-V2-Lite-shaped MoE layer, T=8 tokens
    per step, 64 timed steps (fewer if the budget runs out) after 4 untimed;
    per-stage medians; tok/s = 8 / (MoE layers x the median layer step)."""
    from oracle import cpu_path

    r = cpu_path.run(T=8, steps=64, warmup=4, budget_s=budget_s)
    step = r["step_median_s"]
    return {
        "value": r["tokens_per_step"] / (n_moe_layers * step), "unit": "tok/s",
        "cores": r["threads"], "kind": "port",
        "sample": (f"the path in torch fp32 on one DeepSeek-V2-Lite-shaped MoE layer (64 experts "
                   f"top-6 + 2 shared, 48 slots, weights N(0,0.02), Zipf(1.1) router bias): "
                   f"routing, gap bookkeeping, host row copies, expert product, combine; T=8, "
                   f"{r['steps']} timed steps; tok/s = 8 / ({n_moe_layers} MoE layers x "
                   f"{step * 1e3:.2f} ms median layer step); attention and LM head not counted"),
        "stages_median_us": r["stages_us"], "stages_mean_us": r["stages_mean_us"],
        "layer_step_ms": step * 1e3, "torch_threads": r["threads"],
        "affinity_cores": r["affinity"], "misses": r["misses"], "steps": r["steps"],
    }


def _every(n, fn):
    """A progress callback passing on every n-th message."""
    count = [0]

    def cb(msg):
        count[0] += 1
        if count[0] % n == 0:
            fn(msg)

    return cb


def build_decoder(cfg, slots, max_batch, a, dev, gen_len, uniform=False, stores=None):
    from sluice_amd.decoder import SyntheticDecoder

    t = time.perf_counter()
    dec = SyntheticDecoder(cfg, max_batch=max_batch, slots=slots, prompt_len=PROMPT_LEN,
                           gen_len=gen_len, uniform_routing=uniform, layers=a.layers, device=dev,
                           host_pool=a.host_pool, stores=stores, zipf_s=ROUTING["zipf_s"],
                           rho=ROUTING["rho"], sigma=a.sigma, gate_std=ROUTING["gate_std"],
                           progress=_every(8, log))
    build_s = time.perf_counter() - t
    log(f"built {cfg} decoder in {build_s:.1f}s ({len(dec.moe_layers)} MoE layers, slots={slots}, "
        f"host stores {dec.host_pool}, {dec.host_store_bytes / 2**30:.1f} GiB per layer)")
    return dec, build_s


def measure(cfg, slots, batches, a, dev, gen_len, uniform=False, stores=None, locality=(),
            prefill=True, h2d=False, reference=(), matched=(), steps=None):
    """One configuration: its batches, the routing it ran, the kernels'
    roofline at the largest batch, optional rows in the reference's
    orchestration (same routing) and locality rows; returns the result and
    the decoder's host stores (for reuse by the same shape)."""
    import gc

    import torch

    steps = steps or a.steps
    dec, build_s = build_decoder(cfg, slots, max(batches), a, dev, gen_len, uniform, stores)
    rows = []
    for c in batches:
        r = run_batch(dec, c, steps, a.warmup, prefill=prefill and not uniform,
                      label="uniform" if uniform else "zipf")
        log(f"{cfg} s{slots} c={c} ({r['path']}, {r['routing']}): {r['ms_per_step']:.3f} ms/step "
            f"{r['tok_per_s']:.1f} tok/s misses/layer-step={r['misses_per_layer_step']:.3f} "
            f"fast-hit={r['fast_hit_share']:.2%} H2D {r['h2d_GBs_in_step']:.1f} GB/s "
            f"staged={r['staged']['hit_share_of_misses']:.1%} of misses "
            f"steps min/med/max {'/'.join(f'{v:.2f}' for v in r['step_ms_min_median_max'])} ms")
        rows.append(r)
    c_main = max(batches)
    recorded = record_routing(dec, c_main, 8)
    if a.save_routing and cfg == a.config:
        save_routing(a.save_routing, recorded)
    rstats = routing_stats(dec, recorded)
    roof = kernel_roofline(dec, c_main, recorded)
    rates = h2d_rates(dec) if h2d else None
    if reference:
        # The same batches and routing with the reference's orchestration:
        # each MoE layer's gap runs eagerly between captured pieces, the host
        # waiting for its ids, and a gap with misses answers only after its
        # rows landed (the expert product does not overlap the copies).
        dec.set_gap_mode(server=False, pipelined=False)
        for c in reference:
            r = run_batch(dec, c, steps, a.warmup, prefill=prefill and not uniform,
                          label="uniform" if uniform else "zipf")
            r["orchestration"] = ORCH_REFERENCE
            log(f"{cfg} s{slots} c={c} (reference orchestration): {r['ms_per_step']:.3f} ms/step "
                f"{r['tok_per_s']:.1f} tok/s misses/layer-step={r['misses_per_layer_step']:.3f} "
                f"fast-hit={r['fast_hit_share']:.2%} H2D {r['h2d_GBs_in_step']:.1f} GB/s")
            rows.append(r)
        dec.set_gap_mode(server=True, pipelined=True)
    for c, sigma in matched:
        for rb in dec.bias_tables:
            rb.refill(ROUTING["zipf_s"], ROUTING["rho"], sigma, rb.knobs["seed"])
        r = run_batch(dec, c, steps, a.warmup, prefill=prefill, label="matched")
        r["sigma"] = sigma
        log(f"{cfg} s{slots} c={c} (fast-hit matched, sigma={sigma}): {r['ms_per_step']:.3f} "
            f"ms/step {r['tok_per_s']:.1f} tok/s misses/layer-step="
            f"{r['misses_per_layer_step']:.3f} fast-hit={r['fast_hit_share']:.2%}")
        rows.append(r)
    for c in locality:
        for rb in dec.bias_tables:
            rb.refill(ROUTING["zipf_s"], ROUTING["rho"], LOCALITY_SIGMA, rb.knobs["seed"])
        r = run_batch(dec, c, steps, a.warmup, prefill=prefill, label="locality")
        r["sigma"] = LOCALITY_SIGMA
        log(f"{cfg} s{slots} c={c} (locality sigma={LOCALITY_SIGMA}): {r['ms_per_step']:.3f} "
            f"ms/step {r['tok_per_s']:.1f} tok/s misses/layer-step="
            f"{r['misses_per_layer_step']:.3f} fast-hit={r['fast_hit_share']:.2%}")
        rows.append(r)
    sp = dec.sp
    g1 = roof["gemm1"]
    out = {
        "config": {"model_shape": cfg, "moe_layers": len(dec.moe_layers), "experts": sp["E"],
                   "top_k": sp["k"], "slots": slots, "max_bt": dec.thr,
                   "dtype": "f8e4m3/bf16" if sp["fp8"] else "bf16",
                   "routing": dict(dec.routing_knobs, **rstats),
                   "host_pool": dec.host_pool, "host_pool_note": dec.host_pool_note,
                   "host_store_GiB": dec.host_store_bytes * len({id(st) for st in dec.stores})
                   / 2**30,
                   "build_s": build_s},
        "per_batch": rows,
        "gemm1": {"c": c_main, "avg_us": g1["avg_us"], "achieved_GBs": g1["achieved_GBs"],
                  "frac": g1["achieved_GBs"] / HBM_PEAK_GBS,
                  "algorithmic_bytes_per_launch": g1["algorithmic_bytes"],
                  "mfma_util_pct": g1["mfma_util_pct"],
                  "read_probe_GBs": g1["read_probe_GBs"],
                  "frac_of_read_probe": g1["frac_of_read_probe"]},
        "kernels": {kk: roof[kk] for kk in ("gemm2", "combine", "route")},
        "copy_256MiB_GBs": roof["copy_256MiB_GBs"],
    }
    if rates:
        out["h2d"] = rates
    stores = dec.stores
    dec.close()
    del dec, recorded
    gc.collect()
    torch.cuda.empty_cache()
    return out, stores


def vs_published(rows):
    """Rows (model shape, slots, row) that have a published reference
    figure, each with its ratio to it; None when none has."""
    out = []
    for cfg, slots, r in rows:
        pub = PUBLISHED.get(cfg)
        ref = (pub or {}).get("tok_per_s", {}).get(slots, {}).get(r["c"])
        if ref is None or r["path"] != "gap" or r["orchestration"] != ORCH_GRAPH:
            continue
        out.append({"model_shape": cfg, "slots": slots, "c": r["c"], "routing": r["routing"],
                    "sigma": r.get("sigma"), "tok_per_s": r["tok_per_s"],
                    "reference_tok_per_s": ref, "ratio": r["tok_per_s"] / ref,
                    "fast_hit_share": r["fast_hit_share"],
                    "reference_fast_hit_share": pub["fast_hit_share"]})
    return out or None


def _release():
    """Free host stores and device memory no longer referenced."""
    import gc

    import torch

    gc.collect()
    torch.cuda.empty_cache()


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported on this path "
              "(every box has one GPU and the expert-parallel sharding is design-only).",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from sluice_amd.decoder import SPECS

    cfg = a.config
    sp = SPECS[cfg]
    slots = a.slots or DEFAULT_SLOTS[cfg]
    batches = [int(v) for v in a.batches.split(",")] if a.batches else (
        [1, 8] if cfg == "v2lite" else [1, 8, 12] if cfg == "qwen3" else [8])
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen_len = max(DECODE_LEN, a.warmup + a.steps + 8)
    if a.roofline_only:
        # no decode step runs here: a counter-collecting profiler serialises
        # dispatches, which the gap's device/host hand-off cannot run under
        if not a.load_routing:
            sys.exit("--roofline-only needs --load-routing (written by --save-routing)")
        a.host_pool = "shared"  # the kernels read the slots only; their contents do not matter
        dec, _ = build_decoder(cfg, slots, max(batches), a, dev, gen_len, a.uniform)
        recorded = load_routing(a.load_routing, dev)
        c = int(recorded[0]["ti"].shape[0])
        roof = kernel_roofline(dec, c, recorded)
        print(json.dumps({"config": cfg, "c": c, "roofline": roof}), flush=True)
        dec.close()
        return
    locality = () if (a.no_locality or a.uniform) else tuple(batches)
    reference = () if (a.no_reference or a.uniform) else tuple(batches)
    matched = () if (a.no_locality or a.uniform or slots != DEFAULT_SLOTS[cfg]) else tuple(
        (c, sg) for c, sg in MATCHED_SIGMA.get(cfg, {}).items() if c in batches)
    head, stores = measure(cfg, slots, batches, a, dev, gen_len, uniform=a.uniform,
                           locality=locality, prefill=not a.no_prefill, h2d=True,
                           reference=reference, matched=matched)
    del stores
    _release()
    extras = []
    if not a.no_extras and cfg == "v2lite" and not (a.uniform or a.slots or a.batches
                                                    or a.layers):
        q64, qstores = measure("qwen3", 64, [1, 8], a, dev, gen_len,
                               locality=() if a.no_locality else (8,))
        extras.append(q64)
        q96 = measure("qwen3", 96, [1, 8, 12], a, dev, gen_len, stores=qstores,
                      locality=() if a.no_locality else (12,))[0]
        extras.append(q96)
        # c=12 at 64 slots is above the router-split envelope (12 * 8 > 64): the
        # classic wave path serves it (the reference's router-split has no number)
        q64c = measure("qwen3", 64, [12], a, dev, gen_len, stores=qstores, locality=())[0]
        q64c["config"]["workload"] = "classic wave path: c=12 above the router-split envelope"
        extras.append(q64c)
        stress = measure("qwen3", 32, [4], a, dev, max(gen_len, a.stress_steps + a.warmup + 8),
                         uniform=True, stores=qstores, steps=a.stress_steps)[0]
        stress["config"]["workload"] = (
            f"stress: uniform i.i.d. top-8, no prompt (no locality), {a.stress_steps} timed steps "
            f"after {a.warmup} warm-up steps (the configured run is 512 steps)")
        extras.append(stress)
        del qstores
        _release()
        v3 = measure("v3", 64, [8], a, dev, gen_len)[0]
        extras.append(v3)
    n_moe = sp["layers"] - sp["first_dense"] if a.layers is None else a.layers - min(
        a.layers, sp["first_dense"])
    cpu = None
    if not a.no_cpu_baseline:
        cpu = cpu_baseline(a.cpu_budget_s, n_moe)
        log(f"cpu baseline {cpu['value']:.2f} tok/s, layer step {cpu['layer_step_ms']:.2f} ms, "
            f"stages {cpu['stages_median_us']}")
    record = full_record(a, cfg, sp, slots, batches, gen_len, head, extras, cpu)
    record["record_file"] = os.path.abspath(a.record) if a.record else None
    text = json.dumps(record)
    if a.record:
        with open(a.record, "w") as f:
            f.write(text + "\n")
    # the whole record on stderr, then the headline object as the last stdout line
    log(f"full record: {text}")
    print(json.dumps(compact_line(record), separators=(",", ":"), allow_nan=False), flush=True)


def full_record(a, cfg, sp, slots, batches, gen_len, head, extras, cpu):
    """Everything measured in the run: the headline fields, every batch row
    of every configuration, the kernels' timings, the H2D rates, the CPU
    baseline and the rows with a published reference figure."""
    main_c = max(batches)
    main_row = [r for r in head["per_batch"] if r["c"] == main_c and r["routing"] != "locality"
                and r["orchestration"] == ORCH_GRAPH][0]
    ref_rows = {r["c"]: r for r in head["per_batch"] if r["orchestration"] == ORCH_REFERENCE}
    pub = PUBLISHED_C8.get(cfg) if main_c == 8 and not a.uniform and slots == DEFAULT_SLOTS[cfg] \
        else None
    hc = head["config"]
    line = {
        "metric": "moe_decode_tok_per_s",
        "value": main_row["tok_per_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": main_row["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (main_row["tok_per_s"] / pub) if pub else None,
        "dtype": "f8e4m3/bf16" if sp["fp8"] else "bf16",
        "data": ("synthetic (random-init weights, seeded 128-token prompts processed before "
                 "timing, Zipf(1.1) + AR(1) rho=0.7 routing logits)") if not a.uniform else
                "synthetic (random-init weights, uniform i.i.d. routing)",
        "config": dict(hc, workload=(
            f"{cfg}-shaped decode, {hc['moe_layers']} MoE layers, slots={slots}/{sp['E']}, "
            f"MAX_BT={hc['max_bt']}, c={main_c}, 128-token prompts then decode positions "
            f"{main_row['timed_positions']} of a {gen_len}-token decode"
            + (" (classic wave path)" if main_row["path"] == "classic" else "")),
            batch=main_c, prompt_len=PROMPT_LEN, decode_len=gen_len,
            baseline_ref="reference router-split on 1xH100 with real-model routing (c=8)"
            if pub else None),
        "per_batch": head["per_batch"],
        # this build's kernels in the reference's orchestration, same box,
        # workload and routing: what the pipelined one-graph gap adds
        "vs_reference_orchestration": {
            c: {"ms_per_step": r["ms_per_step"], "tok_per_s": r["tok_per_s"],
                "speedup": next(g["tok_per_s"] for g in head["per_batch"]
                                if g["c"] == c and g["routing"] == r["routing"]
                                and g["orchestration"] == ORCH_GRAPH) / r["tok_per_s"]}
            for c, r in ref_rows.items()} or None,
        # every measured row with a published reference figure (same model
        # shape, slots and batch), with both fast-hit shares: where they
        # match, the routing is like for like
        "vs_published": vs_published(
            [(cfg, slots, r) for r in head["per_batch"]]
            + [(e["config"]["model_shape"], e["config"]["slots"], r) for e in extras
               for r in e["per_batch"]]),
        "roofline": None,
        "kernels": dict(head["kernels"], copy_256MiB_GBs=head["copy_256MiB_GBs"]),
        "h2d": head.get("h2d"),
        "cpu_baseline": cpu,
        "extras": extras,
    }
    g1 = head["gemm1"]
    traffic = measured_traffic(cfg, main_c, slots, a.uniform, g1["algorithmic_bytes_per_launch"])
    line["roofline"] = {
        "bound": "hbm", "achieved": g1["achieved_GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": g1["frac"],
        "traffic": traffic["bytes_per_launch"] if traffic else None,
        "traffic_source": traffic["source"] if traffic else None,
        "kernel": "moe_gemm1_kernel<fp8>" if sp["fp8"] else "moe_gemm1_kernel<bf16>",
        "avg_us": g1["avg_us"], "algorithmic_bytes_per_launch": g1["algorithmic_bytes_per_launch"],
        "mfma_util_pct": g1["mfma_util_pct"],
        # a plain streaming-read kernel timed the same way at the same bytes
        # per launch: the HBM rate a kernel that only reads reaches there
        "read_probe_GBs": g1["read_probe_GBs"], "frac_of_read_probe": g1["frac_of_read_probe"],
    }
    line["gemm1"] = head["gemm1"]
    return line


# columns of the compact line's batch rows
ROW_COLS = ["shape", "slots", "c", "path", "routing", "steps", "ms_per_step", "tok_per_s",
            "misses_per_layer_step", "fast_hit_share", "staged_share_of_misses",
            "coded_layers", "h2d_GBs_in_step", "ref_tok_per_s"]
LINE_LIMIT = 6000  # bytes; the last stdout line must stay whole in a short tail


def _r(v, nd):
    """v rounded to nd digits; None for a missing or non-finite value (the
    line stays strict JSON)."""
    if v is None or not np.isfinite(float(v)):
        return None
    return round(float(v), nd)


def compact_line(rec):
    """The headline object: the contract's fields, the roofline and CPU
    baseline, the H2D rates and one short row per measured batch of every
    configuration (columns ROW_COLS; path "gap", "classic" or "gap/ref-orch"
    for this build's kernels in the reference's orchestration;
    ref_tok_per_s is the reference's published figure for that shape, slots
    and batch, or null).  The full record is in rec["record_file"]."""
    c = rec["config"]
    rows, g1, g2 = [], {}, {}
    configs = [(c["model_shape"], c["slots"], rec["per_batch"], rec.get("gemm1"),
                rec.get("kernels", {}).get("gemm2"))]
    configs += [(e["config"]["model_shape"], e["config"]["slots"], e["per_batch"], e.get("gemm1"),
                 e.get("kernels", {}).get("gemm2")) for e in rec.get("extras") or []]
    for shape, slots, per_batch, k1, k2 in configs:
        for r in per_batch:
            path = r["path"] + ("/ref-orch" if r["orchestration"] == ORCH_REFERENCE else "")
            ref = None
            if r["path"] == "gap" and r["orchestration"] == ORCH_GRAPH:
                ref = PUBLISHED.get(shape, {}).get("tok_per_s", {}).get(slots, {}).get(r["c"])
            routing = r["routing"] + (f"/s{r['sigma']}" if r.get("sigma") is not None else "")
            rows.append([shape, slots, r["c"], path, routing, r.get("steps", rec["steps"]),
                         _r(r["ms_per_step"], 3),
                         _r(r["tok_per_s"], 1), _r(r["misses_per_layer_step"], 3),
                         _r(r["fast_hit_share"], 3),
                         _r((r.get("staged") or {}).get("hit_share_of_misses"), 3),
                         ((r.get("coded") or {}).get("layers")
                          if (r.get("coded") or {}).get("decodes") else 0),
                         _r(r["h2d_GBs_in_step"], 1), ref])
        if k1:
            key = f"{shape}/s{slots}/c{k1['c']}"
            g1[key] = _r(k1.get("frac", k1["achieved_GBs"] / HBM_PEAK_GBS), 3)
            if k2:
                g2[key] = _r(k2["achieved_GBs"] / HBM_PEAK_GBS, 3)
    roof = rec["roofline"]
    cpu = rec.get("cpu_baseline")
    h2d = rec.get("h2d")
    head_rows = [r for r in rec["per_batch"] if r["c"] == c["batch"]
                 and r["orchestration"] == ORCH_GRAPH and r["routing"] not in ("locality",
                                                                              "matched")]
    in_step = head_rows[0]["h2d_GBs_in_step"] if head_rows else None
    staging = (head_rows[0].get("staged") or {}).get("rows_per_layer") if head_rows else None
    coded = (head_rows[0].get("coded") or {}) if head_rows else {}
    line = {
        "metric": rec["metric"], "value": _r(rec["value"], 2), "unit": rec["unit"],
        "n_gpus": rec["n_gpus"], "steps": rec["steps"], "warmup": rec["warmup"],
        "ms_per_step": _r(rec["ms_per_step"], 4), "higher_is_better": rec["higher_is_better"],
        "scaling": rec["scaling"], "vs_baseline": _r(rec["vs_baseline"], 4),
        "dtype": rec["dtype"], "data": rec["data"],
        "config": {"workload": c["workload"], "model_shape": c["model_shape"],
                   "moe_layers": c["moe_layers"], "experts": c["experts"], "top_k": c["top_k"],
                   "slots": c["slots"], "max_bt": c["max_bt"], "batch": c["batch"],
                   "prompt_len": c["prompt_len"], "decode_len": c["decode_len"],
                   "routing": {k: c["routing"][k] for k in ("zipf_s", "rho", "sigma", "gate_std")
                               if k in c["routing"]},
                   "baseline_ref": c.get("baseline_ref"),
                   "staging_rows_per_layer": staging,
                   "coded_store": {"layers": coded.get("layers"), "of_layers": coded.get("of_layers"),
                                   "bytes_frac": _r(coded.get("store_ratio"), 4)}
                   if coded else None},
        "roofline": {"bound": roof["bound"], "achieved": _r(roof["achieved"], 1),
                     "peak": roof["peak"], "unit": roof["unit"], "frac": _r(roof["frac"], 4),
                     "traffic": roof["traffic"], "kernel": roof["kernel"],
                     "avg_us": _r(roof["avg_us"], 2),
                     "algorithmic_bytes_per_launch": _r(roof["algorithmic_bytes_per_launch"], 0),
                     "read_probe_GBs": _r(roof["read_probe_GBs"], 1),
                     "frac_of_read_probe": _r(roof["frac_of_read_probe"], 3),
                     "mfma_util_pct": _r(roof["mfma_util_pct"], 3),
                     "traffic_source": roof.get("traffic_source")},
        "cpu_baseline": None if cpu is None else {
            "value": _r(cpu["value"], 2), "unit": cpu["unit"], "cores": cpu["cores"],
            "kind": cpu["kind"], "sample": cpu["sample"],
            "layer_step_ms": _r(cpu["layer_step_ms"], 2),
            "stages_median_us": {k: _r(v, 1) for k, v in cpu["stages_median_us"].items()}},
        "h2d": None if h2d is None else {
            "peak_pinned_GBs": _r(h2d["peak_pinned_GBs"], 1),
            "expert_stream_GBs": _r(h2d["expert_stream_GBs"], 1),
            "in_step_GBs": _r(in_step, 1),
            "in_step_frac_of_peak": _r(in_step / h2d["peak_pinned_GBs"], 3)
            if in_step is not None else None},
        "gemm1_frac_of_8TBs": g1, "gemm2_frac_of_8TBs": g2,
        "row_cols": ROW_COLS, "rows": rows,
        "record_file": rec.get("record_file"),
    }
    return line


if __name__ == "__main__":
    main()
