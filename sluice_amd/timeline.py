"""Gap timeline of a decode: where the host link idles, without a profiler.

    python -m sluice_amd.timeline [--config v2lite] [--slots 48] [--batch 8]
                                  [--steps 20] [--warmup 5] [--json OUT]

Runs the benchmark's synthetic decode (the same model shape, routing and
window: 128-token prompts, then the timed steps centred in a 256-token decode)
on the gap-timeline build of the library (libsluice_hip_trace.so, built by
``python -m sluice_amd.build --trace``; this module sets SLUICE_TRACE=1 before
the library loads).  The gap kernel, the expert product and the combine stamp
events with the device wall clock and the host gap service with its own
clock; two calibrations (before and after the timed steps) put both on one
timebase.  Reported per MoE layer-step with stream-ins (medians, p10, p90,
microseconds from the gap kernel's start):

  head   record posted, record seen by the host, bookkeeping done, first row
         copy issued, device answered, answer read by the device, gap end;
  copy   first copy issued -> last group seen landed, and its rate;
  tail   after the last group was seen landed: slots marked ready, ready
         seen by the device, the pending gemm1 items' slot waits ending (first,
         last) and the items done (first, last), the pending gemm2 items'
         gemm1 counts reached (first, last) and the last done, combine
         started, next layer's gap started;

the duration of each pending item of the expert product (a gemm1 item from
its slot wait to done, a gemm2 item from its gemm1 count to done), and the
link-idle time per step between copy windows, split into the transitions
between consecutive layers with stream-ins and the stretches that cover
layers without any.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from collections import Counter

import numpy as np

RATE_HZ = 1e8  # the device wall clock (hipDeviceAttributeWallClockRate on MI355X)
TAG_SHIFT = np.uint64(56)
M48 = (1 << 48) - 1


class _HostRec(ctypes.Structure):
    _fields_ = [("tag", ctypes.c_uint32), ("layer", ctypes.c_uint32), ("stamp", ctypes.c_int32),
                ("value", ctypes.c_int32), ("t", ctypes.c_double)]


RING_DEV = 1 << 20   # device records per ring
RING_HOST = 1 << 18


def _lib():
    if os.environ.get("SLUICE_TRACE") != "1":
        if "sluice_amd._lib" in sys.modules:
            raise RuntimeError("the default library is already loaded; run the timeline in a "
                               "process of its own")
        os.environ["SLUICE_TRACE"] = "1"
    from sluice_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        raise RuntimeError(f"{_lib.LIB_PATH} is missing: python -m sluice_amd.build --trace")
    return _lib.load()


def calibrate(lib, n=300):
    hs = (ctypes.c_double * n)()
    dt = (ctypes.c_ulonglong * n)()
    got = lib.sluice_trace_calibrate(n, hs, dt)
    if got <= 0:
        raise RuntimeError(f"sluice_trace_calibrate returned {got}")
    h = np.array(hs[:got])
    d = np.array(dt[:got], dtype=np.float64)
    ok = h > 0
    return h[ok], d[ok]


def read_rings(lib):
    out = {}
    n = ctypes.c_uint()
    buf = (ctypes.c_ulonglong * (2 * RING_DEV))()
    for which, name in ((0, "gap"), (1, "moe")):
        rc = lib.sluice_trace_read(which, buf, ctypes.byref(n))
        if rc != 0:
            raise RuntimeError(f"sluice_trace_read({which}) = {rc}")
        if n.value > RING_DEV:
            raise RuntimeError(f"trace ring {name} overflowed ({n.value} records)")
        out[name] = np.frombuffer(buf, dtype=np.uint64).reshape(RING_DEV, 2)[: n.value].copy()
    hb = (_HostRec * RING_HOST)()
    rc = lib.sluice_trace_read(2, hb, ctypes.byref(n))
    if rc != 0 or n.value > RING_HOST:
        raise RuntimeError(f"host trace ring: rc {rc}, {n.value} records")
    out["host"] = [(r.tag, r.layer, r.stamp, r.value, r.t) for r in hb[: n.value]]
    return out


class Clock:
    """Device wall-clock ticks -> host seconds: the offset of each
    calibration is its smallest (host - device) difference; between the two
    it is interpolated linearly in device time (the clocks drift ~1e-4)."""

    def __init__(self, cal0, cal1):
        (h0, d0), (h1, d1) = cal0, cal1
        i0, i1 = np.argmin(h0 - d0 / RATE_HZ), np.argmin(h1 - d1 / RATE_HZ)
        self.d0, self.d1 = d0[i0], d1[i1]
        self.o0, self.o1 = h0[i0] - d0[i0] / RATE_HZ, h1[i1] - d1[i1] / RATE_HZ

    def __call__(self, ticks):
        t = (np.asarray(ticks, dtype=np.uint64) & np.uint64(M48)).astype(np.float64)
        f = (t - self.d0) / (self.d1 - self.d0)
        return t / RATE_HZ + self.o0 + f * (self.o1 - self.o0)


def analyse(rings, clock, layer_ids, steps, bytes_per_expert):
    """Per-gap rows and the summary the module prints (bytes_per_expert: the
    bytes one streamed expert moves over the link)."""
    lay = {int(v): i for i, v in enumerate(layer_ids)}
    gap = rings["gap"]
    tag = (gap[:, 0] >> TAG_SHIFT).astype(int)
    val = gap[:, 0] & np.uint64((1 << 56) - 1)
    lid = (val >> np.uint64(24)).astype(np.int64)
    stp = (val & np.uint64(0xffffff)).astype(np.int64)
    tg = clock(gap[:, 1])
    G = {}
    for a, l, s, t in zip(tag, lid, stp, tg):
        G.setdefault((lay.get(int(l), -1), int(s)), {})[int(a)] = t
    H = {}
    stage_open, stage_iv = {}, []  # staging chunks: issue time per (layer, lane), intervals
    for a, l, s, v, t in rings["host"]:
        if a in (28, 29):
            q = stage_open.setdefault((int(l), int(v) & 1), [])
            if a == 28:
                q.append(t)
            elif q:
                stage_iv.append((q.pop(0), t, (int(v) >> 1) * 1024))
            continue
        k = (lay.get(int(l), -1), int(s) & 0xffffff)
        d = H.setdefault(k, {"groups": [], "marks": []})
        if a == 26:
            d["groups"].append((int(v), t))
        elif a == 27:
            d["marks"].append(t)
        else:
            d[int(a)] = t
            d[("v", int(a))] = int(v)
    moe = rings["moe"]
    mt = clock(moe[:, 1])
    mtag = (moe[:, 0] >> TAG_SHIFT).astype(int)
    mval = (moe[:, 0] & np.uint64((1 << 56) - 1)).astype(np.int64)
    order = np.argsort(mt)
    mt, mtag, mval = mt[order], mtag[order], mval[order]
    # each pending item's own duration: its two stamps paired by ticket within
    # one split launch (tag 11 opens a launch)
    item_g1, item_g2, open_ = [], [], {}
    for t_, a, v in zip(mt, mtag, mval):
        if a == 11:
            open_ = {}
        elif a in (14, 17):
            open_[(a, int(v))] = t_
        elif a == 15 and (14, int(v)) in open_:
            item_g1.append(t_ - open_.pop((14, int(v))))
        elif a == 16 and (17, int(v)) in open_:
            item_g2.append(t_ - open_.pop((17, int(v))))
    gaps = sorted((v[1], k) for k, v in G.items() if 1 in v)
    starts = np.array([g[0] for g in gaps] + [np.inf])
    rows = []
    for i, (t0, k) in enumerate(gaps):
        g, h = G[k], H.get(k, {"groups": [], "marks": []})
        lo, hi = np.searchsorted(mt, t0), np.searchsorted(mt, starts[i + 1])
        seg_t, seg_tag = mt[lo:hi], mtag[lo:hi]

        def last(x):
            sel = seg_t[seg_tag == x]
            return sel.max() if len(sel) else np.nan

        r = {"layer": k[0], "stamp": k[1], "t0": t0, "streams": h.get(("v", 22), 0),
             "next": starts[i + 1] - t0, "posted": g.get(2, np.nan) - t0,
             "gap_end": g.get(4, np.nan) - t0, "answer_read": g.get(3, np.nan) - t0}
        for key, tg_ in (("seen", 21), ("booked", 22), ("first_copy", 23), ("answered", 24),
                         ("issued", 25)):
            r[key] = h.get(tg_, np.nan) - t0
        r["staged"] = h.get(("v", 23), len(h["groups"]))
        r["landed"] = max(t for _, t in h["groups"]) - t0 if h["groups"] else np.nan
        host = [t for j, t in h["groups"] if j >= r["staged"]]
        r["landed_host"] = max(host) - t0 if host else np.nan
        r["marked"] = max(h["marks"]) - t0 if h["marks"] else np.nan
        def first(x):
            sel = seg_t[seg_tag == x]
            return sel.min() if len(sel) else np.nan

        for key, x in (("ready_seen", 10), ("g1_done", 15), ("g2_done", 16), ("combine", 13),
                       ("g1_started_last", 14), ("g2_counted_last", 17)):
            r[key] = last(x) - t0
        for key, x in (("g1_started_first", 14), ("g1_done_first", 15),
                       ("g2_counted_first", 17)):
            r[key] = first(x) - t0
        rows.append(r)

    def stat(vals):
        v = np.asarray([x for x in vals if np.isfinite(x)]) * 1e6
        if not len(v):
            return None
        return {"median_us": round(float(np.median(v)), 2), "p10_us": round(float(
            np.percentile(v, 10)), 2), "p90_us": round(float(np.percentile(v, 90)), 2),
            "n": int(len(v))}

    miss = [r for r in rows if r["streams"] > 0 and np.isfinite(r["landed"])]
    link = [r for r in miss if np.isfinite(r["first_copy"]) and np.isfinite(r["landed_host"])]
    hit = [r for r in rows if r["streams"] == 0]
    out = {"layer_steps": len(rows), "with_stream_ins": len(miss), "without": len(hit),
           "head": {k: stat(r[k] for r in miss) for k in (
               "posted", "seen", "booked", "first_copy", "answered", "answer_read", "gap_end")},
           "tail_after_landed": {k: stat(r[k] - r["landed"] for r in miss) for k in (
               "marked", "ready_seen", "g1_started_first", "g1_started_last", "g1_done_first",
               "g1_done", "g2_counted_first", "g2_counted_last", "g2_done", "combine", "next")},
           "without_stream_ins": {k: stat(r[k] for r in hit) for k in ("posted", "gap_end",
                                                                         "next")},
           "pending_item": {"gemm1_wait_end_to_done": stat(item_g1),
                            "gemm2_count_to_done": stat(item_g2)}}
    win = [(r["landed_host"] - r["first_copy"], r["streams"] - r["staged"]) for r in link]
    out["copy_window"] = {
        "rate_GBs_median": round(float(np.median([n * bytes_per_expert / w / 1e9
                                                  for w, n in win])), 2),
        "by_experts": {int(n): {"count": int(sum(1 for _, m in win if m == n)),
                                "window_us_median": round(float(np.median(
                                    [w for w, m in win if m == n])) * 1e6, 1)}
                       for n in sorted({n for _, n in win})}}
    # link idle between consecutive copy windows over the link, in stream order
    seq = sorted(rows, key=lambda r: r["t0"])
    idle_tr, idle_skip, last_end, skipped = 0.0, 0.0, None, 0
    for r in seq:
        if r in link:
            if last_end is not None:
                gap_s = r["t0"] + r["first_copy"] - last_end
                if skipped:
                    idle_skip += gap_s
                else:
                    idle_tr += gap_s
            last_end, skipped = r["t0"] + r["landed_host"], 0
        else:
            skipped += 1
    out["gap_copies_idle_ms_per_step"] = {
        "between_consecutive_layers_with_copies_over_the_link": round(idle_tr / steps * 1e3, 3),
        "across_layers_without_them": round(idle_skip / steps * 1e3, 3)}
    # the link's busy time: the gaps' copy windows and the staging chunks
    if seq:
        iv = [(r["t0"] + r["first_copy"], r["t0"] + r["landed_host"]) for r in link]
        iv += [(a, b) for a, b, _ in stage_iv]
        lo = seq[0]["t0"]
        hi = max([r["t0"] + (r["next"] if np.isfinite(r["next"]) else 0.0) for r in seq]
                 + [b for _, b in iv])
        busy, end = 0.0, lo
        for a, b in sorted(iv):
            a, b = max(a, end), min(b, hi)
            if b > a:
                busy += b - a
                end = b
        span = hi - lo
        in_win = [x for x in stage_iv if lo <= x[0] < hi]
        out["link"] = {
            "busy_share": round(busy / span, 4) if span > 0 else None,
            "idle_ms_per_step": round((span - busy) / steps * 1e3, 3),
            "staging_chunks_per_step": round(len(in_win) / steps, 2),
            "staging_MB_per_step": round(sum(x[2] for x in in_win) / steps / 1e6, 2),
            "staging_chunk_us_median": round(float(np.median([b - a for a, b, _ in in_win]))
                                             * 1e6, 1) if in_win else None,
            "gaps_with_staged_misses": sum(1 for r in miss if r["staged"] > 0),
            "gaps_all_staged": sum(1 for r in miss if r["staged"] >= r["streams"]),
            "gaps_by_misses_staged_and_over_the_link": {
                f"{a}+{b}": n for (a, b), n in sorted(Counter(
                    (min(r["staged"], r["streams"]), max(r["streams"] - r["staged"], 0))
                    for r in miss).items())}}
    return out, rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="v2lite")
    ap.add_argument("--slots", type=int, default=48)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--json", default=None, help="also write the summary here")
    a = ap.parse_args()
    lib = _lib()
    import torch

    from sluice_amd.decoder import SyntheticDecoder

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    dec = SyntheticDecoder(a.config, max_batch=a.batch, slots=a.slots, prompt_len=128,
                           gen_len=256, device=dev, host_pool="auto")
    try:
        c = a.batch
        dec.capture(c)
        dec.prefill(c)
        dec.sync()
        for _ in range(max(0, (256 - a.steps) // 2 - a.warmup) + a.warmup):
            dec.step_graphs(c)
        dec.sync()
        cal0 = calibrate(lib)
        if lib.sluice_trace_reset() != 0:
            raise RuntimeError("sluice_trace_reset")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            dec.step_graphs(c)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        dec.sync()
        cal1 = calibrate(lib)
        rings = read_rings(lib)
        ids = [(m._expert_map.data_ptr() >> 8) & 0xffffffff for m in dec.moe_layers]
        per_expert = sum(t.nbytes // t.shape[0] for t in dec.caches[0].cpu_store.values())
        # bytes of an expert over the link: its coded rows in layers whose
        # host store is coded (the mean over the layers, as a mix of both)
        cc = dec.off.codec_counters()
        ratio = cc["coded_bytes"] / cc["store_bytes"] if cc["store_bytes"] else 1.0
        share = cc["layers"] / max(len(dec.moe_layers), 1)
        link_per_expert = per_expert * (1.0 - share + share * ratio)
        summary, _ = analyse(rings, Clock(cal0, cal1), ids, a.steps, link_per_expert)
        summary = {"workload": f"{a.config}-shaped decode, slots={a.slots}, c={c}, "
                               f"{a.steps} steps centred in a 256-token decode after "
                               f"128-token prompts (traced build)",
                   "ms_per_step": round(dt / a.steps * 1e3, 3),
                   "bytes_per_expert": int(per_expert),
                   "coded_layers": int(cc["layers"]), "moe_layers": len(dec.moe_layers),
                   "link_bytes_per_expert": int(link_per_expert), **summary}
    finally:
        dec.close()
    text = json.dumps(summary)
    if a.json:
        with open(a.json, "w") as f:
            f.write(text + "\n")
    print(text, flush=True)


if __name__ == "__main__":
    main()
