"""The gap-timeline analysis (sluice_amd/timeline.py) on synthetic trace
rings whose answers are known: the clock mapping, the head and tail of a
layer-step that streams, a layer-step that streams nothing, a gap with one
miss served from a staged row and one over the link, a staging chunk, the
pending items' own durations, the link-idle split and the link's busy
time.  No GPU: the rings are built here the way the trace build writes
them (trace.h)."""

import numpy as np

from sluice_amd import timeline as tl

US = 100  # device wall-clock ticks per microsecond (100 MHz)


def _dev(tag, value, tick):
    return [np.uint64((tag << 56) | value), np.uint64(tick)]


def _gap_value(layer_id, stamp):
    return (layer_id << 24) | stamp


def _rings():
    L0, L1, L2 = 0x1000, 0x2000, 0x3000  # device map addresses >> 8
    base = 1_000_000  # ticks
    off = 100.0       # host seconds = ticks / 1e8 + off
    h = lambda us: base / 1e8 + off + us * 1e-6  # noqa: E731
    gap = []
    # layer 0, stamp 5: streams one expert; starts at t = 0
    for tag, us in ((1, 0.0), (2, 3.0), (3, 15.0), (4, 25.0)):
        gap.append(_dev(tag, _gap_value(L0, 5), base + int(us * US)))
    # layer 1, stamp 5: streams nothing; starts 380 us later
    for tag, us in ((1, 380.0), (2, 383.0), (4, 387.0)):
        gap.append(_dev(tag, _gap_value(L1, 5), base + int(us * US)))
    # layer 2, stamp 5: streams one expert; starts at 500 us
    for tag, us in ((1, 500.0), (2, 503.0), (3, 515.0), (4, 525.0)):
        gap.append(_dev(tag, _gap_value(L2, 5), base + int(us * US)))
    moe = [_dev(11, 64, base + 30 * US),
           _dev(10, (3 << 24) | 5, base + int(319.2 * US)),
           _dev(14, 0, base + 320 * US), _dev(15, 0, base + 326 * US),
           _dev(17, 1, base + 327 * US), _dev(16, 1, base + 331 * US),
           _dev(13, 8, base + 333 * US),
           _dev(11, 64, base + 540 * US),
           _dev(13, 8, base + 850 * US)]
    host = []
    # layer 0: one miss over the link; layer 2: one miss from a staged row
    # (copy order 0, landed at 540 us) and one over the link (order 1)
    for lid, t0, landed, staged in ((L0, 0.0, 316.0, 0), (L2, 500.0, 800.0, 1)):
        for tag, v, us in ((21, 1 + staged, 2.5), (22, 1 + staged, 2.8), (23, staged, 6.0),
                           (24, 1, 8.0), (25, 1, 9.0)):
            host.append((tag, lid, 5, v, h(t0 + us)))
        if staged:
            host.append((26, lid, 5, 0, h(540.0)))
            host.append((27, lid, 5, 0, h(540.05)))
        host.append((26, lid, 5, staged, h(landed)))
        host.append((27, lid, 5, staged, h(landed + 0.05)))
    # a staging chunk of 1 MiB on staging lane 0, 330 -> 350 us
    host.append((28, L0, 0, (1024 << 1) | 0, h(330.0)))
    host.append((29, L0, 0, (1024 << 1) | 0, h(350.0)))
    host.append((21, L1, 5, 0, h(382.0)))
    host.append((22, L1, 5, 0, h(382.3)))
    rings = {"gap": np.array(gap, dtype=np.uint64), "moe": np.array(moe, dtype=np.uint64),
             "host": host}
    cal0 = (np.array([base / 1e8 + off]), np.array([float(base)]))
    cal1 = (np.array([(base + 10**6) / 1e8 + off]), np.array([float(base + 10**6)]))
    return rings, tl.Clock(cal0, cal1), [L0, L1, L2]


def test_clock_maps_device_ticks_to_host_seconds():
    _, clock, _ = _rings()
    assert abs(clock(np.array([1_000_000 + 250 * US]))[0] - (100.0 + 0.01 + 250e-6)) < 1e-9


def test_analysis_recovers_the_known_timeline():
    rings, clock, ids = _rings()
    out, rows = tl.analyse(rings, clock, ids, steps=1, bytes_per_expert=17_301_504)
    assert out["layer_steps"] == 3 and out["with_stream_ins"] == 2 and out["without"] == 1
    med = lambda sec, key: out[sec][key]["median_us"]  # noqa: E731
    assert abs(med("head", "first_copy") - 6.0) < 0.05
    assert abs(med("head", "answer_read") - 15.0) < 0.05
    first = next(r for r in rows if r["layer"] == 0)
    assert abs((first["ready_seen"] - first["landed"]) * 1e6 - 3.2) < 0.05
    assert abs((first["g1_done"] - first["landed"]) * 1e6 - 10.0) < 0.05
    assert abs((first["combine"] - first["landed"]) * 1e6 - 17.0) < 0.05
    assert abs((first["next"] - first["landed"]) * 1e6 - 64.0) < 0.05
    assert abs(out["pending_item"]["gemm1_wait_end_to_done"]["median_us"] - 6.0) < 0.05
    assert abs(out["pending_item"]["gemm2_count_to_done"]["median_us"] - 4.0) < 0.05
    assert abs(med("without_stream_ins", "next") - 120.0) < 0.05
    # one streamed expert per window: 17.3 MB over (316 - 6) us and (800 - 506) us
    rates = [17_301_504 / 310e-6 / 1e9, 17_301_504 / 294e-6 / 1e9]
    assert abs(out["copy_window"]["rate_GBs_median"] - np.median(rates)) < 0.05
    # the only idle stretch between the gaps' copies over the link crosses the
    # layer that streams nothing: landed at 316 us -> next first copy at 506 us
    idle = out["gap_copies_idle_ms_per_step"]
    assert idle["between_consecutive_layers_with_copies_over_the_link"] == 0.0
    assert abs(idle["across_layers_without_them"] - 0.190) < 1e-3
    # the link over 0..800 us: copies 6-316 and 506-800, the staging chunk
    # 330-350: busy 624 us, idle 176 us
    link = out["link"]
    assert abs(link["busy_share"] - 624 / 800) < 1e-3
    assert abs(link["idle_ms_per_step"] - 0.176) < 1e-3
    assert link["staging_chunks_per_step"] == 1.0
    assert abs(link["staging_chunk_us_median"] - 20.0) < 0.05
    assert abs(link["staging_MB_per_step"] - 1.05) < 1e-2
    assert link["gaps_with_staged_misses"] == 1 and link["gaps_all_staged"] == 0
