"""bench.py's command line: the one-GPU contract is enforced before any
device work (a request for several GPUs exits with status 2 and says why)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("n", [2, 8])
def test_bench_refuses_more_than_one_gpu(n):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", str(n)],
                       cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert r.stdout == ""  # no JSON line for a refused run
    assert f"--gpus {n} is not supported" in r.stderr and "one GPU" in r.stderr


def test_bench_rejects_unknown_config():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--config", "nope"],
                       cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "invalid choice" in r.stderr


def _fixture_record():
    import gzip
    import json

    with gzip.open(os.path.join(ROOT, "tests", "fixtures", "bench_record_v2lite.json.gz"),
                   "rt") as f:
        return json.load(f)


def test_compact_line_fits_and_parses():
    """The last stdout line is built from the full record of a default run
    (DeepSeek-V2-Lite headline plus the Qwen3, V3 and stress rows) and stays
    under LINE_LIMIT bytes, so a driver keeping only the end of stdout
    receives it whole; it parses and carries the contract's fields."""
    import json

    sys.path.insert(0, ROOT)
    import bench

    rec = _fixture_record()
    text = json.dumps(bench.compact_line(rec), separators=(",", ":"), allow_nan=False)
    assert len(text.encode()) <= bench.LINE_LIMIT, len(text)
    line = json.loads(text)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline", "h2d", "rows"):
        assert key in line, key
    assert line["value"] == round(rec["value"], 2)
    assert line["config"]["workload"] == rec["config"]["workload"]
    roof = line["roofline"]
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    assert line["cpu_baseline"]["cores"] >= 1 and line["cpu_baseline"]["kind"] == "port"
    # one row per measured batch of every configuration, headline first
    n_rows = len(rec["per_batch"]) + sum(len(e["per_batch"]) for e in rec["extras"])
    assert len(line["rows"]) == n_rows
    cols = line["row_cols"]
    first = dict(zip(cols, line["rows"][0]))
    assert first["shape"] == rec["config"]["model_shape"]
    head = dict(zip(cols, next(r for r in line["rows"] if r[2] == line["config"]["batch"])))
    assert head["ref_tok_per_s"] == 1062.6  # README.md:51, V2-Lite c=8
    # the staging rows the headline ran with, and the share of its misses they served
    assert line["config"]["staging_rows_per_layer"] == 6
    assert 0.0 < head["staged_share_of_misses"] < 1.0
    # coded host stores: every V2-Lite layer, at ~0.75 of the rows; the rows in
    # the reference's orchestration decode nothing
    coded = line["config"]["coded_store"]
    assert coded["layers"] == coded["of_layers"] == 26 and 0.74 < coded["bytes_frac"] < 0.76
    assert head["coded_layers"] == 26
    assert all(dict(zip(cols, r))["coded_layers"] == 0 for r in line["rows"]
               if r[cols.index("path")].endswith("/ref-orch"))


def test_compact_line_stays_under_the_limit_with_every_row_doubled():
    """Headroom: twice as many batch rows still fit."""
    import json

    import bench

    rec = _fixture_record()
    for e in rec["extras"]:
        e["per_batch"] = e["per_batch"] * 2
    rec["per_batch"] = rec["per_batch"] * 2
    text = json.dumps(bench.compact_line(rec), separators=(",", ":"))
    assert len(text.encode()) <= bench.LINE_LIMIT, len(text)


def test_compact_line_is_strict_json_when_a_figure_is_missing():
    """A non-finite figure (a row that streamed nothing, a kernel not timed)
    becomes null, so the line parses with a strict JSON reader."""
    import json

    import bench

    rec = _fixture_record()
    rec["per_batch"][0]["h2d_GBs_in_step"] = float("nan")
    rec["roofline"]["read_probe_GBs"] = float("inf")
    line = json.loads(json.dumps(bench.compact_line(rec), allow_nan=False))
    assert line["rows"][0][line["row_cols"].index("h2d_GBs_in_step")] is None
    assert line["roofline"]["read_probe_GBs"] is None
