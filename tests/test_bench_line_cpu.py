"""The bench line on the CPU: built from a synthetic measurement the size of a
real one (19 shapes, the dominant kernel's roofline with its traffic source,
both CPU baselines with a per-shape list), it stays under the size bound,
round-trips through JSON, carries every key the driver reads, and leaves the
per-shape CPU list and the extra sections to the detail lines before it."""
import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402


def synthetic():
    per_shape = []
    for i, h in enumerate(bench.H_SWEEP):
        us = 5.0 * h / 1024 + 1.7
        per_shape.append({"rows": bench.B, "hidden": h, "us_per_call": round(us, 2), "us_p10": round(us * 0.99, 2),
                          "us_p90": round(us * 1.01, 2),
                          "gbs": round(bench.fused_bytes(bench.B, h) / (us * 1e-6) / 1e9, 1),
                          "kernel": {"lanes_per_row": 1024, "vec_per_lane": 4, "lds_vec_per_lane": 4 * (i % 2),
                                     "block": 1024, "flags": 159}})
    roofline = {"bound": "hbm", "achieved": 6321.4, "peak": bench.PEAK_GBS, "unit": "GB/s", "frac": 0.7902,
                "traffic": 1074326881,
                "kernel": ("fused_vec_kernel<bf16, fused, lanes_per_row=1024, vec_per_lane=4, lds_vec_per_lane=0, "
                           "block=1024, flags=159>"),
                "kernel_hidden": [28672, 32768], "avg_launch_us": 169.78,
                "algorithmic_bytes_per_launch": 1073807360,
                "traffic_source": {"profiled_shape": [4096, 32768], "hbm_bytes_per_launch_profiled": 1074326881,
                                   "algorithmic_bytes_per_launch_profiled": 1073807360, "ratio": 1.00048,
                                   "source": "profiles/fused_add_rmsnorm_bf16_4096x32768_counters.md"}}
    cpu = {"value": 8.123, "unit": "GB/s", "cores": 16, "kind": "port",
           "what": "the reference test's torch formula (test/test_hp_rms_norm.py:6-19), torch eager on the CPU",
           "sample": "the full benchmark workload: bf16 (4096, H) for the 19 H of the sweep, 3.73 GB algorithmic; "
                     "per shape 1 warm-up + median of 3 calls",
           "torch_threads": 16, "os_cpu_count": 256, "cpu_model": "AMD EPYC 9575F 64-Core Processor",
           "per_shape": [{"rows": bench.B, "hidden": h, "ms_per_call": 123.45, "gbs": 8.01} for h in bench.H_SWEEP]}
    cpu_oracle = {"value": 15.2, "unit": "GB/s", "cores": 16, "kind": "port",
                  "what": "the CPU oracle (oracle/hprms_oracle.c, OpenMP over rows)",
                  "sample": "256 rows x each H of the sweep (bf16, 19 shapes, 233 MB algorithmic per pass), "
                            "median of 40 passes"}
    extra = {"decode_bf16": [{"rows": b, "hidden": h, "us_per_call": 2.5} for b in (1, 8) for h in (4096, 8192)],
             "ceiling_bf16": [{"hidden": 4096, "timeline": {"workgroups": 4096, "span_us": 22.9}}]}
    return per_shape, roofline, cpu, cpu_oracle, extra


def make_line():
    per_shape, roofline, cpu, cpu_oracle, extra = synthetic()
    details = bench.detail_lines(extra, cpu)
    step_bytes = sum(bench.fused_bytes(bench.B, h) for h in bench.H_SWEEP)
    line = bench.headline(value=6158.3, steps=20, warmup=5, step_ms=1.2318, step_bytes=step_bytes,
                          per_shape=per_shape, roofline=roofline, cpu=cpu, cpu_oracle=cpu_oracle,
                          details=[d["bench_detail"] for d in details])
    return line, details, per_shape, cpu


def test_bench_line_fits_and_round_trips():
    line, details, per_shape, cpu = make_line()
    text = json.dumps(line)
    assert "\n" not in text
    assert len(text.encode()) <= bench.HEADLINE_MAX_BYTES
    back = json.loads(text)
    assert back == line
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "per_shape", "roofline", "cpu_baseline"):
        assert k in back, k
    assert back["metric"] == json.load(open(os.path.join(ROOT, "BASELINE.json")))["metric"]
    assert back["n_gpus"] == 1 and back["vs_baseline"] is None and back["dtype"] == "bf16"
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in back["roofline"], k
    assert back["roofline"]["frac"] == pytest.approx(back["roofline"]["achieved"] / back["roofline"]["peak"], 1e-3)
    for k in ("value", "unit", "cores", "kind", "sample", "torch_threads", "cpu_model"):
        assert k in back["cpu_baseline"], k
    assert "per_shape" not in back["cpu_baseline"] and "extra" not in back
    # one compact entry per shape of the sweep, in order, with its kernel
    assert [p["hidden"] for p in back["per_shape"]] == bench.H_SWEEP
    for p, q in zip(back["per_shape"], per_shape):
        assert p["us"] == q["us_per_call"] and p["gbs"] == q["gbs"]
        assert p["us_p10_p90"] == [q["us_p10"], q["us_p90"]]
        assert p["kernel"].startswith("1024x4")
    assert back["per_shape"][1]["kernel"] == "1024x4 (4)/1024 f159"


def test_detail_lines_carry_what_the_bench_line_leaves_out():
    line, details, per_shape, cpu = make_line()
    names = [d["bench_detail"] for d in details]
    assert names == ["decode_bf16", "ceiling_bf16", "cpu_baseline_per_shape"]
    assert line["details_on_earlier_lines"] == names
    assert details[-1]["data"] == cpu["per_shape"]
    for d in details:
        assert json.loads(json.dumps(d)) == d


def test_oversized_bench_line_is_refused():
    per_shape, roofline, cpu, cpu_oracle, extra = synthetic()
    roofline = dict(roofline, padding="x" * bench.HEADLINE_MAX_BYTES)
    with pytest.raises(RuntimeError, match="exceeds"):
        bench.headline(value=1.0, steps=1, warmup=0, step_ms=1.0, step_bytes=1, per_shape=per_shape,
                       roofline=roofline, cpu=cpu, cpu_oracle=cpu_oracle)
