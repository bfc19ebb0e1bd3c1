"""The bench's stdout line: strict JSON, under 4 KB, with the keys the
driver reads, built from a fixture shaped like a full default run (every
workload, long descriptions, the CPU baseline) without a GPU."""
from __future__ import annotations

import json

import bench


def _fixture_results():
    res = {}
    for i, nm in enumerate(bench.DEFAULT_WORKLOADS):
        us = 1.5 + 13.7 * i
        r = {"workload": f"{nm}: a long description of the workload, its shapes and its dtype " * 2,
             "kernel": f"nsrk_some_kernel_name_{nm}_b512_v40_l18", "dtype": "f32",
             "algorithmic_bytes": 943727104, "buffer_sets": 60, "footprint_MB": 1283.4,
             "us_per_call": round(us, 3), "GBs": round(943727104 / us / 1e3, 1),
             "frac_of_peak": 0.7123, "first_touch_us_per_call": round(us * 1.2, 3),
             "warm_us_per_call": us, "warm_GBs": 1.0, "host_us_per_call": 7.23,
             "copy_floor_us": 144.945, "frac_of_copy": 0.87, "traffic": 1887436800}
        if nm.startswith("kconv") or nm.startswith("kchain"):
            r["TFLOPs"] = 434.46
        res[nm] = r
    res["c4b"]["row_copy_floor_us"] = 172.267
    res["c3"]["frac_of_peak"] = float("nan")  # a non-finite figure must not break the line
    return res


def _fixture_cpu():
    per = {nm: [123456.7, 9876.5] for nm in bench.CONFIG_WORKLOADS}
    return {"value": 0.812, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": "oracle C restatement of the reference CPU path on c4b: 8 of the 1024 rows (x[1,8,115200]), "
                      "scaled; median of 20 runs after 3 warm-ups, 1 thread",
            "cpu_model": "AMD EPYC 9575F 64-Core Processor", "host_threads": 16, "us_per_call": per,
            "us_per_call_fields": ["1 thread", "16 threads"]}


def test_line_is_compact_strict_json():
    line = bench.compact_line(_fixture_results(), 20, 5, _fixture_cpu(),
                              {"start": 2400, "after_mfma": 2100, "end": 2400})
    text = json.dumps(line, allow_nan=False)
    assert len(text.encode()) < bench.LINE_LIMIT_BYTES, len(text)
    back = json.loads(text)
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in back, k
    assert back["metric"] == json.load(open(bench.ROOT / "BASELINE.json"))["metric"]
    assert back["value"] == back["roofline"]["achieved"]
    assert back["roofline"]["bound"] == "hbm" and back["roofline"]["peak"] == 8000.0
    assert back["config"]["workload"].startswith("configs[4]")
    assert "c4a" in back["config"]["alongside"]
    assert back["cpu_baseline"]["kind"] == "port" and back["cpu_baseline"]["cores"] == 1
    # every non-copy workload has its short array; the copies appear only as their configs' copy_floor_us
    n = len(bench.PER_CONFIG_FIELDS)
    for nm in bench.DEFAULT_WORKLOADS:
        if nm.startswith("copy_") and nm != "copy_rows_c4b":
            assert nm not in back["per_config"]
        else:
            assert len(back["per_config"][nm]) in (n, n + 1), nm
    assert back["per_config"]["c3"][bench.PER_CONFIG_FIELDS.index("frac_of_peak")] is None


def test_gpus_above_one_exits_with_message(monkeypatch, capsys):
    import pytest

    monkeypatch.setattr("sys.argv", ["bench.py", "--gpus", "2"])
    with pytest.raises(SystemExit) as e:
        bench.main()
    assert e.value.code == 2
    assert "single MI355X" in capsys.readouterr().err
