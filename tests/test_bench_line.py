"""The bench's stdout line stays small enough for a log tail to hold it whole.

The line is built from a canned result for every default workload (the real names and
descriptions, figures and CPU legs of the size a run produces); it must be valid JSON,
carry the contract's fields, and stay under 6,000 bytes whatever the workload count."""

from __future__ import annotations

import importlib.util
import json
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent


def _bench():
    if str(REPO) not in sys.path:
        sys.path.insert(0, str(REPO))
    import __graft_entry__

    __graft_entry__.load_package()
    if "_omnia_bench" in sys.modules:
        return sys.modules["_omnia_bench"]
    spec = importlib.util.spec_from_file_location("_omnia_bench", REPO / "bench.py")
    module = importlib.util.module_from_spec(spec)
    sys.modules["_omnia_bench"] = module
    spec.loader.exec_module(module)
    return module


def _canned(bench, extra: int = 0) -> dict:
    results = {}
    names = [(w.name, w.description, w.kernel, w.bytes_per_launch)
             for w in bench.workloads() if w.default]
    names += [(f"extra_workload_{i}", "x" * 200, "extra_kernel", 1 << 20) for i in range(extra)]
    for i, (name, description, kernel, nbytes) in enumerate(names):
        us = 16.907 + i
        gbs = nbytes / (us * 1e-6) / 1e9
        results[name] = dict(
            us=round(us, 3), GBps=round(gbs, 1), frac=round(gbs / 8000.0, 4), bytes=nbytes,
            copies=7, kernel=kernel, workload=description, ms_total=3.3814, launch="direct",
            cpu_baseline=dict(
                value=0.5037, unit="GB/s", us_per_launch=170688.5, cores=16, kind="port",
                sample="numpy oracle, 512 of the 4096 tokens: 18 run(s) in 3.02 s",
                affinity_cores=16,
                threads_env={"OMP_NUM_THREADS": "16", "OPENBLAS_NUM_THREADS": "16",
                             "MKL_NUM_THREADS": "16"}))
    return results


def test_bench_line_is_compact_json():
    bench = _bench()
    results = _canned(bench)
    assert len(results) >= 30 and bench.HEADLINE in results
    line = bench.bench_line(results, bench.HEADLINE, 200, 20)
    text = json.dumps(line, separators=(",", ":"))
    assert len(text.encode()) < 6000, len(text)
    back = json.loads(text)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline"):
        assert key in back, key
    head = results[bench.HEADLINE]
    assert back["value"] == head["GBps"]
    assert back["ms_per_step"] == round(head["us"] / 1000.0, 6)
    assert back["roofline"]["achieved"] == head["GBps"]
    assert back["roofline"]["frac"] == head["frac"]
    assert back["roofline"]["peak"] == bench.PEAK_GBS
    assert back["cpu_baseline"]["kind"] == "port" and back["cpu_baseline"]["cores"] == 16
    assert set(back["kernels"]) == set(results)
    for name, (us, frac, cpu) in back["kernels"].items():
        assert us == results[name]["us"] and frac == results[name]["frac"] and cpu == 0.5037


def test_bench_line_grows_slowly_with_workloads():
    bench = _bench()
    results = _canned(bench, extra=10)
    text = json.dumps(bench.bench_line(results, bench.HEADLINE, 20, 5), separators=(",", ":"))
    # ten more workloads with long descriptions add only their compact entries
    assert len(text.encode()) < 6000 + 10 * 80


def test_bench_line_without_cpu_leg():
    bench = _bench()
    results = _canned(bench)
    for r in results.values():
        r.pop("cpu_baseline")
    line = bench.bench_line(results, bench.HEADLINE, 20, 5)
    assert line["cpu_baseline"] is None
    assert all(entry[2] is None for entry in line["kernels"].values())
