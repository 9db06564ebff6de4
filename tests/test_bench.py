"""bench.py's contract on the CPU: it measures one GPU only, and the committed rocprof summaries it cites hold the
kernels it reports (the roofline objects take their `traffic` from the HBM-traffic summary by kernel name)."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from hummingbird_amd import workloads as wl  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=300)
    assert res.returncode == 2
    assert "one GPU only" in json.loads(res.stdout.strip().splitlines()[-1])["error"]


def test_traffic_summary_holds_the_reported_kernels():
    measured = json.loads(bench.TRAFFIC_FILE.read_text())["hbm_bytes_per_launch"]
    algorithmic = {bench.DENSE_KERNEL: wl.dense_bytes(2, 2584, 24, 64), bench.BAND_KERNEL: wl.band_bytes(1, 82688, 8, 64)}
    for kernel, alg in algorithmic.items():
        assert kernel in measured, f"{kernel} missing from {bench.TRAFFIC_FILE.name}"
        # counted HBM bytes can only exceed the algorithmic ones by re-reads; far below them means a wrong kernel
        assert 0.95 <= measured[kernel] / alg <= 2.0, (kernel, measured[kernel], alg)


def test_kernel_traces_name_the_reported_kernels():
    for name in ("kernel_trace_120s_clip.md", "hbm_traffic_120s_clip.md", "counters_120s_clip.md"):
        text = (ROOT / "profiles" / name).read_text()
        for kernel in (bench.DENSE_KERNEL, bench.BAND_KERNEL):
            assert f"`{kernel}`" in text, f"{kernel} not in profiles/{name}"
