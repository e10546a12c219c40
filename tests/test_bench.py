"""CPU checks of bench.py's contract: the one-GPU refusal, the CPU-baseline record and the
traffic figure read from the committed counter summary."""
import json
import os
import subprocess
import sys

import numpy as np

from tests.conftest import ROOT


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr)


def test_cpu_baseline_record():
    import bench
    from kandiga_amd import synth

    shape = synth.LayerShape(512, 256, 16, 4, 3)
    r = bench.cpu_baseline(shape, 0.5, synth.LayerShape(512, 256, 16, 4, 4))
    assert r["kind"] == "port" and r["unit"] == "GB/s" and r["value"] > 0
    assert r["cores"] == min(shape.top_k, os.cpu_count() or 1, 16)
    assert r["single_thread"]["tokens"] >= 1 and r["single_thread"]["us_per_token"] > 0
    assert r["checker_restatement"]["us_per_token"] > 0
    assert r["layer_4bit"]["us_per_token"] > 0
    assert abs(r["prefill_T512_s_extrapolated"] - 512 * r["us_per_token"] * 1e-6) < 1e-3
    assert r["host"]["nproc"] == os.cpu_count()


def test_kernel_traffic_reads_committed_summaries():
    """Every committed counter summary turns into a traffic figure: (FETCH + WRITE) KiB per
    dispatch over the copy-calibrated ratios; a kernel without a summary gives null."""
    import glob

    import bench

    files = glob.glob(os.path.join(bench.PROFILES, "*_decode_t1_k8_traffic.json"))
    assert files
    for fn in files:
        with open(fn) as f:
            t = json.load(f)
        want = t["fetch_kib_per_dispatch"] * 1024 / t["copy_fetch_ratio"] + \
            t["write_kib_per_dispatch"] * 1024 / t["copy_write_ratio"]
        assert bench.kernel_traffic(t["kernel"]) == round(want)
    assert bench.kernel_traffic("no_such_kernel") is None
