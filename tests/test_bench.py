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
    layer = synth.make_layer(shape, 5)

    class HostExperts:  # the one method cpu_baseline uses, over host arrays
        def host_subset(self, ids):
            return {k: v[np.asarray(ids)] for k, v in layer.items()}

    r = bench.cpu_baseline(HostExperts(), shape, 1.0)
    assert r["kind"] == "port" and r["unit"] == "GB/s" and r["value"] > 0
    assert r["cores"] == min(shape.top_k, os.cpu_count() or 1, 16)
    assert r["single_thread"]["tokens"] >= 1 and r["single_thread"]["us_per_token"] > 0
    assert abs(r["prefill_T512_s_extrapolated"] - 512 * r["us_per_token"] * 1e-6) < 1e-3
    assert r["host"]["nproc"] == os.cpu_count()


def test_stage1_traffic_matches_committed_summary():
    import bench

    with open(bench.TRAFFIC_FILE) as f:
        t = json.load(f)
    want = t["fetch_kib_per_dispatch"] * 1024 / t["copy_fetch_ratio"] + t["write_kib_per_dispatch"] * 1024 / t["copy_write_ratio"]
    got = bench.stage1_traffic(7361600)
    assert got == round(want)
    # the kernel reads what it should: within 10% of the algorithmic bytes of the workload
    assert 1.0 <= got / 7361600 < 1.1
