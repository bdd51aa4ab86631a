"""bench.py's host-side contract, without a GPU: one GPU only, the host
description beside the CPU baseline, and the committed PMC traffic figures
that its roofline objects report."""

import os
import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parent.parent


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_host_description():
    host = bench._host_cpu()
    assert host["nproc"] == os.cpu_count()
    assert host["cpu"] is None or isinstance(host["cpu"], str)


def test_traffic_of_the_roofline_kernels_is_committed():
    # The kernels whose roofline objects carry a `traffic` figure.
    for kernel in ("dn_mfma_scan", "dn_step_row", "dn_recurrent_row", "dn_frontend",
                   "dn_out_norm", "dn_mfma_chunk_bwd"):
        t = bench.traffic_from_profiles(kernel)
        assert t is not None and t > 0, kernel
    assert bench.traffic_from_profiles("no_such_kernel") is None
