"""bench.py's contract checked on the host: one GPU only, and the
algorithmic byte and flop counts its roofline figures divide by are the ones
the design notes quote."""

from __future__ import annotations

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr and not proc.stdout.strip()


def test_decode_bytes_of_the_measured_workloads():
    # B=64, Hk=16, Hv=32, d=128, 4 taps (pooled decode): the state tiles read
    # and written once (8 Hv d^2 bytes a sequence) are ~97 % of the bytes, the
    # conv state (3 C bf16 values read and written) and the inputs the rest
    per_token, per_step, total = bench.decode_bytes(64, 16, 32, 128, 4, False)
    assert total == 276_439_296
    assert 0.96 < 8 * 32 * 128 * 128 / per_token < 0.98
    # the fused gated norm adds z (2 bytes an element) and the norm weight
    _, _, with_z = bench.decode_bytes(64, 16, 32, 128, 4, True)
    assert with_z == total + 64 * 2 * 32 * 128 + 4 * 128


def test_prefill_flops_of_the_measured_workload():
    # T=4096, Hv=32: T Hv (10 64 d + 6 d^2), 23.62 GFLOP
    assert bench.prefill_flops(4096, 32) == 23_622_320_128


def test_committed_traffic_figures_match_the_algorithmic_bytes():
    """The rocprofv3 FETCH/WRITE totals the roofline lines carry: the decode
    launches move within a few percent of their algorithmic bytes (no
    re-reads); the prefill call's 2.6x is its records and the slices'
    re-reads of K, Q and the records."""

    b64 = bench.load_traffic("gdn_decode_step_b64_hv32_traffic.json")
    b256 = bench.load_traffic("gdn_decode_step_b256_hv64_traffic.json")
    prefill = bench.load_traffic("gdn_prefill_chunked_t4096_traffic.json")
    assert 1.0 <= b64 / bench.decode_bytes(64, 16, 32, 128, 4, False)[2] < 1.05
    assert 1.0 <= b256 / bench.decode_bytes(256, 16, 64, 128, 4, True)[2] < 1.05
    assert 2.0 < prefill / 105e6 < 3.0
