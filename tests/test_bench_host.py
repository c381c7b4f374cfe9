"""bench.py's host side without a GPU: the headline workload, the HBM-traffic
figure each bench line carries (read from the committed rocprofv3 summary of
that workload, none for a workload without one), and the one-GPU contract
(a request for more GPUs exits with a message before touching the GPU)."""

import os
import re
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_headline_workload():
    assert bench.WORKLOADS["gemm4096"] == (4096, 4096, 4096, "row", torch.float16)
    assert bench.WORKLOADS["gemm8192"] == (8192, 8192, 8192, "row", torch.float16)


def test_traffic_comes_from_the_workloads_own_summary():
    for workload, name in (("gemm4096", "gemm_4096"), ("gemm8192", "gemm_8192")):
        path = os.path.join(ROOT, "profiles", f"{name}_fp16out_rowmajorB_traffic.txt")
        want = float(re.search(r"^traffic_bytes_per_launch:\s*(\d+)", open(path).read(), re.M).group(1))
        assert bench.read_traffic(workload) == want
    # the two sizes move different bytes: one figure must not stand in for the other
    assert bench.read_traffic("gemm8192") > 4 * bench.read_traffic("gemm4096")
    assert bench.read_traffic("qwen_qo") is None


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and '"metric"' not in r.stdout


@pytest.mark.parametrize("n, rounds", [(2, 4), (2, 6), (3, 6), (7, 4), (8, 4)])
def test_every_op_is_timed_first_equally_often(n, rounds):
    """bench.round_order: each round times every op once, and over the
    rounds each op goes first as often as any other (within one), so the
    slow first burst after a switch is not charged to one op."""
    names = [f"op{i}" for i in range(n)]
    firsts = {k: 0 for k in names}
    for r in range(rounds):
        order = bench.round_order(names, r)
        assert sorted(order) == sorted(names)
        firsts[order[0]] += 1
    counts = [firsts[k] for k in names]
    assert max(counts) - min(counts) <= 1
