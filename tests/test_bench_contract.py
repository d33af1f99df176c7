"""bench.py's contract on the CPU: the one-GPU rule and the algorithmic byte
counts its GB/s figures divide by (BASELINE's formula: per sequence and layer
(pos+1)*2*row + 2*row + 4*(2*nq + 2*nkv))."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_step_bytes_follow_the_baseline_formula():
    shape = bench.CONFIGS["c4"][0]
    poss = [8192] * 256
    row = 1088  # ceil(1024 / 32) * 34
    per = (8192 + 1) * 2 * row + 2 * row + 4 * (2 * 2048 + 2 * 1024)
    assert bench.row_bytes(shape) == row
    assert bench.step_bytes(shape, poss) == 256 * 28 * per == 127982632960
    assert bench.launch_bytes(shape, poss, 1) == 256 * per == 4570808320
    assert bench.launch_bytes(shape, poss, 28) == bench.step_bytes(shape, poss)


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5"])
def test_other_configs_rows(name):
    shape = bench.CONFIGS[name][0]
    nkv = shape.n_kv_heads * shape.head_dim
    want = -(-nkv // 32) * 34 if shape.kv_q8 else nkv * 4
    assert bench.row_bytes(shape) == want
    assert bench.step_bytes(shape, [0]) == shape.n_layers * (
        2 * want + 2 * want + 4 * (2 * shape.nq + 2 * nkv))
