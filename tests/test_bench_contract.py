"""bench.py's driver contract and bookkeeping, on the CPU: one GPU only (any
other --gpus or a multi-rank launch exits with status 2 before touching a
GPU), the seeded per-layer format plan, the stack's FLOP count per frame and
the roofline bound min(MFMA peak, arithmetic intensity x 8 TB/s)."""
import os
import subprocess
import sys

import pytest

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}), ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused(argv, env):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *argv], capture_output=True, text=True,
                       timeout=120, env=dict(os.environ, **env), cwd=ROOT)
    assert r.returncode == 2, (r.returncode, r.stderr[-500:])
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_format_plan_is_seeded_and_complete():
    plan = bench.format_plan()
    assert plan == bench.format_plan(0x5EED0005)
    assert len(plan) == bench.LAYERS and all(len(layer) == len(bench.LINEARS) for layer in plan)
    used = {f for layer in plan for f in layer}
    assert used == set(bench.FORMATS)  # the mix exercises every format
    assert bench.format_plan(1) != plan


def test_flop_per_frame():
    # per layer: FF1 and FF2 (1024 -> 4096 -> 1024), QKV 1024 -> 3072, attention
    # out 1024 -> 1024, pointwise 1024 -> 2048 and 1024 -> 1024
    d, ff = 1024, 4096
    per_layer = 2 * (2 * ff * d) * 2 + 2 * 3 * d * d + 2 * d * d + 2 * 2 * d * d + 2 * d * d
    assert bench.FLOP_PER_FRAME == 24 * per_layer == 1157627904


def test_roofline_bound():
    assert bench.roof(1e12, 1e9, 5000.0) == 5000.0  # 1000 flop per byte: MFMA bound
    assert bench.roof(1e12, 1e12, 5000.0) == pytest.approx(8.0)  # 1 flop per byte: 8 TB/s
    assert bench.PEAK["fp8"] == bench.PEAK["int8"] == 2 * bench.PEAK["fp16"] == 5000.0
