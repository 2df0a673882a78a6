"""CPU tests of bench.py's contract pieces that need no GPU: the exit for more
than one GPU, the CPU baseline's quantizers (the reference's PyTorch forms
that cpu_baseline times) against the oracle byte for byte, and the synthetic
BASELINE inputs."""
from __future__ import annotations

import json
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import bench
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int32).numpy()


@pytest.mark.parametrize("seed,scale", [(0, 0.02), (1, 3.0)])
def test_cpu_baseline_channel_form_matches_oracle(seed, scale):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(48, 7168, generator=g) * scale)
    x[5, 100] = 0.0
    x[7] = 0.0  # an all-zero row takes the eps floor
    x = x.bfloat16()
    q, s = bench.torch_channel_quant(torch, x)
    q_ref, s_ref = O.quant_channel(x, -2)
    assert np.array_equal(q.view(torch.uint8).numpy(), q_ref)
    assert np.array_equal(_bits(s), np.asarray(s_ref, np.float32).view(np.int32))


@pytest.mark.parametrize("seed", [0, 1])
def test_cpu_baseline_group_form_matches_oracle(seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(32, 7168, generator=g)
    x[torch.rand(32, 7168, generator=g) < 0.01] *= 50
    x[3, :128] = 0.0  # a zero group
    x = x.bfloat16()
    q, s = bench.torch_group_quant(torch, x)
    q_ref, s_ref = O.quant_block(x, 1, 128)
    assert np.array_equal(q.view(torch.uint8).numpy(), q_ref)
    assert np.array_equal(_bits(s), np.asarray(s_ref, np.float32).view(np.int32))


def test_config_inputs_follow_baseline():
    x1 = bench.make_config1(torch)
    assert x1.shape == (4096, 7168) and x1.dtype == torch.bfloat16
    big = (x1.float().abs() > 6).float().mean().item()  # outliers (x50) dominate |x| > 6
    assert 0.0005 < big < 0.002
    x3 = bench.make_config3(torch)
    assert x3.shape == (4096, 7168) and x3.dtype == torch.bfloat16
    # per-block magnitudes spread over about two decades (log-uniform multipliers in [0.1, 10])
    blk = x3.float().view(32, 128, 56, 128).abs().amax(dim=(1, 3))
    assert blk.max().item() / blk.min().item() > 30
