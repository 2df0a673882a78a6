"""Measurement helpers (reference fp8_training/fp8_bench/utils.py interface):
percentile against numpy's linear interpolation, accuracy_metrics against
closed forms, dtype parsing."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from practice_cuda_amd import utils as U


def test_percentile_matches_linear_interpolation():
    rng = np.random.default_rng(0)
    for n in (1, 2, 5, 8):
        v = list(rng.standard_normal(n))
        for q in (0.0, 0.2, 0.5, 0.8, 1.0):
            assert math.isclose(U.percentile(v, q), float(np.percentile(v, 100 * q)), rel_tol=1e-12, abs_tol=1e-12)
    assert math.isnan(U.percentile([], 0.5))


def test_accuracy_metrics_closed_forms():
    e = torch.tensor([3.0, 4.0, 0.0, 0.0])
    a = torch.tensor([3.0, 4.0, 0.0, 2.0])            # error 2 in one element
    m = U.accuracy_metrics(a, e)
    assert m["finite"] and m["nan_count"] == 0 and m["inf_count"] == 0
    assert m["max_abs"] == 2.0 and m["mean_abs"] == 0.5
    assert m["mse"] == 1.0 and m["rmse"] == 1.0
    assert math.isclose(m["rel_l2"], 2.0 / 5.0, rel_tol=1e-6)
    assert math.isclose(m["cosine"], 25.0 / (5.0 * math.sqrt(29.0)), rel_tol=1e-6)
    same = U.accuracy_metrics(e, e)
    assert same["max_abs"] == 0.0 and same["rel_l2"] == 0.0 and math.isclose(same["cosine"], 1.0, rel_tol=1e-6)
    bad = U.accuracy_metrics(torch.tensor([float("nan"), float("inf"), 1.0]), torch.ones(3))
    assert not bad["finite"] and bad["nan_count"] == 1 and bad["inf_count"] == 1


def test_parse_dtype():
    assert U.parse_dtype("BF16") is torch.bfloat16 and U.parse_dtype("e4m3") is torch.float8_e4m3fn
    with pytest.raises(ValueError, match="unknown dtype"):
        U.parse_dtype("int8")


@pytest.mark.gpu
def test_benchmark_cuda(dev):
    x = torch.randn(1 << 20, device=dev)
    r = U.benchmark_cuda(lambda: x.mul_(1.0), warmup=2, iters=5, repeats=3)
    assert len(r["samples_ms"]) == 3 and r["min_ms"] <= r["median_ms"] <= r["max_ms"]
    assert r["min_ms"] <= r["p20_ms"] <= r["p80_ms"] <= r["max_ms"] and r["min_ms"] > 0
