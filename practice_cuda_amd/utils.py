"""Measurement helpers with the reference's interface.

Counterpart of xuOAO/practice_cuda ``fp8_training/fp8_bench/utils.py``:
``parse_dtype`` (:28-32), ``seed_everything`` (:35-38), ``percentile``
(:41-49, linear interpolation between order statistics), ``benchmark_cuda``
(:52-84: warmup, then the median of ``repeats`` timed loops of ``iters``
calls, HIP events on the current stream) and ``accuracy_metrics`` (:88-112).
Same names, arguments and result keys, so the reference's bench scripts can
import them from here.
"""
from __future__ import annotations

import math
import statistics
from typing import Any, Callable

import torch

DTYPES: dict[str, torch.dtype] = {
    "fp32": torch.float32, "float32": torch.float32,
    "fp16": torch.float16, "float16": torch.float16,
    "bf16": torch.bfloat16, "bfloat16": torch.bfloat16,
    "e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2,
}


def parse_dtype(name: str) -> torch.dtype:
    """torch dtype for a name in ``DTYPES`` (case-insensitive); ValueError otherwise."""
    dt = DTYPES.get(name.lower())
    if dt is None:
        raise ValueError(f"unknown dtype {name}; choices={sorted(DTYPES)}")
    return dt


def seed_everything(seed: int) -> None:
    torch.manual_seed(seed)
    if torch.cuda.is_available():
        torch.cuda.manual_seed_all(seed)


def percentile(values: list[float], q: float) -> float:
    """q-quantile (0 <= q <= 1) by linear interpolation between the sorted
    values at ranks floor / ceil of (n - 1) q; NaN for an empty list."""
    xs = sorted(values)
    if not xs:
        return math.nan
    pos = (len(xs) - 1) * q
    lo = math.floor(pos)
    frac = pos - lo
    if frac == 0.0:
        return xs[lo]
    return xs[lo] + (xs[lo + 1] - xs[lo]) * frac


def benchmark_cuda(fn: Callable[[], Any], *, warmup: int = 20, iters: int = 100,
                   repeats: int = 5) -> dict[str, Any]:
    """Per-call milliseconds of ``fn`` on the current stream: ``warmup`` untimed
    calls, then ``repeats`` loops of ``iters`` calls, each bracketed by events."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    samples = []
    for _ in range(repeats):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            fn()
        end.record()
        torch.cuda.synchronize()
        samples.append(start.elapsed_time(end) / iters)
    mean = statistics.fmean(samples)
    sd = statistics.pstdev(samples) if len(samples) > 1 else 0.0
    return {"median_ms": statistics.median(samples), "p20_ms": percentile(samples, 0.2),
            "p80_ms": percentile(samples, 0.8), "min_ms": min(samples), "max_ms": max(samples),
            "cv": sd / mean if mean else 0.0, "samples_ms": samples}


@torch.no_grad()
def accuracy_metrics(actual: torch.Tensor, expected: torch.Tensor) -> dict[str, Any]:
    """Error statistics of ``actual`` against ``expected`` in fp32: finiteness
    counts, max / mean absolute error, MSE, RMSE, relative L2 error
    (|a - e| / max(|e|, 1e-12)) and cosine similarity."""
    a, e = actual.float(), expected.float()
    d = a - e
    mse = d.square().mean()
    e_norm = torch.linalg.vector_norm(e)
    return {
        "finite": bool(torch.isfinite(a).all().item()),
        "nan_count": int(torch.isnan(a).sum().item()),
        "inf_count": int(torch.isinf(a).sum().item()),
        "max_abs": float(d.abs().max().item()),
        "mean_abs": float(d.abs().mean().item()),
        "mse": float(mse.item()),
        "rmse": float(mse.sqrt().item()),
        "rel_l2": float((torch.linalg.vector_norm(d) / e_norm.clamp(min=1e-12)).item()),
        "cosine": float(((a * e).sum() / (torch.linalg.vector_norm(a) * e_norm).clamp(min=1e-12)).item()),
    }
