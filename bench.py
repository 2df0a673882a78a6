"""Benchmark of the MI355X FP8 hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-components] [--no-cpu-baseline]

Prints ONE JSON line. The headline workload is BASELINE.json configs[1]:
per-channel (one scale per row) bf16 -> fp8 e4m3 quantization of an
[18432, 7168] weight. A step is one quantization of that tensor; K steps are
captured back to back in a HIP graph over 4 rotating input/output sets
(1.6 GB, far beyond the 256 MB MALL, so every step streams from HBM) and
timed with HIP events on the stream the kernels run on. Inputs are resident
in HBM before the timed region starts.

``components`` reports the other BASELINE configs the same way (1x128 quant,
128x128 quant, config 2's weight with one scale per column, the block-scaled
BMM of config 4 and the config-5 GEMM trio). ``cpu_baseline`` times the
reference's PyTorch CPU path on the host cores: the eager form of the same
quantizer (the lead value), the oracle's C restatement (OpenMP) beside it,
and fp32 torch.bmm / torch.mm of dequantized operands for configs 4 and 5.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
# the kernel pcamd_quant_channel launches for the headline workload (rows of
# 7168 bf16 elements: one 256-thread workgroup per row, up to 4 chunks per thread)
HEADLINE_KERNEL = "quant_rowblock_kernel<bf16,e4m3,4,nt,grid2,noclamp> (256 threads)"
FP8_PEAK_TFLOPS = 5000.0     # MI355X dense fp8 MFMA (5.0 PFLOP/s)
SETTLE_MS = 100.0            # untimed load before the first (headline) measurement
# the kernels configs 4 and 5 launch (as rocprofv3 names them), to match the
# committed counter summary (profiles/pmc_bmm.json) to the code that runs now
CONFIG4_KERNEL = "pcamd::bmms::bmm_stream_kernel<3>"
# template arguments: A K-major, B K-major, A / B fp8 formats, scale mode, B-scale kind,
# sub-tiles per wave, ragged K, transposed output (wgrad: 256 x 224 tiles of C^T)
CONFIG5_KERNELS = {"fwd_a_k_b_k": ("fwd", ["pcamd::bmmw::bmm_wide_kernel<true, true, 3, 3, 0, 0, 8, false, false>"]),
                   "dgrad_a_k_b_n": ("dgrad",
                                     ["pcamd::bmmw::bmm_wide_kernel<true, false, 3, 3, 0, 0, 8, false, false>"]),
                   "wgrad_a_m_b_n": ("wgrad_a_m_b_n",
                                     ["pcamd::bmmw::bmm_wide_kernel<false, false, 3, 3, 0, 2, 7, false, true>"])}


def pmc_field(workload, kernels, keys):
    """Sum of `keys` of one workload in profiles/pmc_bmm.json (rocprofv3
    counter passes), or None when that file is missing or was taken on
    other kernels than `kernels` (a str or a list of names)."""
    path = os.path.join(ROOT, "profiles", "pmc_bmm.json")
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        rec = json.load(fh).get("workloads", {}).get(workload)
    want = sorted([kernels] if isinstance(kernels, str) else kernels)
    if not rec or sorted(rec.get("kernels", [])) != want:
        return None
    vals = [rec.get(k) for k in (keys if isinstance(keys, tuple) else (keys,))]
    return None if any(v is None for v in vals) else sum(vals)


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-components", action="store_true")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--components-only", default="", help="comma list of component names")
    p.add_argument("--pmc-probe-bmm", action="store_true",
                   help="eager launches for rocprofv3 --pmc passes: 3 plain bf16 copies of 256 MiB, then 3 "
                        "each of config 4 and the config-5 forward, dgrad, wgrad and layer wgrad")
    p.add_argument("--pmc-probe-fused", action="store_true",
                   help="eager launches for rocprofv3 --pmc passes: 3 plain bf16 copies of 256 MiB, then 3 "
                        "fused quant-A BMMs each at N = 128 and N = 256 (M = 32768, K = 4096)")
    p.add_argument("--pmc-probe", action="store_true",
                   help="eager launches for rocprofv3 --pmc passes: 3 plain bf16 copies of "
                        "256 MiB (calibration) then 3 config-2 quantizations")
    p.add_argument("--mem-ceiling", action="store_true",
                   help="graph-timed torch copy / conversion / fill kernels with the traffic mixes of the "
                        "workloads (one JSON line): what plain memory-bound kernels reach on this GPU")
    p.add_argument("--gemm-ref", choices=["graph", "eager"], default=None,
                   help="the config-5 GEMM shapes with tensor and row/column scales, this build's kernels "
                        "next to hipBLASLt (torch._scaled_mm): 'graph' times them (HIP graphs, one JSON "
                        "line), 'eager' launches each 3 times for rocprofv3 passes")
    p.add_argument("--published", choices=["graph", "eager"], default=None,
                   help="the reference's 31 published per-tensor fp8 BMM shapes (fp16 C + fp16 bias, "
                        "B N-major / K-major as published): 'graph' times them (one JSON line), 'eager' "
                        "launches each 3 times for rocprofv3")
    p.add_argument("--fused", action="store_true",
                   help="the fused activation-quant BMM (pcamd_bmm_quant_a) against quantize-then-multiply, "
                        "bf16 A [M, 4096] x e4m3 B [4096, N] 128x128-scaled, over N (one JSON line)")
    p.add_argument("--repack", action="store_true",
                   help="the transpose variants' operand copy at the config-5 shapes: torch's strided "
                        "copy (the reference's .contiguous()) next to pcamd_repack_fp8 (one JSON line)")
    return p.parse_args()


# ---------------------------------------------------------------------------
# timing helpers
# ---------------------------------------------------------------------------
def graph_time(torch, launch, steps: int, warmup: int, reps: int = 5, settle_ms: float = 0.0):
    """Capture `steps` calls of launch(i) into one HIP graph and time `reps`
    replays (the reference's benchmark_cuda takes the median of 5 repeats,
    utils.py:52-84).

    settle_ms: before the warmup launches, keep launching the same work,
    untimed, for about that long. The GPU's clocks take tens of milliseconds
    of load to settle after start-up; the first kernel timed in a fresh process
    otherwise reads a few percent slow.

    Returns (median ms per step over the replays, list of per-replay ms)."""
    if settle_ms > 0:
        t_end = time.perf_counter() + settle_ms / 1000.0
        i = 0
        while time.perf_counter() < t_end:
            for _ in range(64):
                launch(i)
                i += 1
            torch.cuda.synchronize()
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            launch(i)
    g.replay()  # untimed replay: first-touch of the graph itself
    torch.cuda.synchronize()
    samples = []
    for _ in range(reps):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        g.replay()
        end.record()
        torch.cuda.synchronize()
        samples.append(start.elapsed_time(end) / steps)
    return statistics.median(samples), samples


# ---------------------------------------------------------------------------
# inputs (CPU generator seeded 0, then copied to HBM)
# ---------------------------------------------------------------------------
def make_config1(torch):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4096, 7168, generator=g)
    m = torch.rand(4096, 7168, generator=g) < 0.001
    x[m] *= 50
    return x.bfloat16()


def make_config2(torch):
    g = torch.Generator().manual_seed(0)
    return (torch.randn(18432, 7168, generator=g) * 0.02).bfloat16()


def make_config3(torch):
    g = torch.Generator().manual_seed(0)
    w = torch.randn(4096, 7168, generator=g) * 0.02
    mult = torch.exp(torch.empty(32, 56).uniform_(math.log(0.1), math.log(10.0), generator=g))
    return (w * mult.repeat_interleave(128, 0).repeat_interleave(128, 1)).bfloat16()


def rotate_sets(torch, x_cpu, nsets, dev):
    """nsets distinct device copies of the input (first one exact, the others
    perturbed in the last mantissa bit so no two sets share cache lines)."""
    sets = []
    for i in range(nsets):
        x = x_cpu.to(dev)
        if i:
            x.view(torch.int16).bitwise_xor_(i & 1)
        sets.append(x)
    return sets


# ---------------------------------------------------------------------------
# quantizer workloads through the C ABI with preallocated outputs
# ---------------------------------------------------------------------------
def quant_channel_launcher(torch, L, xs, ys, ss):
    def launch(i):
        x, y, s = xs[i % len(xs)], ys[i % len(ys)], ss[i % len(ss)]
        rc = L.lib().pcamd_quant_channel(
            L.ptr(x), L.BF16, 1, x.shape[0], x.shape[1], 0, x.stride(0), 1,
            L.ptr(y), L.E4M3FN, 0, y.stride(0), 1, L.ptr(s), 0, 1, -2, 448.0, 1e-12,
            L.stream_of(x))
        L.check(rc, "pcamd_quant_channel")
    return launch


def quant_columns_launcher(torch, L, xs, ys, ss):
    def launch(i):
        x, y, s = xs[i % len(xs)], ys[i % len(ys)], ss[i % len(ss)]
        rc = L.lib().pcamd_quant_channel(
            L.ptr(x), L.BF16, 1, x.shape[0], x.shape[1], 0, x.stride(0), 1,
            L.ptr(y), L.E4M3FN, 0, y.stride(0), 1, L.ptr(s), 0, 1, -1, 448.0, 1e-12,
            L.stream_of(x))
        L.check(rc, "pcamd_quant_channel")
    return launch


def quant_block_launcher(torch, L, xs, ys, ss, bm, bn):
    def launch(i):
        x, y, s = xs[i % len(xs)], ys[i % len(ys)], ss[i % len(ss)]
        rc = L.lib().pcamd_quant_block(
            L.ptr(x), L.BF16, 1, x.shape[0], x.shape[1], 0, x.stride(0), 1,
            L.ptr(y), L.E4M3FN, 0, y.stride(0), 1, L.ptr(s), 0, s.stride(0), 1,
            bm, bn, 448.0, 1e-12, L.stream_of(x))
        L.check(rc, "pcamd_quant_block")
    return launch


def quant_dual_launcher(torch, L, xs, yrs, ycs, srs, scs):
    def launch(i):
        x = xs[i % len(xs)]
        yr, yc, sr, sc = yrs[i % len(yrs)], ycs[i % len(ycs)], srs[i % len(srs)], scs[i % len(scs)]
        rc = L.lib().pcamd_quant_block_dual(
            L.ptr(x), L.BF16, 1, x.shape[0], x.shape[1], 0, x.stride(0), 1,
            L.ptr(yr), 0, yr.stride(0), 1, L.ptr(yc), 0, 1, x.shape[0], L.E4M3FN,
            L.ptr(sr), 0, sr.stride(0), 1, L.ptr(sc), 0, sc.stride(0), 1, 128, 448.0, 1e-12,
            L.stream_of(x))
        L.check(rc, "pcamd_quant_block_dual")
    return launch


def bench_quant_dual(torch, name, x_dev, steps, warmup, nsets, dev):
    """1x128 and 128x1 quantization of one bf16 [m, n] tensor in one kernel, the
    128x1 result stored transposed (as the training layer keeps it)."""
    from practice_cuda_amd import _lib as L
    m, n = x_dev.shape
    xs = [x_dev] + [x_dev.view(torch.int16).bitwise_xor(i & 1).view(torch.bfloat16) for i in range(1, nsets)]
    yrs = [torch.empty(m, n, dtype=torch.float8_e4m3fn, device=dev) for _ in range(nsets)]
    ycs = [torch.empty(n, m, dtype=torch.float8_e4m3fn, device=dev) for _ in range(nsets)]  # 128x1 stored transposed
    srs = [torch.empty(m, n // 128, dtype=torch.float32, device=dev) for _ in range(nsets)]
    scs = [torch.empty(m // 128, n, dtype=torch.float32, device=dev) for _ in range(nsets)]
    ms, samples = graph_time(torch, quant_dual_launcher(torch, L, xs, yrs, ycs, srs, scs), steps, warmup)
    nbytes = m * n * 2 + 2 * m * n + 4 * (m * (n // 128) + (m // 128) * n)
    gbs = nbytes / (ms * 1e-3) / 1e9
    del xs, yrs, ycs, srs, scs
    torch.cuda.empty_cache()
    return {"name": name, "ms_per_step": ms, "bytes_per_step": nbytes, "value": gbs, "unit": "GB/s",
            "frac_of_hbm_peak": gbs / HBM_PEAK_GBS}


def bench_quant(torch, name, x_cpu, kind, steps, warmup, nsets, dev, bm=1, bn=128, settle_ms=0.0):
    from practice_cuda_amd import _lib as L
    m, n = x_cpu.shape
    xs = rotate_sets(torch, x_cpu, nsets, dev)
    ys = [torch.empty(m, n, dtype=torch.float8_e4m3fn, device=dev) for _ in range(nsets)]
    if kind == "channel":
        ss = [torch.empty(m, dtype=torch.float32, device=dev) for _ in range(nsets)]
        launch = quant_channel_launcher(torch, L, xs, ys, ss)
        scale_bytes = m * 4
    elif kind == "columns":
        ss = [torch.empty(n, dtype=torch.float32, device=dev) for _ in range(nsets)]
        launch = quant_columns_launcher(torch, L, xs, ys, ss)
        scale_bytes = n * 4
    else:
        mb, nb = -(-m // bm), -(-n // bn)
        ss = [torch.empty(mb, nb, dtype=torch.float32, device=dev) for _ in range(nsets)]
        launch = quant_block_launcher(torch, L, xs, ys, ss, bm, bn)
        scale_bytes = mb * nb * 4
    ms, samples = graph_time(torch, launch, steps, warmup, settle_ms=settle_ms)
    nbytes = m * n * 2 + m * n + scale_bytes
    gbs = nbytes / (ms * 1e-3) / 1e9
    del xs, ys, ss
    torch.cuda.empty_cache()
    return {"name": name, "ms_per_step": ms, "samples_ms": samples, "bytes_per_step": nbytes,
            "value": gbs, "unit": "GB/s", "frac_of_hbm_peak": gbs / HBM_PEAK_GBS}


# ---------------------------------------------------------------------------
# BMM workloads
# ---------------------------------------------------------------------------
def config4_launcher(torch, dev, nsets):
    """BASELINE config 4 over nsets rotating operand / output sets: launch(i)
    runs the block-scaled BMM on set i % nsets through the C ABI."""
    from practice_cuda_amd import _lib as L
    from practice_cuda_amd.impls.hip_per_block import hip_per_block_quant
    g = torch.Generator().manual_seed(0)
    ah = torch.randn(128, 2048, 128, generator=g).bfloat16().to(dev)
    bh = torch.randn(128, 128, 512, generator=g).bfloat16().to(dev)
    qas, qbs, outs = [], [], []
    for i in range(nsets):
        qa = hip_per_block_quant(ah if i == 0 else ah * (1 + i / 64), block_m=1, block_n=128)
        qb = hip_per_block_quant(bh, block_m=128, block_n=128)
        qas.append(qa), qbs.append(qb)
        outs.append(torch.empty(128, 2048, 512, dtype=torch.bfloat16, device=dev))

    def launch(i):
        qa, qb, c = qas[i % nsets], qbs[i % nsets], outs[i % nsets]
        a, b, sa, sb = qa.tensor, qb.tensor, qa.dequant_scale, qb.dequant_scale
        rc = L.lib().pcamd_bmm_scaled(
            L.ptr(a), L.ptr(b), L.E4M3FN, 128, 2048, 512, 128, *a.stride(), *b.stride(),
            L.ptr(c), L.BF16, *c.stride(), None, 0, 0, 0, 0,
            L.ptr(sa), *sa.stride(), L.ptr(sb), *sb.stride(),
            L.SCALE_BLOCK, 0, 1, 128, 128, L.ACT_NONE, L.stream_of(c))
        L.check(rc, "pcamd_bmm_scaled")

    return launch


def bench_config4(torch, steps, warmup, dev, nsets=4):
    launch = config4_launcher(torch, dev, nsets)
    # ~100 ms of untimed launches first: the clocks settle under this load
    # (without it the five replays of a cold start fall from ~58 to ~50 us)
    ms, samples = graph_time(torch, launch, steps, warmup, settle_ms=SETTLE_MS)
    flops = 2 * 128 * 2048 * 512 * 128
    nbytes = 128 * 2048 * 128 + 128 * 128 * 512 + 128 * 2048 * 512 * 2 + 128 * 2048 * 4 + 128 * 4 * 4
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = nbytes / (ms * 1e-3) / 1e9
    attainable = min(FP8_PEAK_TFLOPS, HBM_PEAK_GBS * flops / nbytes / 1e3)
    return {"name": "config4_block_bmm_b128_m2048_n512_k128", "ms_per_step": ms, "samples_ms": samples,
            "value": tflops, "unit": "TFLOP/s", "frac_of_fp8_peak": tflops / FP8_PEAK_TFLOPS,
            "hbm_GBps": gbs, "frac_of_hbm_peak": gbs / HBM_PEAK_GBS,
            "frac_of_attainable_roofline": tflops / attainable, "bytes_per_step": nbytes,
            "flops_per_step": flops,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "kernel": CONFIG4_KERNEL,
                         "traffic": pmc_field("config4", CONFIG4_KERNEL, ("fetch_bytes", "write_bytes"))}}


CONFIG5_DIMS = (8192, 4096, 14336)  # M (tokens), K (in features), N (out features)
CONFIG5_SETS = 4  # rotating GEMM operand sets: 4 x 92-176 MB, beyond the 256 MB MALL


def config5_inputs(torch):
    """BASELINE config 5 inputs on the host, CPU generator seed 0, in this
    order: X [M, K] ~ N(0, 1), W [N, K] ~ N(0, 0.02), dY [M, N] ~ N(0, 1e-3),
    all bf16. The GPU parity tests draw the same tensors."""
    M, K, N = CONFIG5_DIMS
    g = torch.Generator().manual_seed(0)
    X = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    dY = (torch.randn(M, N, generator=g) * 1e-3).bfloat16()
    return X, W, dY


def config5_operands(torch, dev):
    """BASELINE config 5 (M=8192 K=4096 N=14336), CPU generator seed 0:
    the bf16 tensors and their block quantizations."""
    from practice_cuda_amd.impls.hip_per_block import hip_per_block_quant
    M, K, N = CONFIG5_DIMS
    X, W, dY = (t.to(dev) for t in config5_inputs(torch))
    q = {
        "x": hip_per_block_quant(X[None], block_m=1, block_n=128),      # [1, M, K] 1x128
        "w": hip_per_block_quant(W[None], block_m=128, block_n=128),    # [1, N, K] 128x128
        "dy": hip_per_block_quant(dY[None], block_m=1, block_n=128),    # [1, M, N] 1x128
        "dy_m": hip_per_block_quant(dY[None], block_m=128, block_n=1),  # [1, M, N] 128x1
        "x_m": hip_per_block_quant(X[None], block_m=128, block_n=1),    # [1, M, K] 128x1
    }
    return (M, K, N), (X, W, dY), q


def quant_copy(r):
    """The same QuantResult in storage of its own (same bytes, same strides)."""
    import torch
    from practice_cuda_amd.registry import QuantResult

    def like(t):
        c = torch.empty_strided(t.shape, t.stride(), dtype=t.dtype, device=t.device)
        c.copy_(t)
        return c
    return QuantResult(like(r.tensor), like(r.dequant_scale), r.impl, r.granularity, dict(r.meta))


def config5_gemms(torch, dev, q, dims, nsets=1):
    """The trio (fwd X W^T a_k_b_k, dgrad dY W a_k_b_n, wgrad dY^T X a_m_b_n
    with the 128x1 requant) as launch closures over preallocated outputs;
    launch(i) uses operand set i % nsets (set 0 is q, the others copies of
    it in storage of their own, so that nsets > 2 keeps the operands from
    staying in the 256 MB MALL between launches)."""
    from practice_cuda_amd.impls.hip_per_block import hip_per_block_bmm
    from practice_cuda_amd.registry import QuantResult
    M, K, N = dims

    def tr(r: QuantResult, bm, bn):
        # logical transpose of the last two dims (a strided view) with its scales
        return QuantResult(r.tensor.transpose(-1, -2), r.dequant_scale.transpose(-1, -2), r.impl,
                           "block", {"block_m": bn, "block_n": bm})

    sets = [q] + [{k: quant_copy(v) for k, v in q.items()} for _ in range(nsets - 1)]
    ops = [{"x": s["x"], "wt": tr(s["w"], 128, 128), "w": s["w"], "dy": s["dy"],
            "dyt": tr(s["dy_m"], 128, 1), "x_m": s["x_m"]} for s in sets]
    out_f = [torch.empty(1, M, N, dtype=torch.bfloat16, device=dev) for _ in range(nsets)]
    out_d = [torch.empty(1, M, K, dtype=torch.bfloat16, device=dev) for _ in range(nsets)]
    out_w = [torch.empty(1, N, K, dtype=torch.bfloat16, device=dev) for _ in range(nsets)]
    gemms = {
        "fwd_a_k_b_k": lambda i: hip_per_block_bmm(ops[i % nsets]["x"], ops[i % nsets]["wt"], out=out_f[i % nsets]),
        "dgrad_a_k_b_n": lambda i: hip_per_block_bmm(ops[i % nsets]["dy"], ops[i % nsets]["w"], out=out_d[i % nsets]),
        "wgrad_a_m_b_n": lambda i: hip_per_block_bmm(ops[i % nsets]["dyt"], ops[i % nsets]["x_m"],
                                                     out=out_w[i % nsets]),
    }
    return gemms, ops, (out_f, out_d, out_w)


def bench_config5(torch, steps, warmup, dev, nsets=CONFIG5_SETS):
    """FP8 training-linear GEMM trio at M=8192 K=4096 N=14336: fwd X W^T
    (a_k_b_k), dgrad dY W (a_k_b_n), wgrad dY^T X (a_m_b_n, 128x1 requant),
    each over nsets rotating operand sets (beyond the MALL)."""
    from practice_cuda_amd.impls.hip_per_block import hip_per_block_bmm
    from practice_cuda_amd.registry import QuantResult
    dims, (X, W, dY), q = config5_operands(torch, dev)
    M, K, N = dims
    gemms, ops, (out_f, out_d, out_w) = config5_gemms(torch, dev, q, dims, nsets)
    flops = 2 * M * N * K
    res = {}
    for name, fn in gemms.items():
        ms, samples = graph_time(torch, fn, steps, warmup)
        t = flops / (ms * 1e-3) / 1e12
        res[name] = {"ms": ms, "TFLOP/s": t, "frac_of_fp8_peak": t / FP8_PEAK_TFLOPS}
    total_ms = sum(r["ms"] for r in res.values())
    # the training layer's wgrad: the same product on K-major operands (its
    # dual quantizer stores the 128x1 results transposed); not part of the trio
    lay = [(QuantResult(o["dyt"].tensor.contiguous(), o["dyt"].dequant_scale, o["dyt"].impl, "block",
                        dict(o["dyt"].meta)),
            QuantResult(o["x_m"].tensor.transpose(-1, -2).contiguous().transpose(-1, -2), o["x_m"].dequant_scale,
                        o["x_m"].impl, "block", dict(o["x_m"].meta))) for o in ops]
    ms, _ = graph_time(torch, lambda i: hip_per_block_bmm(*lay[i % nsets], out=out_w[i % nsets]), steps, warmup)
    t = flops / (ms * 1e-3) / 1e12
    res["wgrad_layer_a_k_b_k"] = {"ms": ms, "TFLOP/s": t, "frac_of_fp8_peak": t / FP8_PEAK_TFLOPS,
                                  "note": "not in the trio total"}
    del lay
    # the channel-scaled recipe (one scale per row of X and of W) on the forward shape
    from practice_cuda_amd.impls.hip_per_channel import hip_per_channel_bmm, hip_per_channel_quant
    cx = hip_per_channel_quant(X[None], channel_axis=-2)
    cw = hip_per_channel_quant(W[None], channel_axis=-2)
    cwt = QuantResult(cw.tensor.transpose(-1, -2), cw.dequant_scale, cw.impl, "channel",
                      {**cw.meta, "channel_axis": -1})
    chan = [(cx, cwt)] + [(quant_copy(cx), quant_copy(cwt)) for _ in range(nsets - 1)]
    ms, _ = graph_time(torch, lambda i: hip_per_channel_bmm(*chan[i % nsets], out=out_f[i % nsets]), steps, warmup)
    t = flops / (ms * 1e-3) / 1e12
    res["fwd_channel_a_k_b_k"] = {"ms": ms, "TFLOP/s": t, "frac_of_fp8_peak": t / FP8_PEAK_TFLOPS,
                                  "note": "channel scales (per-channel recipe); not in the trio total"}
    # the trio with one operand set, for comparison: its operands stay in the MALL
    res_mall = {}
    g1, _, _ = config5_gemms(torch, dev, q, dims, 1)
    for name, fn in g1.items():
        ms, _ = graph_time(torch, fn, steps, warmup)
        res_mall[name] = ms
    del g1, cx, cw, cwt, chan
    tflops = 3 * flops / (total_ms * 1e-3) / 1e12
    del ops, out_f, out_d, out_w, gemms, q
    torch.cuda.empty_cache()
    # the layer step's quantization launches: X and dY each quantized 1x128
    # and 128x1 by one kernel, W 128x128
    quants = [bench_quant_dual(torch, "x_dual_1x128_128x1", X, steps, warmup, 4, dev),
              bench_quant_dual(torch, "dy_dual_1x128_128x1", dY, steps, warmup, 4, dev),
              bench_quant(torch, "w_128x128", W.cpu(), "block", steps, warmup, 4, dev, bm=128, bn=128)]
    for q in quants:
        q.pop("samples_ms", None)
    layer = layer_step(torch, X, W, dY, steps, dev)
    layer["TFLOP/s"] = 3 * flops / (layer["ms"] * 1e-3) / 1e12
    # roofline of the trio: MFMA-bound; busy fractions from the committed
    # counter passes when they were taken on the kernels that run now
    busy = {name: pmc_field(wl, ks, "mfma_busy") for name, (wl, ks) in CONFIG5_KERNELS.items()}
    roof = {"bound": "mfma", "achieved": tflops, "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tflops / FP8_PEAK_TFLOPS, "flops_per_gemm": flops,
            "kernels": {name: ks for name, (_, ks) in CONFIG5_KERNELS.items()},
            "mfma_busy": busy if all(v is not None for v in busy.values()) else None}
    return {"name": "config5_training_linear_m8192_k4096_n14336", "ms_per_step": total_ms,
            "value": tflops, "unit": "TFLOP/s", "frac_of_fp8_peak": tflops / FP8_PEAK_TFLOPS,
            "operand_sets": nsets, "gemms": res, "gemms_one_operand_set_ms": res_mall,
            "flops_per_step": 3 * flops, "roofline": roof, "quant": quants, "layer_step": layer}


def layer_step(torch, X, W, dY, steps, dev):
    """Forward + backward of Float8BMMLinear at the config-5 shape: three fp8
    quantization launches (X 1x128 + 128x1 in one kernel, W 128x128, dY
    1x128 + 128x1 in one kernel) and the three GEMMs, eager (autograd).

    Timed with events in blocks of five steps, alternating with blocks of the
    same six launches issued without autograd (layer_sequence), so that both
    see the same clocks; `ms` and `sequence_ms` are the medians over the
    blocks. `per_op_ms`: each launch of the sequence bracketed by its own
    events over `steps` steps, all recorded before one synchronize (the host
    stays ahead of the GPU, so no launch waits for it)."""
    from practice_cuda_amd.modules import Float8BMMLinear
    layer = Float8BMMLinear(1, X.shape[1], W.shape[0], bias=False, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        layer.weight.copy_(W[None])
    xg = X[None].detach().requires_grad_(True)
    dy = dY[None]

    def step():
        layer.weight.grad = None
        xg.grad = None
        layer(xg).backward(dy)

    seq, names = layer_sequence(torch, X, W, dY)

    def block(fn, n=5):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(n):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / n

    for _ in range(5):
        step()
        seq()
    torch.cuda.synchronize()
    auto, bare = [], []
    for _ in range(max(2, steps // 5)):
        auto.append(block(step))
        bare.append(block(seq))
    evs = []
    for _ in range(steps):
        ev = {n: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for n in names}
        seq(ev)
        evs.append(ev)
    torch.cuda.synchronize()
    per_op = {n: statistics.median(ev[n][0].elapsed_time(ev[n][1]) for ev in evs) for n in names}
    return {"ms": statistics.median(auto), "sequence_ms": statistics.median(bare), "per_op_ms": per_op,
            "per_op_sum_ms": sum(per_op.values()),
            "what": "Float8BMMLinear forward + backward, 3 quantization launches (X and dY each 1x128 + 128x1 "
                    "in one kernel, W 128x128) + 3 GEMMs, eager; sequence: the same launches without autograd"}


def layer_sequence(torch, X, W, dY):
    """The layer step's six launches in its own order: the custom ops its
    autograd function calls, with the same arguments. Returns (seq, names):
    seq(ev=None) issues them, recording ev[name] = (start, end) events around
    each when given."""
    ops = torch.ops.pcamd
    f8, blk, eps = torch.float8_e4m3fn, 128, 1e-12
    x, w, dy = X[None], W[None], dY[None]
    names = ["quant_x_dual", "quant_w_128x128", "fwd_gemm", "quant_dy_dual", "dgrad_gemm", "wgrad_gemm"]

    def seq(ev=None):
        out = {}

        def mark(name, fn):
            if ev is not None:
                ev[name][0].record()
            out[name] = fn()
            if ev is not None:
                ev[name][1].record()
        mark("quant_x_dual", lambda: ops.quant_block_dual(x, blk, f8, eps))
        mark("quant_w_128x128", lambda: ops.quant_block(w, blk, blk, f8, eps))
        qx, sx, qxm, sxm = out["quant_x_dual"]
        qw, sw = out["quant_w_128x128"]
        mark("fwd_gemm", lambda: ops.block_scaled_bmm(qx, sx, qw.transpose(-2, -1), sw.transpose(-2, -1), None,
                                                      1, blk, blk, x.dtype))
        mark("quant_dy_dual", lambda: ops.quant_block_dual(dy, blk, f8, eps))
        qdy, sdy, qdt, sdt = out["quant_dy_dual"]
        mark("dgrad_gemm", lambda: ops.block_scaled_bmm(qdy, sdy, qw, sw, None, 1, blk, blk, dy.dtype))
        mark("wgrad_gemm", lambda: ops.block_scaled_bmm(qdt.transpose(-2, -1), sdt.transpose(-2, -1), qxm, sxm,
                                                        None, 1, blk, 1, dy.dtype))
    return seq, names


# ---------------------------------------------------------------------------
# CPU baseline: the reference's PyTorch CPU path on the host cores
# ---------------------------------------------------------------------------
def host_cpu():
    """(threads to use, facts about the host). The thread count is the
    process's CPU share: OMP_NUM_THREADS when the host sets it (the GPU boxes
    here set it to the cores granted per GPU), else every core this process
    may run on."""
    model = None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    threads = max(1, min(int(env), usable)) if env.isdigit() and int(env) > 0 else usable
    return threads, {"os_cpu_count": os.cpu_count(), "usable_cpus": usable, "cpu_model": model,
                     "omp_num_threads_env": env or None,
                     "threads_rule": "OMP_NUM_THREADS if set (the host's per-GPU CPU share), "
                                     "else every usable core"}


def cpu_baseline(torch, x_cpu, dev):
    """The lead value is the reference's PyTorch form of the headline
    quantizer (kernels/quant/per_channel.py:9-29, fp32 math) run eagerly on
    the host cores over the full config-2 tensor. Beside it: the oracle's C
    restatement with OpenMP, BASELINE configs[0] (1x128 groups, eager
    PyTorch), and the BMM configs through the reference's kernel_reference
    (fp8_training/fp8_bench/bench_bmm.py:414-416: fp32 torch.bmm / torch.mm of
    the dequantized operands)."""
    from oracle import oracle as O
    threads, host = host_cpu()
    torch.set_num_threads(threads)
    sample = x_cpu.contiguous()                 # the full workload tensor
    lead = torch_eager_baseline(torch, sample, threads)
    O.quant_channel(sample[:64], -2, threads=threads)   # warm (page-in, thread pool)
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        O.quant_channel(sample, -2, threads=threads)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    m, n = sample.shape
    nbytes = m * n * 3 + m * 4
    oracle_c = {"value": nbytes / t / 1e9, "unit": "GB/s", "threads": threads,
                "sample": f"bf16 [{m},{n}], median of 5 runs of oracle/fp8_oracle.c per-row quant "
                          f"(OpenMP), {t * 1e3:.1f} ms/run"}
    torch.set_num_threads(threads)  # the oracle call sets the process's OpenMP thread count too
    out = {"value": lead["value"], "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
           "sample": lead["sample"], "matches_oracle": lead["matches_oracle"], "host": host,
           "torch_threads": torch.get_num_threads(), "oracle_c": oracle_c,
           "config0": config0_baseline(torch, threads)}
    torch.set_num_threads(threads)
    out["config4_bmm"] = cpu_bmm_config4(torch, dev)
    out["config5_gemms"] = cpu_gemms_config5(torch, dev)
    return out


def cpu_bmm_config4(torch, dev):
    """BASELINE config 4 through kernel_reference on the host cores: fp32
    torch.bmm of the dequantized [128,2048,128] x [128,128,512] operands
    (quantized by this build's kernels on the GPU, then copied over), 1 warmup
    and the median of 3 runs; checked against the GPU kernel's output."""
    from practice_cuda_amd.impls.hip_per_block import hip_per_block_bmm, hip_per_block_quant
    g = torch.Generator().manual_seed(0)
    ah = torch.randn(128, 2048, 128, generator=g).bfloat16()
    bh = torch.randn(128, 128, 512, generator=g).bfloat16()
    qa = hip_per_block_quant(ah.to(dev), block_m=1, block_n=128)
    qb = hip_per_block_quant(bh.to(dev), block_m=128, block_n=128)
    gpu = hip_per_block_bmm(qa, qb).float().cpu()
    a, b = qa.dequantize().cpu(), qb.dequantize().cpu()
    ref = torch.bmm(a, b)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        torch.bmm(a, b)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    flops = 2 * 128 * 2048 * 512 * 128
    err = ((gpu - ref).abs().max() / ref.abs().max()).item()
    return {"value": flops / t / 1e12, "unit": "TFLOP/s", "ms": t * 1e3, "threads": torch.get_num_threads(),
            "gpu_max_abs_rel": err,
            "sample": "the full config-4 product, fp32 torch.bmm of dequantized operands, median of 3 runs"}


def cpu_gemms_config5(torch, dev):
    """The config-5 GEMM trio through kernel_reference on the host cores: three
    fp32 torch.mm of dequantized operands at M=8192 K=4096 N=14336, one run
    each (about a second per GEMM on 16 cores), each checked against the GPU
    kernel's output."""
    from practice_cuda_amd.impls.hip_per_block import hip_per_block_bmm, hip_per_block_quant
    from practice_cuda_amd.registry import QuantResult
    M, K, N = 8192, 4096, 14336
    g = torch.Generator().manual_seed(0)
    X = torch.randn(M, K, generator=g).bfloat16().to(dev)[None]
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16().to(dev)[None]
    dY = (torch.randn(M, N, generator=g) * 1e-3).bfloat16().to(dev)[None]

    def tr(q):
        return QuantResult(q.tensor.transpose(-1, -2), q.dequant_scale.transpose(-1, -2), q.impl, "block",
                           {**q.meta, "block_m": q.meta["block_n"], "block_n": q.meta["block_m"]})

    qx = hip_per_block_quant(X, block_m=1, block_n=128)
    qw = hip_per_block_quant(W, block_m=128, block_n=128)
    qdy = hip_per_block_quant(dY, block_m=1, block_n=128)
    qdy_m = hip_per_block_quant(dY, block_m=128, block_n=1)
    qx_m = hip_per_block_quant(X, block_m=128, block_n=1)
    cases = {"fwd": (qx, tr(qw)), "dgrad": (qdy, qw), "wgrad": (tr(qdy_m), qx_m)}
    res, total = {}, 0.0
    for name, (qa, qb) in cases.items():
        gpu = hip_per_block_bmm(qa, qb)[0].float().cpu()
        a = qa.dequantize()[0].contiguous().cpu()
        b = qb.dequantize()[0].contiguous().cpu()
        t0 = time.perf_counter()
        ref = torch.mm(a, b)
        t = time.perf_counter() - t0
        total += t
        err = ((gpu - ref).abs().max() / ref.abs().max()).item()
        res[name] = {"ms": t * 1e3, "TFLOP/s": 2 * M * N * K / t / 1e12, "gpu_max_abs_rel": err}
        del gpu, a, b, ref
    return {"value": 3 * 2 * M * N * K / total / 1e12, "unit": "TFLOP/s", "threads": torch.get_num_threads(),
            "gemms": res, "sample": "fwd, dgrad and wgrad at the full config-5 shape, fp32 torch.mm of "
                                    "dequantized operands, one run each"}


def torch_channel_quant(torch, x, fp8_max=448.0, eps=1e-12):
    """The reference's PyTorch form of the per-row quantizer
    (kernels/quant/per_channel.py:9-29, channel_axis=-2): fp32 math, amax
    per row, s = max(amax, eps), q = fp8(clamp(x * (fp8_max / s))), scale
    s / fp8_max. fp8_max / s is a true fp32 division, as in the reference's
    Triton kernels and its compiled form; eager `float / tensor` would
    compute reciprocal(s) * fp8_max, which differs in the last bit for some
    s."""
    xf = x.float()
    s = xf.abs().amax(dim=-1, keepdim=True).clamp(min=eps)
    qs = torch.full_like(s, fp8_max) / s  # a true division (scalar / tensor is reciprocal * scalar)
    q = (xf * qs).clamp(-fp8_max, fp8_max).to(torch.float8_e4m3fn)
    return q, (s / fp8_max).squeeze(-1)


def torch_group_quant(torch, x, group=128, fp8_max=448.0, eps=1e-12):
    """The reference's 1 x 128 group quantizer in eager PyTorch (the math of
    kernels/quant/per_block.py:35-48): per group s = max(amax, eps),
    qs = fp8_max / s, q = fp8(clamp(x * qs)), scale 1 / qs."""
    m, n = x.shape
    xf = x.float().view(m, n // group, group)
    s = xf.abs().amax(dim=-1, keepdim=True).clamp(min=eps)
    qs = torch.full_like(s, fp8_max) / s  # a true division (scalar / tensor is reciprocal * scalar)
    q = (xf * qs).clamp(-fp8_max, fp8_max).to(torch.float8_e4m3fn).view(m, n)
    return q, (1.0 / qs).squeeze(-1)


def config0_baseline(torch, threads):
    """the 1 x 128 quantizer of config 1's input through
    eager PyTorch on the host cores, checked against the oracle."""
    from oracle import oracle as O
    x = make_config1(torch)
    q_ref, s_ref = O.quant_block(x[:64], 1, 128, threads=threads)
    torch.set_num_threads(threads)  # after the oracle call: both set the process's OpenMP thread count
    q, s = torch_group_quant(torch, x[:64])
    same = bool((q.view(torch.uint8).numpy() == q_ref).all() and (s.numpy().view("uint32") == s_ref.view("uint32")).all())
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        torch_group_quant(torch, x)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    m, n = x.shape
    nbytes = m * n * 3 + m * (n // 128) * 4
    return {"value": nbytes / t / 1e9, "unit": "GB/s", "threads": torch.get_num_threads(), "matches_oracle": same,
            "sample": f"BASELINE configs[0]: bf16 [{m},{n}] 1x128 groups, median of 3 runs of the eager-PyTorch "
                      f"group quantizer (fp32 math), {t * 1e3:.1f} ms/run"}


def torch_eager_baseline(torch, sample, threads):
    """The same workload through eager PyTorch on the host cores (the
    reference's CPU path), checked against the oracle on the first rows."""
    from oracle import oracle as O
    q_ref, s_ref = O.quant_channel(sample[:64], -2, threads=threads)
    torch.set_num_threads(threads)  # after the oracle call: both set the process's OpenMP thread count
    q, s = torch_channel_quant(torch, sample[:64])
    same = bool((q.view(torch.uint8).numpy() == q_ref).all() and (s.numpy().view("uint32") == s_ref.view("uint32")).all())
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        torch_channel_quant(torch, sample)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    m, n = sample.shape
    return {"value": (m * n * 3 + m * 4) / t / 1e9, "unit": "GB/s", "threads": torch.get_num_threads(),
            "matches_oracle": same,
            "sample": f"bf16 [{m},{n}], median of 3 runs of the eager-PyTorch per-row quantizer "
                      f"(fp32 math), {t * 1e3:.1f} ms/run"}


def pmc_probe(torch, dev):
    """Known-size copy (calibration), the headline kernel, then configs 1 and
    3 (three dispatches each, rotating inputs), launched eagerly so every
    dispatch carries its own counters."""
    from practice_cuda_amd import _lib as L
    src = torch.ones(1 << 27, dtype=torch.bfloat16, device=dev)  # 256 MiB
    dst = torch.empty_like(src)
    x2 = make_config2(torch)
    xs = rotate_sets(torch, x2, 3, dev)
    ys = [torch.empty(x2.shape, dtype=torch.float8_e4m3fn, device=dev) for _ in range(3)]
    ss = [torch.empty(x2.shape[0], dtype=torch.float32, device=dev) for _ in range(3)]
    launch = quant_channel_launcher(torch, L, xs, ys, ss)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    for i in range(3):
        launch(i)
    torch.cuda.synchronize()
    del xs, ys, ss
    out = {"copy_bytes_read": src.numel() * 2, "copy_bytes_written": dst.numel() * 2,
           "quant_bytes_read": x2.numel() * 2, "quant_bytes_written": x2.numel() + x2.shape[0] * 4}
    for name, make, bm, bn in (("config1", make_config1, 1, 128), ("config3", make_config3, 128, 128)):
        x = make(torch)
        xs = rotate_sets(torch, x, 3, dev)
        ys = [torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=dev) for _ in range(3)]
        ss = [torch.empty(-(-x.shape[0] // bm), -(-x.shape[1] // bn), device=dev) for _ in range(3)]
        launch = quant_block_launcher(torch, L, xs, ys, ss, bm, bn)
        for i in range(3):
            launch(i)
        torch.cuda.synchronize()
        out[name] = {"bytes_read": x.numel() * 2, "bytes_written": x.numel() + ss[0].numel() * 4}
        del xs, ys, ss
    print(json.dumps(out))


def pmc_probe_bmm(torch, dev):
    """Eager launches for rocprofv3 --pmc passes over the BMM kernels, each
    dispatch carrying its own counters: three 256 MiB bf16 copies
    (calibration), then three launches each of config 4 and of the config-5
    forward, dgrad, wgrad (a_m_b_n) and the layer's K-major wgrad, in that
    order."""
    from practice_cuda_amd.impls.hip_per_block import hip_per_block_bmm
    from practice_cuda_amd.registry import QuantResult
    src = torch.ones(1 << 27, dtype=torch.bfloat16, device=dev)  # 256 MiB
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    launch4 = config4_launcher(torch, dev, 3)
    for i in range(3):
        launch4(i)
    torch.cuda.synchronize()
    del launch4
    torch.cuda.empty_cache()
    dims, _, q = config5_operands(torch, dev)
    gemms, ops, outs = config5_gemms(torch, dev, q, dims)
    dyt = ops[0]["dyt"]
    dyt_k = QuantResult(dyt.tensor.contiguous(), dyt.dequant_scale, dyt.impl, "block", dict(dyt.meta))
    qx_m = q["x_m"]
    qx_mk = QuantResult(qx_m.tensor.transpose(-1, -2).contiguous().transpose(-1, -2), qx_m.dequant_scale,
                        qx_m.impl, "block", dict(qx_m.meta))
    gemms["wgrad_layer_a_k_b_k"] = lambda i: hip_per_block_bmm(dyt_k, qx_mk, out=outs[2])
    for name, fn in gemms.items():
        for i in range(3):
            fn(i)
        torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": (1 << 28), "copy_bytes_written": (1 << 28),
                      "order": ["copy x3", "config4 x3"] + [f"{k} x3" for k in gemms]}))


def pmc_probe_fused(torch, dev):
    """Eager launches for rocprofv3 --pmc passes over the streaming fused
    quant-A BMM, each dispatch carrying its own counters: three 256 MiB bf16
    copies (calibration), then three launches each at N = 128 and N = 256 of
    bf16 A [32768, 4096] (two tensors in turn) times e4m3fn B [4096, N],
    128x128 B scales, bf16 C - the shapes of `--fused`."""
    from practice_cuda_amd.impls.hip_per_block import hip_per_block_bmm_quant_a, hip_per_block_quant
    src = torch.ones(1 << 27, dtype=torch.bfloat16, device=dev)  # 256 MiB
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    g = torch.Generator(device=dev).manual_seed(0)
    m, k = 32768, 4096
    xs = [torch.randn(1, m, k, generator=g, device=dev).bfloat16() for _ in range(2)]
    for n in (128, 256):
        qb = hip_per_block_quant((torch.randn(1, k, n, generator=g, device=dev) * 0.02).bfloat16(),
                                 block_m=128, block_n=128)
        out = torch.empty(1, m, n, device=dev, dtype=torch.bfloat16)
        for i in range(3):
            hip_per_block_bmm_quant_a(xs[i % 2], qb, out=out)
        torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": (1 << 28), "copy_bytes_written": (1 << 28),
                      "order": ["copy x3", "fused n=128 x3", "fused n=256 x3"]}))


def mem_ceiling(torch, dev, steps, warmup):
    """What plain memory-bound kernels (PyTorch's own elementwise kernels)
    reach for the read:write mixes of this build's workloads, graph-timed
    like the workloads over rotating buffers beyond the 256 MB MALL:
    - 2:1 (the quantizers): bf16 -> fp8 conversion of [18432, 7168] (config 2's shape);
    - 1:1 (the dual quantizer): bf16 copy of [8192, 14336] (config 5's dY);
    - 0:1 (config 4's output, 268 MB of its 311 MB): bf16 fill of [128, 2048, 512];
    and the 1:1 mix once more with this library's own streaming copy
    (pcamd_selftest_copy16: one 16-byte non-temporal load and store per lane)
    at the shapes of config 5's dY and X, and the 2:1 mix with its own
    narrowing (pcamd_selftest_narrow16: the high byte of each bf16, two
    16-byte loads and then two 8-byte stores per lane, the 1x128
    quantizer's streaming layout) at the shapes of configs 2 and 1."""
    from practice_cuda_amd import _lib as L

    def hip_copy(src, dst):
        L.check(L.lib().pcamd_selftest_copy16(L.ptr(src), L.ptr(dst), src.numel() * src.element_size(),
                                              L.stream_of(src)), "pcamd_selftest_copy16")

    def hip_narrow(src, dst):
        L.check(L.lib().pcamd_selftest_narrow16(L.ptr(src), L.ptr(dst), src.numel() * src.element_size(),
                                                L.stream_of(src)), "pcamd_selftest_narrow16")

    res = {}
    cases = {
        "convert_bf16_to_fp8_18432x7168": ((18432, 7168), lambda src, dst: dst.copy_(src), torch.float8_e4m3fn, 3),
        "copy_bf16_8192x14336": ((8192, 14336), lambda src, dst: dst.copy_(src), torch.bfloat16, 4),
        "fill_bf16_128x2048x512": ((128, 2048, 512), lambda src, dst: dst.zero_(), torch.bfloat16, 2),
        "hip_copy_bf16_8192x14336": ((8192, 14336), hip_copy, torch.bfloat16, 4),
        "hip_copy_bf16_8192x4096": ((8192, 4096), hip_copy, torch.bfloat16, 4),
        "hip_narrow_bf16_18432x7168": ((18432, 7168), hip_narrow, torch.uint8, 3),
        "hip_narrow_bf16_4096x7168": ((4096, 7168), hip_narrow, torch.uint8, 3),
    }
    for name, (shape, op, odt, bpe) in cases.items():
        nsets = 8 if name == "hip_narrow_bf16_4096x7168" else 4  # config 1 is timed over 8 sets too
        srcs = [torch.randn(*shape, device=dev).bfloat16() for _ in range(nsets)] if bpe != 2 else [None] * nsets
        dsts = [torch.empty(*shape, dtype=odt, device=dev) for _ in range(nsets)]
        ms, _ = graph_time(torch, lambda i: op(srcs[i % nsets], dsts[i % nsets]), steps, warmup, settle_ms=SETTLE_MS)
        nbytes = math.prod(shape) * bpe
        res[name] = {"ms": ms, "bytes": nbytes, "GB/s": nbytes / (ms * 1e-3) / 1e9,
                     "frac_of_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        del srcs, dsts
        torch.cuda.empty_cache()
    # per-launch floor: the 1x128 quantizer on one row, back to back in a graph
    tiny = torch.randn(1, 7168, device=dev).bfloat16()
    ty = torch.empty(1, 7168, dtype=torch.float8_e4m3fn, device=dev)
    ts = torch.empty(1, 56, device=dev)
    launch = quant_block_launcher(torch, L, [tiny], [ty], [ts], 1, 128)
    ms, _ = graph_time(torch, launch, steps, warmup)
    res["launch_floor_1x128_one_row"] = {"ms": ms, "note": "one workgroup; the fixed cost of one launch in a graph"}
    print(json.dumps({"mem_ceiling": res}))


def repack_probe(torch, dev, steps, warmup):
    """The copies behind the transpose BMM variants (an M-major A or an
    N-major B made K-major) at the config-5 operand shapes, graph-timed over
    rotating buffers: torch's copy of the strided fp8 view (what the
    reference's `.contiguous()` runs) and pcamd_repack_fp8. Both must give
    the same bytes; GB/s counts the bytes read and written."""
    from practice_cuda_amd.impls._common import repack_rows_major
    res = {}
    for name, (rows, cols) in {"dgrad_B_W_14336x4096": (4096, 14336), "wgrad_A_dY_8192x14336": (14336, 8192),
                               "X_8192x4096": (4096, 8192)}.items():
        nsets = 3
        g = torch.Generator(device=dev).manual_seed(rows + cols)
        srcs = [torch.randint(0, 256, (cols, rows), generator=g, device=dev, dtype=torch.uint8)
                .view(torch.float8_e4m3fn).t() for _ in range(nsets)]   # [rows, cols], stride(-2) == 1
        dsts = [torch.empty(rows, cols, dtype=torch.float8_e4m3fn, device=dev) for _ in range(nsets)]
        ms_t, _ = graph_time(torch, lambda i: dsts[i % nsets].copy_(srcs[i % nsets]), steps, warmup)
        ms_h, _ = graph_time(torch, lambda i: repack_rows_major(srcs[i % nsets][None]), steps, warmup)
        same = torch.equal(repack_rows_major(srcs[0][None])[0].view(torch.uint8), srcs[0].contiguous().view(torch.uint8))
        nbytes = 2 * rows * cols
        res[name] = {"torch_copy_ms": ms_t, "repack_ms": ms_h, "bytes": nbytes,
                     "torch_copy_GB/s": nbytes / (ms_t * 1e-3) / 1e9, "repack_GB/s": nbytes / (ms_h * 1e-3) / 1e9,
                     "identical": same}
        del srcs, dsts
        torch.cuda.empty_cache()
    print(json.dumps({"repack": res}))


def gemm_ref(torch, dev, steps, warmup, eager):
    """Reference point for the config-5 GEMMs: the same three products with
    per-tensor scales and the forward with row / column scales, run by this
    build's kernels and by hipBLASLt through torch._scaled_mm (which takes
    no 1x128 / 128x128 block scales, so the block-scaled trio has no library
    counterpart). Both sides use the same fp8 operands and scales; their
    outputs are compared (max-abs-rel). 'graph': median HIP-graph time per
    launch, one JSON line; 'eager': three launches of each, for counters."""
    from practice_cuda_amd.impls.hip_per_channel import hip_per_channel_bmm, hip_per_channel_quant
    from practice_cuda_amd.impls.hip_per_tensor import hip_per_tensor_bmm, hip_per_tensor_quant
    from practice_cuda_amd.registry import QuantResult
    M, K, N = 8192, 4096, 14336
    g = torch.Generator().manual_seed(0)
    X = torch.randn(M, K, generator=g).bfloat16().to(dev)
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16().to(dev)
    dY = (torch.randn(M, N, generator=g) * 1e-3).bfloat16().to(dev)
    tx, tw, tdy = (hip_per_tensor_quant(t[None]) for t in (X, W, dY))

    def view(r, t):
        return QuantResult(t, r.dequant_scale, r.impl, r.granularity, dict(r.meta))

    bf = torch.bfloat16
    sx, sw, sdy = (r.dequant_scale.reshape(()).float() for r in (tx, tw, tdy))
    x8, w8, dy8 = tx.tensor[0], tw.tensor[0], tdy.tensor[0]
    w_cm = w8.t().contiguous().t()               # [N, K] column-major: dgrad's B contiguous along N
    dyt8 = dy8.t().contiguous()                  # [N, M] row-major
    x_cm = x8.t().contiguous().t()               # [M, K] column-major
    out_f = torch.empty(1, M, N, dtype=bf, device=dev)
    out_d = torch.empty(1, M, K, dtype=bf, device=dev)
    out_w = torch.empty(1, N, K, dtype=bf, device=dev)
    a_w, b_w = view(tdy, dyt8[None]), view(tx, x_cm[None])    # wgrad on K-major operands
    cx = hip_per_channel_quant(X[None], channel_axis=-2)
    cw = hip_per_channel_quant(W[None], channel_axis=-2)
    cwt = QuantResult(cw.tensor.transpose(-1, -2), cw.dequant_scale, cw.impl, "channel",
                      {**cw.meta, "channel_axis": -1})
    csa = cx.dequant_scale.reshape(M, 1).contiguous()
    csb = cw.dequant_scale.reshape(1, N).contiguous()
    cases = {
        "tensor_fwd": (lambda i: hip_per_tensor_bmm(tx, view(tw, tw.tensor.transpose(-1, -2)), out=out_f),
                       lambda i: torch._scaled_mm(x8, w8.t(), scale_a=sx, scale_b=sw, out_dtype=bf)),
        "tensor_dgrad": (lambda i: hip_per_tensor_bmm(tdy, view(tw, w_cm[None]), out=out_d),
                         lambda i: torch._scaled_mm(dy8, w_cm, scale_a=sdy, scale_b=sw, out_dtype=bf)),
        "tensor_wgrad": (lambda i: hip_per_tensor_bmm(a_w, b_w, out=out_w),
                         lambda i: torch._scaled_mm(dyt8, x_cm, scale_a=sdy, scale_b=sx, out_dtype=bf)),
        "channel_fwd": (lambda i: hip_per_channel_bmm(cx, cwt, out=out_f),
                        lambda i: torch._scaled_mm(cx.tensor[0], cw.tensor[0].t(),
                                                   scale_a=csa, scale_b=csb, out_dtype=bf)),
    }
    flops = 2 * M * N * K
    res = {}
    for name, (ours, lib) in cases.items():
        if eager:
            for fn in (ours, lib):
                for i in range(3):
                    fn(i)
                torch.cuda.synchronize()
            continue
        o = ours(0)
        a = o.float().reshape(-1, o.shape[-1])
        b = lib(0).float()
        rel = ((a - b).abs().max() / b.abs().max()).item()
        del a, b
        row = {"max_abs_rel_vs_hipblaslt": rel}
        for side, fn in (("ours", ours), ("hipblaslt", lib)):
            ms, _ = graph_time(torch, fn, steps, warmup)
            row[side] = {"ms": ms, "TFLOP/s": flops / (ms * 1e-3) / 1e12}
        res[name] = row
    if not eager:
        print(json.dumps({"gemm_ref": res, "shape": {"M": M, "K": K, "N": N},
                          "note": "fwd X W^T, dgrad dY W, wgrad dY^T X; both sides get the same operand "
                                  "layouts, contiguous along the reduction (what torch._scaled_mm takes)"}))


# The per-tensor fp8 BMM shapes the reference publishes timings for, (B, M,
# N, K), B's layout, and the published best time in ms (Triton config sweeps
# on unstated NVIDIA hardware, fp16 C + fp16 bias; xuOAO/practice_cuda
# kernels/fp8_bmm/bench/fp8_quant_bmm_best.json:9-1045 for N-major B,
# fp8_quant_bmm_best_k_order.json:9-1119 for K-major B). Context, not targets.
PUBLISHED_BMM = [
    (16, 512, 960, 1280, "n", 0.1461), (16, 2048, 640, 1280, "n", 0.3532), (16, 2048, 1280, 1280, "n", 0.6807),
    (16, 2048, 1280, 960, "n", 0.5803), (32, 2048, 640, 1280, "n", 0.6987), (32, 2048, 960, 1600, "n", 1.2715),
    (32, 2048, 1280, 1600, "n", 1.7056), (32, 2048, 1600, 1600, "n", 2.1081), (32, 2048, 1280, 960, "n", 1.1478),
    (80, 512, 640, 1280, "n", 0.4437), (80, 2048, 640, 640, "n", 1.0126), (80, 2048, 960, 640, "n", 1.4863),
    (80, 2048, 1280, 640, "n", 1.9913), (80, 2048, 1280, 960, "n", 2.8504), (80, 2048, 640, 1280, "n", 1.7068),
    (80, 512, 1280, 960, "k", 0.3642), (80, 512, 1280, 640, "k", 0.2535), (80, 512, 960, 640, "k", 0.1935),
    (32, 512, 1280, 960, "k", 0.1524), (32, 512, 1280, 1600, "k", 0.2462), (32, 512, 960, 1600, "k", 0.1881),
    (16, 512, 1280, 160, "k", 0.0332), (16, 512, 1280, 960, "k", 0.0803), (16, 512, 1280, 1280, "k", 0.1033),
    (16, 512, 960, 1280, "k", 0.0800), (80, 512, 80, 640, "k", 0.0353), (16, 512, 160, 1280, "k", 0.0231),
    (80, 512, 640, 1280, "k", 0.2481), (32, 512, 640, 1280, "k", 0.1034), (16, 512, 640, 1280, "k", 0.0575),
    (512, 512, 512, 512, "k", 0.5420),
]


def published_bmm(torch, dev, steps, warmup, eager):
    """The legacy per-tensor BMM (C = (A @ B) * s + bias, fp16 C, fp16 bias
    [B, M, N]: the signature of the reference's sweep,
    kernels/fp8_bmm/bench/find_fp8_bmm_best.py:34-53) on PUBLISHED_BMM, with
    preallocated outputs and enough rotating input sets to exceed the MALL."""
    from practice_cuda_amd import _lib
    from practice_cuda_amd.impls import _common as C
    f8 = torch.float8_e4m3fn
    g = torch.Generator(device=dev).manual_seed(0)
    rows = []
    for bsz, m, n, k, lay, ref_ms in PUBLISHED_BMM:
        nbytes = bsz * (m * k + k * n + 4 * m * n)  # A, B fp8; bias, C fp16
        nsets = 1 if eager else max(1, min(8, -(-(512 << 20) // nbytes)))
        sets = []
        for _ in range(nsets):
            a = torch.randn(bsz, m, k, generator=g, device=dev).to(f8)
            if lay == "n":
                b = torch.randn(bsz, k, n, generator=g, device=dev).to(f8)
            else:
                b = torch.randn(bsz, n, k, generator=g, device=dev).to(f8).transpose(1, 2)
            bias = torch.randn(bsz, m, n, generator=g, device=dev).half()
            out = torch.empty(bsz, m, n, device=dev, dtype=torch.float16)
            sets.append((a, b, bias, out))
        scale = torch.ones(1, device=dev, dtype=torch.float32)

        def launch(i, sets=sets, scale=scale, bsz=bsz, m=m, n=n, k=k):
            a, b, bias, out = sets[i % len(sets)]
            C.launch_bmm(a, b, out, bias, tuple(bias.stride()), _lib.dtype_code(bias.dtype), scale, (0, 0, 0),
                         None, (0, 0, 0), _lib.SCALE_TENSOR, False, 1, 128, 1, "none", bsz, m, n, k)

        flops = 2 * bsz * m * n * k
        if eager:
            for i in range(3):
                launch(i)
            torch.cuda.synchronize()
            continue
        ms, _ = graph_time(torch, launch, steps, warmup)
        rows.append({"shape": [bsz, m, n, k], "b_layout": lay, "ms": round(ms, 5),
                     "TFLOP/s": round(flops / ms / 1e9, 1), "GB/s": round(nbytes / ms / 1e6, 1),
                     "frac_of_fp8_peak": round(flops / ms / 1e9 / FP8_PEAK_TFLOPS, 4),
                     "frac_of_hbm_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
                     "published_ms": ref_ms, "published_TFLOP/s": round(flops / ref_ms / 1e9, 1),
                     "rotating_sets": nsets})
        del sets
        torch.cuda.empty_cache()
    if not eager:
        print(json.dumps({"published_bmm": rows, "what": "per-tensor fp8 e4m3 BMM, fp16 C + fp16 bias [B,M,N], "
                          "graph-timed median of 5 replays; published_* = the reference's Triton sweep on "
                          "unstated hardware (context, not a target)"}))


def fused_probe(torch, dev, steps, warmup):
    """pcamd_bmm_quant_a (A quantized 1x128 inside the GEMM's K loop) next to
    its unfused equal (hip_per_block_quant, then hip_per_block_bmm), graph-
    timed on the same inputs: bf16 A [M, K] (two tensors in turn), e4m3 B
    [K, N] (N-major, 128x128 scales), bf16 C. The fused kernel quantizes each A row block once
    per N tile, so it wins where few N tiles share A (small N) and loses as N
    grows; `default_path` names what hip_per_block_bmm_quant_a runs without
    always_fused (the fused call inside the streaming kernel's envelope: here
    up to FUSED_MAX_N columns, K = 4096). Inside that envelope both paths are
    timed again with a bf16 bias [M, N] and GELU in the epilogue."""
    from practice_cuda_amd.impls.hip_per_block import (fused_streams, hip_per_block_bmm,
                                                       hip_per_block_bmm_quant_a, hip_per_block_quant)
    g = torch.Generator(device=dev).manual_seed(0)
    rows = []
    for idx, (m, k, n) in enumerate([(32768, 4096, 64), (32768, 4096, 128), (32768, 4096, 192), (32768, 4096, 256),
                                     (16384, 4096, 512), (8192, 4096, 1024), (8192, 4096, 4096),
                                     (8192, 4096, 14336)]):
        # two A inputs in turn (2 x 268 MB at M = 32768: beyond the 256 MB MALL)
        xs = [torch.randn(1, m, k, generator=g, device=dev).bfloat16() for _ in range(2)]
        qb = hip_per_block_quant((torch.randn(1, k, n, generator=g, device=dev) * 0.02).bfloat16(),
                                 block_m=128, block_n=128)
        out = torch.empty(1, m, n, device=dev, dtype=torch.bfloat16)
        fused = lambda i: hip_per_block_bmm_quant_a(xs[i % 2], qb, out=out, always_fused=True)  # noqa: E731
        # the clocks settle under load before the first timing of the process
        fused_ms, _ = graph_time(torch, fused, steps, warmup, settle_ms=SETTLE_MS if idx == 0 else 0.0)

        def unfused(i):
            hip_per_block_bmm(hip_per_block_quant(xs[i % 2], block_m=1, block_n=128), qb, out=out)

        unfused_ms, _ = graph_time(torch, unfused, steps, warmup)
        streams = fused_streams(n, k, 128)
        rows.append({"m": m, "k": k, "n": n, "fused_us": round(fused_ms * 1e3, 1),
                     "quantize_then_multiply_us": round(unfused_ms * 1e3, 1),
                     "fused_speedup": round(unfused_ms / fused_ms, 3),
                     "default_path": "fused" if streams else "quantize_then_multiply"})
        if streams:
            bias = torch.randn(1, m, n, generator=g, device=dev).bfloat16()

            def fused_bg(i):
                hip_per_block_bmm_quant_a(xs[i % 2], qb, out=out, bias=bias, activation="gelu", always_fused=True)

            def unfused_bg(i):
                hip_per_block_bmm(hip_per_block_quant(xs[i % 2], block_m=1, block_n=128), qb, out=out, bias=bias,
                                  activation="gelu")

            rows[-1]["fused_bias_gelu_us"] = round(graph_time(torch, fused_bg, steps, warmup)[0] * 1e3, 1)
            rows[-1]["quantize_then_multiply_bias_gelu_us"] = round(
                graph_time(torch, unfused_bg, steps, warmup)[0] * 1e3, 1)
            del bias
        print(rows[-1], file=sys.stderr, flush=True)
        del xs, qb, out
        torch.cuda.empty_cache()
    print(json.dumps({"fused_quant_bmm": rows}))


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; --gpus must be 1 "
                          "(the path shards by rows and batch with no exchange for the quantizers; "
                          "multi-GPU runs are not launched)"}))
        sys.exit(2)
    import torch

    from practice_cuda_amd import _lib
    _lib.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.pmc_probe:
        pmc_probe(torch, dev)
        return
    if args.pmc_probe_bmm:
        pmc_probe_bmm(torch, dev)
        return
    if args.pmc_probe_fused:
        pmc_probe_fused(torch, dev)
        return
    if args.mem_ceiling:
        mem_ceiling(torch, dev, args.steps, args.warmup)
        return
    if args.gemm_ref:
        gemm_ref(torch, dev, args.steps, args.warmup, args.gemm_ref == "eager")
        return
    if args.repack:
        repack_probe(torch, dev, args.steps, args.warmup)
        return
    if args.fused:
        fused_probe(torch, dev, args.steps, args.warmup)
        return
    if args.published:
        published_bmm(torch, dev, args.steps, args.warmup, args.published == "eager")
        return

    x2 = make_config2(torch)
    head = bench_quant(torch, "config2_per_channel_quant_18432x7168", x2, "channel",
                       args.steps, args.warmup, 4, dev, settle_ms=SETTLE_MS)
    ms = head["ms_per_step"]
    line = {
        "metric": "quant GB/s and FP8 BMM TFLOP/s at 1 MI355X, % of HBM / fp8-MFMA peak",
        "value": round(head["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16->fp8e4m3 (fp32 math)",
        "data": "synthetic (BASELINE configs, CPU generator seed 0)",
        "config": {"workload": "BASELINE configs[1]: per-channel fp8 quant, bf16 weight [18432,7168] "
                               "-> e4m3 + fp32 row scales [18432], channel_axis=-2",
                   "shape": [18432, 7168], "rotating_buffer_sets": 4,
                   "metric_halves": "value and roofline are the quantizer half of the metric (GB/s, % of HBM "
                                    "peak); the FP8 BMM half is in components: config 5 (the block-scaled "
                                    "GEMM trio) carries its own roofline block (TFLOP/s, % of dense fp8 "
                                    "peak), config 4 one against HBM",
                   "timing": "HIP graph of K launches, median of 5 replays, after ~100 ms untimed settle "
                             "and W warmup launches"},
        "roofline": {"bound": "hbm", "achieved": round(head["value"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(head["value"] / HBM_PEAK_GBS, 4),
                     "traffic": None, "kernel": HEADLINE_KERNEL,
                     "bytes_per_launch": head["bytes_per_step"]},
    }
    # HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    # passes, used only if they were taken on the kernel that runs now
    traffic_file = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(traffic_file):
        with open(traffic_file) as fh:
            t = json.load(fh).get("config2_per_channel_quant")
        if t and t.get("kernel") == HEADLINE_KERNEL:
            line["roofline"]["traffic"] = t["hbm_bytes_per_launch"]

    if not args.no_components:
        only = set(filter(None, args.components_only.split(",")))
        comps = []
        try:
            if not only or "config1" in only:
                comps.append(bench_quant(torch, "config1_1x128_quant_4096x7168", make_config1(torch),
                                         "block", args.steps, args.warmup, 8, dev, 1, 128))
            if not only or "config3" in only:
                comps.append(bench_quant(torch, "config3_128x128_quant_4096x7168", make_config3(torch),
                                         "block", args.steps, args.warmup, 8, dev, 128, 128))
            if not only or "columns" in only:
                # config 2's weight with one scale per column (channel_axis=-1: the
                # reference bench's default axis, and the per-channel BMM's B operand)
                comps.append(bench_quant(torch, "config2_weight_per_column_quant_18432x7168", make_config2(torch),
                                         "columns", args.steps, args.warmup, 4, dev))
            if not only or "config4" in only:
                comps.append(bench_config4(torch, args.steps, args.warmup, dev))
            if not only or "config5" in only:
                # ~20 untimed launches bring the GPU to its steady MFMA clock
                # (measured: the first few ms of GEMMs after start-up run ~15% slower)
                comps.append(bench_config5(torch, max(5, args.steps // 5), 20, dev))
        except Exception as exc:  # a component failure must not hide the headline
            comps.append({"error": repr(exc)})
        for c in comps:
            for k, v in list(c.items()):
                if isinstance(v, float):
                    c[k] = round(v, 5)
        line["components"] = comps

    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(torch, x2, dev)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
