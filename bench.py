#!/usr/bin/env python3
"""Benchmark of the CSR sparse x dense hot path on one MI355X.

A step is one CSR SpMV ``y = A @ x`` through the drop-in API (``CSRArray``
with its cached bound plan, ``A @ x`` on torch's current stream) on the
headline workload: n = 4,194,304 rows, exactly 16 columns per row drawn
uniformly without replacement, float32 values / int32 indices (synthetic,
seeded).  Inputs are resident in HBM before timing starts.  The plan is the
library's automatic choice for this matrix: LDS column panels (two passes,
panel_products then panel_rows).

Prints ONE JSON line.  ``value`` is the effective bandwidth on compulsory
traffic, nnz*(4+4) + (n+1)*4 + 4n (x) + 4n (y) bytes per step.  Extra fields:

- ``roofline``: achieved GB/s of one SpMV call (both kernels of the plan,
  back to back on the launch stream) from HIP events around HIP-graph
  replays, against the 8 TB/s HBM peak; ``traffic`` is the measured HBM
  bytes per call from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
  summary (profiles/spmv_random16_traffic.txt) when it was taken on the same
  plan kind, else null;
- ``cold``: the same SpMV with a 1 GiB buffer written between launches
  (evicts the 256 MB Infinity Cache), median of per-launch times;
- ``spmm``: CSR SpMM with k=64 on the 3D 7-point Poisson matrix (128^3),
  GFLOP/s, and its ratio to SpMV GFLOP/s on the same matrix and on the
  headline matrix;
- ``batched_spmv``: 8 vectors at once on the same Poisson matrix (native
  batched entry point), against 8 single SpMVs;
- ``cg``: conjugate gradients (device-resident loop) on the Poisson matrix,
  time per iteration against its bytes (the single-threaded reference loop
  on the host is timed in the CPU leg);
- ``krylov``: BiCGSTAB, MINRES and GMRES(20) (device-resident loops) at n = 128^3, the
  same figures;
- ``mtx`` (with ``--mtx PATH``): SpMV on a Matrix Market matrix read by the
  native reader (``mmread``);
- ``adjoint``: on the headline matrix, ``A^T x`` by atomic scatter and over
  the cached transpose, the transpose build, the SpMV value gradient and one
  autograd step (forward + ``A^T g``);
- ``configs`` (skipped with ``--no-configs``): SpMV on every configuration
  of the benchmark definition (the headline, 2D Laplacian, power law with
  int64 indices, 3D Poisson, the banded matrix in float32 / bfloat16 /
  float16 / complex64) and SpMM at k = 8 / 64 / 256 (Poisson) and k = 64
  (float16 and bfloat16 banded), graph-replay (warm) and cold timed against
  each one's compulsory bytes, with the plan kind and its footprint;
- ``cpu_baseline``: the product's CPU path (``ms.use_cpu()``, the C++
  restatement of the reference CPU kernel in csrc/csr_cpu.cpp, ``-O3``
  without ``-march=native``) on the headline matrix, at the reference-resolved
  worker count and at one thread, on this host's cores, with the CPU model;
  and (``solvers``) the oracle's single-threaded restatements of the
  reference solver loops on the solver legs' systems, whose per-iteration
  times and speedups are added to the ``cg`` and ``krylov`` rows.  With
  ``--no-cpu`` no CPU figure is taken.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "mlx-sparse_amd"))
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402
import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
# The allocation-free transposed product's file-scope device array
# (csr_transpose.hip), resident on every GPU the library runs on.
NOALLOC_SCRATCH_BYTES = 32 << 20


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _events_time(fn, iters: int) -> float:
    """Mean milliseconds per call of ``fn`` from HIP events on the current
    stream (the stream the kernels are launched on)."""
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / iters


class GraphTime(float):
    """Median milliseconds per call over the replays (the float value), with
    the mean over all of them as ``.mean``."""

    mean: float
    replays: int


def _graph_time(fn, calls: int = 20, replays: int = 50) -> tuple[GraphTime, torch.Tensor]:
    """Milliseconds per call of ``fn`` with the host out of the loop:
    ``calls`` launches are captured in one HIP graph, replayed ``replays``
    times, each replay between its own HIP events.  The result is the median
    over the replays of (replay time / calls), with the mean beside it.
    Every replay's last output is compared with the eager result (the
    kernels are deterministic), so a replay that went wrong cannot go
    unnoticed.  Returns (ms per call, eager output)."""
    eager = fn()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [fn() for _ in range(calls)]
    graph.replay()
    torch.cuda.synchronize()
    if not torch.equal(outs[-1], eager):
        raise RuntimeError("graph replay result differs from the eager call")
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(replays)]
    for a, b in events:
        a.record()
        graph.replay()
        b.record()
    events[-1][1].synchronize()
    if not torch.equal(outs[-1], eager):
        raise RuntimeError("graph replay result differs from the eager call")
    per = [a.elapsed_time(b) / calls for a, b in events]
    ms = GraphTime(statistics.median(per))
    ms.mean = statistics.fmean(per)
    ms.replays = replays
    del graph, outs
    return ms, eager


def _cold_time(fn, iters: int, scratch: torch.Tensor, clean: bool = False) -> float:
    """Median ms per call with a 1 GiB write between calls (untimed).
    ``clean``: the write is followed by a 1 GiB read, so the Infinity Cache
    holds clean lines of the scratch buffer when the call starts and the
    call does not pay for writing back the flush's own dirty lines."""
    times = []
    for _ in range(iters):
        scratch.fill_(1.0)
        if clean:
            torch.amax(scratch)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b))
    return statistics.median(times)


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_wall(fn, seconds: float, lo: int = 10, hi: int = 30) -> tuple[float, int]:
    """Median wall seconds per call after 3 warm-up calls, over at least
    ``lo`` calls (and up to ``hi`` while ``seconds`` last)."""
    for _ in range(3):
        fn()
    samples = []
    t_end = time.perf_counter() + seconds
    while len(samples) < lo or (time.perf_counter() < t_end and len(samples) < hi):
        t0 = time.perf_counter()
        fn()
        samples.append(time.perf_counter() - t0)
    return statistics.median(samples), len(samples)


def cpu_baseline(m, x, seconds: float = 10.0) -> dict:
    """The product's CPU path, ``ms.use_cpu()`` then ``A @ x`` on the same
    matrix: the C++ restatement of the reference CPU kernel
    (csrc/csr_cpu.cpp: stored-order row sums, the O(n) row-work prepass,
    nnz-balanced ranges, std::threads spawned per call; reference
    csr_matvec.cpp:116-168, cpu_parallel.h:50-97), at the reference-resolved
    worker count and at one thread.  The oracle's C restatement is timed
    beside it as a cross-check (3 calls)."""
    import mlx_sparse as ms
    from mlx_sparse import runtime, synthetic
    from oracle import oracle as orc

    nbytes = synthetic.compulsory_bytes(m.nnz, m.shape[0], m.shape[1], 4, 4)
    prev = ms.default_torch_device()
    ms.use_cpu()
    try:
        A = ms.csr_array((torch.from_numpy(m.data), torch.from_numpy(m.indices),
                          torch.from_numpy(m.indptr)), shape=m.shape)
        xc = torch.from_numpy(x)
        assert A.data.device.type == "cpu"
        threads = runtime.resolve_n_threads()[0]
        med, n = _median_wall(lambda: A @ xc, seconds)
        with runtime.context(n_threads=1):
            med1, n1 = _median_wall(lambda: A @ xc, seconds, lo=10, hi=10)
    finally:
        if prev.type == "cuda":
            ms.use_gpu(prev.index or 0)
    t0 = time.perf_counter()
    for _ in range(3):
        orc.csr_matvec(m.data, m.indices, m.indptr, x, m.shape[0], n_threads=threads)
    oracle_ms = (time.perf_counter() - t0) / 3 * 1e3
    model = _cpu_model()
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "ms": round(med * 1e3, 2),
        "threads_1": {"value": round(nbytes / med1 / 1e9, 3), "unit": "GB/s",
                      "ms": round(med1 * 1e3, 2)},
        "cpu_model": model,
        "affinity_cores": len(os.sched_getaffinity(0)),
        "oracle_check_ms": round(oracle_ms, 2),
        "sample": (f"ms.use_cpu() A @ x on the headline matrix, median of {n} calls at "
                   f"{threads} threads and {n1} at 1 thread; g++ -O3 -ffp-contract=off, "
                   f"no -march=native"),
    }


def adjoint_leg(ext, A, m, x, spmv_bytes: int) -> dict:
    """The adjoint path on the headline matrix, HIP events around back-to-back
    calls (the transpose and the f16 products take stream-ordered scratch):

    - ``A^T x`` by atomic scatter (msx_csr_spmv_transpose), compulsory bytes
      as the SpMV's;
    - the CSR transpose build (radix sort; read and write nnz*(4+4) + (n+1)*4);
    - ``A^T x`` as SpMV over the cached transpose with its own plan;
    - the SpMV value gradient (indices + indptr + x + cot read, nnz*4 written),
      through the matrix's plan (its panel layout: what autograd uses) and
      plan-free;
    - one autograd step ``(A @ x).backward(g)`` with x requiring grad
      (forward SpMV + A^T g over the cached transpose, "auto" route warm)."""
    n_rows, n_cols = m.shape
    data, indices, indptr = A.buffers(x.device)
    g = torch.randn(n_rows, device=x.device, generator=torch.Generator(x.device).manual_seed(4))
    out = {"workload": "random16 n=4194304 nnz=67108864 f32/i32 (the headline matrix)"}
    scatter = lambda: ext.csr_matvec_transpose(data, indices, indptr, g, n_rows, n_cols)
    for _ in range(3):
        scatter()
    t = _events_time(scatter, 20)
    out["atomic_us"] = round(t * 1e3, 1)
    out["atomic_frac"] = round(spmv_bytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    build = lambda: ext.csr_transpose(data, indices, indptr, n_rows, n_cols)
    build()
    t = _events_time(build, 5)
    tb = 2 * (m.nnz * 8 + (n_cols + 1) * 4)
    out["transpose_build_us"] = round(t * 1e3, 1)
    out["transpose_build_frac"] = round(tb / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    T = A.T
    td, ti, tp = T.buffers(x.device)
    tplan = T.plan(x.device)
    cached = lambda: ext.csr_matvec(td, ti, tp, g, n_cols, n_rows, plan=tplan)
    for _ in range(3):
        cached()
    t = _events_time(cached, 20)
    out["cached_transpose_us"] = round(t * 1e3, 1)
    out["cached_transpose_frac"] = round(spmv_bytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    vb = m.nnz * 8 + (n_rows + 1) * 4 + 4 * (n_rows + n_cols)
    plan = A.plan(x.device)
    for key, pl in (("data_vjp", plan), ("data_vjp_planfree", None)):
        vjp = lambda: ext.csr_matvec_data_vjp(indices, indptr, x, g, n_rows, n_cols, plan=pl)
        for _ in range(3):
            vjp()
        t = _events_time(vjp, 20)
        out[f"{key}_us"] = round(t * 1e3, 1)
        out[f"{key}_frac"] = round(vb / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    xr = x.clone().requires_grad_()

    def train_step():
        xr.grad = None
        (A @ xr).backward(g)

    for _ in range(3):
        train_step()
    t = _events_time(train_step, 20)
    out["autograd_step_us"] = round(t * 1e3, 1)
    out.update(inplace_training(A, x, g))
    log(f"adjoint: {out}")
    return out


def inplace_training(A, x, g) -> dict:
    """One SGD step on the headline matrix's values, in place: the forward
    ``A @ x`` (the bound panel plan refreshed from the new values first),
    the backward (``x.grad = A^T g`` over the cached transpose, its values
    regathered after the update; ``A.data.grad`` by the value gradient
    through the panel plan) and ``A.data -= lr * A.data.grad``.  Timed with
    HIP events over 20 steps after 3 warm-up steps (the first backward
    scatters, the second builds the transpose, later ones regather); the
    plan refresh and the transposed-values regather are also timed alone."""
    import mlx_sparse as ms
    from mlx_sparse import _native

    vals = A.data.detach().clone().requires_grad_()
    A2 = ms.csr_array((vals, A.indices, A.indptr), shape=A.shape)
    x2 = x.clone().requires_grad_()

    def sgd_step():
        x2.grad = None
        (A2 @ x2).backward(g)
        with torch.no_grad():
            vals.add_(vals.grad, alpha=-1e-3)  # torch.optim.SGD's update, one pass
        vals.grad = None

    for _ in range(3):
        sgd_step()
    out = {"inplace_train_step_us": round(_events_time(sgd_step, 20) * 1e3, 1)}
    plan = A2.plan(x.device)
    d = vals.detach()
    refresh = lambda: plan.refresh(d)
    refresh()
    out["plan_refresh_us"] = round(_events_time(refresh, 20) * 1e3, 1)
    _, i, p = A2.buffers(x.device)
    pos = _native.csr_transpose_positions(i, p, A2.shape)[0]
    t_vals = torch.empty_like(d)
    gather = lambda: _native.csr_transpose_values(d, pos, False, t_vals)
    gather()
    out["transpose_gather_us"] = round(_events_time(gather, 20) * 1e3, 1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    layout = _native.csr_transpose_layout(pos, d)
    torch.cuda.synchronize()
    out["transpose_layout_build_ms"] = round((time.perf_counter() - t0) * 1e3, 2)
    scratch = torch.empty_like(d)
    regather = lambda: _native.csr_transpose_values_layout(d, layout, False, scratch, t_vals)
    regather()
    out["transpose_regather_us"] = round(_events_time(regather, 20) * 1e3, 1)
    out["inplace_train_step"] = ("SGD step on A.data in place: plan refresh + forward SpMV + "
                                 "A^T g over the cached transpose (values regathered in two "
                                 "streaming passes) + value gradient through the panel plan + "
                                 "the update; transpose_gather_us: the one-pass random gather "
                                 "it replaces")
    del A2, vals, x2, pos, t_vals, layout, scratch
    return out


def mtx_leg(ext, path: str, dev) -> dict:
    """SpMV on a Matrix Market file read with ``mmread`` (native reader):
    ingestion time, then the cached-plan SpMV timed like the headline step,
    against the matrix's compulsory bytes."""
    import mlx_sparse as ms
    from mlx_sparse import synthetic

    t0 = time.perf_counter()
    A = ms.mmread(path)
    torch.cuda.synchronize()
    read_s = time.perf_counter() - t0
    if A.dtype != torch.float32:
        return {"file": path, "skipped": f"dtype {A.dtype}"}
    n_rows, n_cols = A.shape
    x = torch.linspace(-1, 1, n_cols, device=dev)
    data, indices, indptr = A.buffers(dev)
    plan = A.plan(dev)
    info = plan.info()
    spmv_ms, _ = _graph_time(lambda: ext.csr_matvec(data, indices, indptr, x, n_rows, n_cols,
                                                    plan=plan))
    nbytes = synthetic.compulsory_bytes(A.nnz, n_rows, n_cols, 4, indices.element_size())
    kind = "panels" if info.get("n_panels") else ("slices" if info.get("n_slices") else "blocks")
    out = {"file": os.path.basename(path), "shape": [n_rows, n_cols], "nnz": A.nnz,
           "read_s": round(read_s, 3), "plan": kind, "kernel_us": round(spmv_ms * 1e3, 2),
           "gbs": round(nbytes / (spmv_ms * 1e-3) / 1e9, 1),
           "frac": round(nbytes / (spmv_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    log(f"mtx: {out}")
    return out


def cg_leg(dev) -> dict:
    """Conjugate gradients (``linalg.cg``, device-resident loop) on the 3D
    Poisson matrix 128^3, b = 1, x0 = 0, rtol = 1e-6.  Bytes per iteration:
    the SpMV's compulsory bytes plus 11 float vectors of n (p.ap reads p, ap;
    the update reads x, p, r, ap and writes x, r; the direction reads r, p and
    writes p).  Its CPU figure comes from the CPU baseline leg
    (``cpu_solver_baselines``)."""
    import mlx_sparse as ms
    from mlx_sparse import linalg, synthetic

    p = synthetic.poisson_3d(128)
    n = p.shape[0]
    P = ms.csr_array((p.data, p.indices, p.indptr), shape=p.shape, canonical=True)
    b = torch.ones(n, device=dev)
    P.plan(dev)
    x, info = linalg.cg(P, b, rtol=1e-6, return_info=True)  # warm-up (plan, allocator)
    times = []
    for _ in range(3):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        x, info = linalg.cg(P, b, rtol=1e-6, return_info=True)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    solve_s = statistics.median(times)
    its = info.iterations
    per_it = solve_s / max(its, 1)
    it_bytes = synthetic.compulsory_bytes(p.nnz, n, n, 4, 4) + 11 * 4 * n
    out = {
        "workload": "poisson3d 128^3 n=2097152 nnz=14581760 f32/i32, b=1, x0=0, rtol=1e-6",
        "info": info.status, "iterations": its, "residual": info.residual_norm,
        "solve_ms": round(solve_s * 1e3, 2), "us_per_iteration": round(per_it * 1e6, 1),
        "bytes_per_iteration": it_bytes,
        "gbs": round(it_bytes / per_it / 1e9, 1),
        "frac": round(it_bytes / per_it / 1e9 / HBM_PEAK_GBS, 4),
    }
    log(f"cg: {out}")
    return out


# Benchmark configurations: short id -> (label,
# matrix generator, value type, rhs width k or None, complex values).  The
# matrix generators are seeded; x ~ U[-1, 1] (cfg3: U[0, 1]), X ~ N(0, 1).
CASES = {
    "cfg1": ("cfg1 laplacian2d 1024^2 f32/i32", "laplacian", torch.float32, None),
    "cfg2": ("cfg2 random16 n=2^22 f32/i32", "random16", torch.float32, None),
    "cfg3": ("cfg3 powerlaw zipf2 n=2^21 f32/i64", "powerlaw", torch.float32, None),
    "cfg4": ("cfg4 poisson3d 128^3 f32/i32", "poisson", torch.float32, None),
    "cfg4-k8": ("cfg4 poisson3d 128^3 f32/i32", "poisson", torch.float32, 8),
    "cfg4-k64": ("cfg4 poisson3d 128^3 f32/i32", "poisson", torch.float32, 64),
    "cfg4-k256": ("cfg4 poisson3d 128^3 f32/i32", "poisson", torch.float32, 256),
    "cfg5-f32": ("cfg5 banded hb32 f32/i32", "banded", torch.float32, None),
    "cfg5-bf16": ("cfg5 banded hb32 bf16/i32", "banded", torch.bfloat16, None),
    "cfg5-f16": ("cfg5 banded hb32 f16/i32", "banded", torch.float16, None),
    "cfg5-f16-k64": ("cfg5 banded hb32 f16/i32", "banded", torch.float16, 64),
    "cfg5-bf16-k64": ("cfg5 banded hb32 bf16/i32", "banded", torch.bfloat16, 64),
    "cfg5-c64": ("cfg5 banded hb32 c64/i32", "banded", torch.complex64, None),
}


def _matrix(kind: str):
    from mlx_sparse import synthetic

    if kind == "laplacian":
        return synthetic.laplacian_2d(1024)
    if kind == "random16":
        return synthetic.random_fixed_row(1 << 22, 16, seed=0)
    if kind == "powerlaw":
        return synthetic.power_law(1 << 21, 2.0, 200_000, seed=0)
    if kind == "poisson":
        return synthetic.poisson_3d(128)
    return synthetic.banded(1 << 20, 32, 0.65, 70.0, seed=0)


def _operands(case: str, m, dev):
    """(values, x or X) of a case on ``dev``."""
    from mlx_sparse import synthetic

    _, kind, dt, k = CASES[case]
    n = m.shape[1]
    if dt == torch.complex64:
        data = torch.from_numpy(synthetic.complex_values(m, seed=3))
        x = torch.complex(torch.from_numpy(synthetic.uniform(n, -1.0, 1.0, seed=4)),
                          torch.from_numpy(synthetic.uniform(n, -1.0, 1.0, seed=5)))
        return data, x.to(dev)
    data = torch.from_numpy(m.data).to(dt)
    if k is not None:
        return data, torch.from_numpy(synthetic.normal(n, seed=2, k=k)).to(dev).to(dt)
    low = 0.0 if kind == "powerlaw" else -1.0
    return data, torch.from_numpy(synthetic.uniform(n, low, 1.0, seed=1)).to(dev).to(dt)


def _case_call(ext, case: str, m, data, X, dev):
    """(call, info, compulsory bytes, flops, keep-alive) of a case through its
    cached bound plan (AUTO's choice); the keep-alive tuple ends with the
    plan's build time in ms (its first-call cost)."""
    import mlx_sparse as ms
    from mlx_sparse import synthetic

    _, _, dt, k = CASES[case]
    n_rows, n_cols = m.shape
    A = ms.csr_array((data, torch.from_numpy(m.indices), torch.from_numpy(m.indptr)),
                     shape=m.shape)
    d, i, p = A.buffers(dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    plan = A.plan(dev)  # the first call's cost: the bound plan is built here
    torch.cuda.synchronize()
    build_ms = round((time.perf_counter() - t0) * 1e3, 2)
    if k is None:
        fn = lambda: ext.csr_matvec(d, i, p, X, n_rows, n_cols, plan=plan)
    else:
        fn = lambda: ext.csr_matmul(d, i, p, X, n_rows, n_cols, plan=plan)
    vb, ib = data.element_size(), m.indices.dtype.itemsize
    nbytes = synthetic.compulsory_bytes(m.nnz, n_rows, n_cols, vb, ib, k=k or 1)
    nflops = synthetic.flops(m.nnz, k or 1, dt == torch.complex64)
    return fn, plan.info(), nbytes, nflops, (A, d, i, p, plan, build_ms)


def _kind(info) -> str:
    return "panels" if info.get("n_panels") else ("slices" if info.get("n_slices") else "blocks")


def krylov_leg(dev) -> dict:
    """BiCGSTAB and MINRES (device-resident loops) at n = 128^3: MINRES on
    the 3D Poisson matrix with shift -1, BiCGSTAB on a nonsymmetric
    convection-diffusion variant of it (x-direction off-diagonals -1.3 and
    -0.7, diagonal 8); b ~ U[-1, 1], rtol 1e-5.  Bytes per iteration: two
    SpMVs' compulsory bytes plus the vector passes (BiCGSTAB 20, MINRES 18
    float vectors of n).  Their CPU figures come from the CPU baseline leg
    (``cpu_solver_baselines``)."""
    import mlx_sparse as ms
    from mlx_sparse import linalg, synthetic

    m = synthetic.poisson_3d(128)
    n = m.shape[0]
    rows = np.repeat(np.arange(n), np.diff(m.indptr))
    cols = m.indices.astype(np.int64)
    conv = m.data.copy()
    conv[cols == rows + 1] = -0.7
    conv[cols == rows - 1] = -1.3
    conv[cols == rows] = 8.0
    b_np = synthetic.uniform(n, -1.0, 1.0, seed=7)
    b = torch.from_numpy(b_np).to(dev)
    spmv_bytes = synthetic.compulsory_bytes(m.nnz, n, n, 4, 4)
    out = {"workload": "n=2097152 (128^3) f32/i32, b~U[-1,1], rtol=1e-5"}
    for name, data, kw, nvec in (("minres", m.data, {"shift": -1.0}, 18),
                                 ("bicgstab", conv, {}, 20)):
        A = ms.csr_array((data, m.indices, m.indptr), shape=m.shape, canonical=True)
        solver = getattr(linalg, name)
        solver(A, b, rtol=1e-5, maxiter=500, **kw)  # plan, allocator
        times = []
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            x, info = solver(A, b, rtol=1e-5, maxiter=500, return_info=True, **kw)
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        solve_s = statistics.median(times)
        its = max(info.iterations, 1)
        it_bytes = 2 * spmv_bytes + nvec * 4 * n
        out[name] = {"matrix": "poisson3d + shift -1" if name == "minres" else
                     "convection-diffusion variant of poisson3d",
                     "info": info.status, "iterations": info.iterations,
                     "residual": info.residual_norm, "solve_ms": round(solve_s * 1e3, 2),
                     "us_per_iteration": round(solve_s / its * 1e6, 1),
                     "bytes_per_iteration": it_bytes,
                     "gbs": round(it_bytes / (solve_s / its) / 1e9, 1),
                     "frac": round(it_bytes / (solve_s / its) / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"{name}: {out[name]}")
        del A
        torch.cuda.empty_cache()
    out["gmres"] = gmres_row(dev, m, conv, b, b_np, spmv_bytes)
    return out


def gmres_row(dev, m, conv, b, b_np, spmv_bytes) -> dict:
    """Restarted GMRES(20) on the convection-diffusion variant at n = 128^3,
    rtol 1e-5.  Bytes per Arnoldi step j (0-based): the SpMV's compulsory
    bytes, then the paired Gram-Schmidt passes - 12 n for the first (w and
    two basis vectors read), 24 n for each of the j later pairs (w and four
    basis vectors read, w written), 16 n for the last pass (w and two basis
    vectors read, w written, w.w) - and 8 n for the normalisation; per cycle
    also the residual (12 n) and the update ((used + 2) 4 n).  Its CPU
    figure comes from the CPU baseline leg (``cpu_solver_baselines``)."""
    import mlx_sparse as ms
    from mlx_sparse import linalg

    n = m.shape[0]
    restart = 20
    A = ms.csr_array((conv, m.indices, m.indptr), shape=m.shape, canonical=True)
    linalg.gmres(A, b, rtol=1e-5, restart=restart, maxiter=500)  # plan, allocator
    times = []
    for _ in range(3):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        x, info = linalg.gmres(A, b, rtol=1e-5, restart=restart, maxiter=500, return_info=True)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    solve_s = statistics.median(times)
    its = max(info.iterations, 1)
    cycles = -(-its // restart)
    step_bytes = 0
    for j in range(restart):
        step_bytes += spmv_bytes + 12 * n + j * 24 * n + 16 * n + 8 * n
    cycle_bytes = step_bytes + 12 * n + (restart + 2) * 4 * n + spmv_bytes
    total_bytes = cycles * cycle_bytes
    row = {"matrix": "convection-diffusion variant of poisson3d", "restart": restart,
           "info": info.status, "iterations": info.iterations, "residual": info.residual_norm,
           "solve_ms": round(solve_s * 1e3, 2),
           "us_per_iteration": round(solve_s / its * 1e6, 1),
           "bytes_per_cycle": cycle_bytes,
           "gbs": round(total_bytes / solve_s / 1e9, 1),
           "frac": round(total_bytes / solve_s / 1e9 / HBM_PEAK_GBS, 4)}
    log(f"gmres: {row}")
    del A
    torch.cuda.empty_cache()
    return row


def configs_leg(ext, dev, scratch) -> list:
    """SpMV / SpMM on each benchmark configuration but the headline, through
    the cached bound plan (AUTO's choice), timed like the headline (graph
    replay) and cold (1 GiB written between calls; cold_clean: written, then
    read, so no dirty lines of the flush remain), against the compulsory
    bytes nnz*(value+index) + indptr + x once + y once (X, Y at width k)."""
    rows = []
    m_kind, m = None, None
    for case, (label, kind, dt, k) in CASES.items():
        if case == "cfg2":
            continue  # the headline leg
        if kind != m_kind:
            m, m_kind = None, None
            torch.cuda.empty_cache()
            m, m_kind = _matrix(kind), kind
        data, X = _operands(case, m, dev)
        fn, info, nbytes, nflops, keep = _case_call(ext, case, m, data, X, dev)
        t, _ = _graph_time(fn, calls=10 if k else 20)
        cold = _cold_time(fn, 10, scratch)
        clean = _cold_time(fn, 10, scratch, clean=True)
        row = {"case": label, "id": case, "nnz": m.nnz,
               "op": "spmv" if k is None else f"spmm k={k}",
               "plan": _kind(info), "plan_bytes": info["plan_bytes"],
               "plan_build_ms": keep[-1], "kernel_us_mean": round(t.mean * 1e3, 2),
               "block_nnz": info["block_nnz"], "window_rows": info["window_rows"],
               "long_rows": info["n_long_rows"], "compulsory_bytes": nbytes, "flops": nflops,
               "kernel_us": round(t * 1e3, 2), "gbs": round(nbytes / (t * 1e-3) / 1e9, 1),
               "frac": round(nbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
               "gflops": round(nflops / (t * 1e-3) / 1e9, 1),
               "cold_us": round(cold * 1e3, 2),
               "cold_frac": round(nbytes / (cold * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
               "cold_clean_us": round(clean * 1e3, 2),
               "cold_clean_frac": round(nbytes / (clean * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"config: {row}")
        rows.append(row)
        del fn, keep, data, X
        torch.cuda.empty_cache()
    return rows


def solver_system(name: str):
    """(csr arrays, b, keyword arguments) of a solver leg's system at n =
    128^3: CG on the Poisson matrix with b = 1 and rtol 1e-6; MINRES on
    the Poisson matrix with shift -1; BiCGSTAB and GMRES(20) on the
    convection-diffusion variant (x-direction off-diagonals -1.3 and -0.7,
    diagonal 8) with b ~ U[-1, 1]; rtol 1e-5."""
    from mlx_sparse import synthetic

    m = synthetic.poisson_3d(128)
    n = m.shape[0]
    if name == "cg":
        return m, m.data, np.ones(n, np.float32), {"rtol": 1e-6}
    b = synthetic.uniform(n, -1.0, 1.0, seed=7)
    if name == "minres":
        return m, m.data, b, {"rtol": 1e-5, "maxiter": 500, "shift": -1.0}
    rows = np.repeat(np.arange(n), np.diff(m.indptr))
    cols = m.indices.astype(np.int64)
    conv = m.data.copy()
    conv[cols == rows + 1] = -0.7
    conv[cols == rows - 1] = -1.3
    conv[cols == rows] = 8.0
    kw = {"rtol": 1e-5, "maxiter": 500}
    if name == "gmres":
        kw["restart"] = 20
    return m, conv, b, kw


def cpu_solver_baselines(result: dict) -> dict:
    """Part of the CPU baseline leg: the oracle's single-threaded
    restatements of the reference solver loops timed on the solver legs'
    systems (``solver_system``) - CG over 20 iterations, MINRES and BiCGSTAB
    over their whole solves, GMRES over one cycle of 20 steps - and the
    per-iteration speedup of the device loops in ``result``, whose rows gain
    ``cpu_us_per_iteration`` and ``speedup_per_iteration`` in place."""
    from oracle import oracle as orc

    runs = {"cg": (orc.csr_cg, {"maxiter": 20}),
            "minres": (orc.csr_minres, {}),
            "bicgstab": (orc.csr_bicgstab, {}),
            "gmres": (orc.csr_gmres, {"maxiter": 20})}
    krylov = result.get("krylov") or {}
    rows = {"cg": result.get("cg"), "minres": krylov.get("minres"),
            "bicgstab": krylov.get("bicgstab"), "gmres": krylov.get("gmres")}
    out = {}
    for name, (f, over) in runs.items():
        if rows[name] is None:
            continue
        m, data, b_np, kw = solver_system(name)
        t0 = time.perf_counter()
        _, _, _, its = f(data, m.indices, m.indptr, b_np, **{**kw, **over})
        cpu_us = (time.perf_counter() - t0) / max(its, 1) * 1e6
        out[name] = {"us_per_iteration": round(cpu_us, 1), "iterations": its}
        rows[name]["cpu_us_per_iteration"] = round(cpu_us, 1)
        rows[name]["cpu_iterations"] = its
        rows[name]["speedup_per_iteration"] = round(cpu_us / rows[name]["us_per_iteration"], 1)
        log(f"cpu {name}: {out[name]}")
    return out


def profile_solver(dev, name: str) -> dict:
    """One solver alone, for rocprofv3 --kernel-trace --stats: its system
    (``solver_system``), a warm-up solve (plan, allocator), then one timed
    solve."""
    import mlx_sparse as ms
    from mlx_sparse import linalg

    m, data, b_np, kw = solver_system(name)
    A = ms.csr_array((data, m.indices, m.indptr), shape=m.shape, canonical=True)
    b = torch.from_numpy(b_np).to(dev)
    solver = getattr(linalg, name)
    solver(A, b, **kw)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    x, info = solver(A, b, return_info=True, **kw)
    torch.cuda.synchronize()
    t = time.perf_counter() - t0
    return {"profile_solver": name, "n": m.shape[0], "info": info.status,
            "iterations": info.iterations, "residual": info.residual_norm,
            "solve_ms": round(t * 1e3, 2),
            "us_per_iteration": round(t / max(info.iterations, 1) * 1e6, 1)}


def profile_case(ext, dev, case: str, calls: int) -> dict:
    """One configuration alone, for rocprofv3 (kernel trace or counters):
    a 1 GiB copy of known traffic (the counters' scale), then ``calls``
    back-to-back calls through the case's bound plan, synchronised."""
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()
    label, kind, dt, k = CASES[case]
    m = _matrix(kind)
    data, X = _operands(case, m, dev)
    fn, info, nbytes, nflops, keep = _case_call(ext, case, m, data, X, dev)
    torch.cuda.synchronize()
    t_ms = _events_time(fn, calls)
    return {"profile_case": case, "label": label, "calls": calls, "nnz": m.nnz,
            "plan": _kind(info), "compulsory_bytes": nbytes, "flops": nflops,
            "events_us_per_call": round(t_ms * 1e3, 2)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-spmm", action="store_true", help="skip the SpMM leg")
    ap.add_argument("--no-adjoint", action="store_true", help="skip the adjoint leg")
    ap.add_argument("--no-cg", action="store_true", help="skip the conjugate gradient leg")
    ap.add_argument("--no-krylov", action="store_true", help="skip the BiCGSTAB / MINRES leg")
    ap.add_argument("--mtx", default=None,
                    help="also time SpMV on a Matrix Market file (e.g. a SuiteSparse matrix)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the SpMV/SpMM rows of the other benchmark configurations")
    ap.add_argument("--calibrate", action="store_true",
                    help="first copy 1 GiB once (a kernel of known traffic for counter scaling)")
    ap.add_argument("--traffic", default=str(ROOT / "profiles" / "spmv_random16_traffic.txt"))
    ap.add_argument("--profile-case", default=None, choices=sorted(CASES),
                    help="run only this configuration (calls back to back, for rocprofv3)")
    ap.add_argument("--calls", type=int, default=10, help="calls of --profile-case")
    ap.add_argument("--profile-solver", default=None,
                    choices=["cg", "minres", "bicgstab", "gmres"],
                    help="run only this solver at n = 128^3 (two solves, for rocprofv3)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path).", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device.", file=sys.stderr)
        return 2

    import mlx_sparse as ms
    from mlx_sparse import _native, synthetic
    from mlx_sparse._ext_loader import extension

    ext = extension()
    ms.use_gpu(0)
    dev = torch.device("cuda", 0)
    if args.profile_case:
        print(json.dumps(profile_case(ext, dev, args.profile_case, args.calls)), flush=True)
        return 0
    if args.profile_solver:
        print(json.dumps(profile_solver(dev, args.profile_solver)), flush=True)
        return 0
    if args.calibrate:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration: copied 1 GiB (1073741824 bytes read, 1073741824 written)")
        del src, dst

    # ---- headline: random 16/row SpMV -----------------------------------------
    t0 = time.perf_counter()
    m = synthetic.random_fixed_row(1 << 22, 16, seed=0)
    x_np = synthetic.uniform(m.shape[1], -1.0, 1.0, seed=1)
    log(f"generated {m.name} nnz={m.nnz} in {time.perf_counter() - t0:.1f}s")
    A = ms.csr_array((m.data, m.indices, m.indptr), shape=m.shape)
    x = torch.from_numpy(x_np).to(dev)
    A.buffers(dev)  # the matrix on the device: the copy is not the plan's cost
    torch.cuda.synchronize()

    # The first build in the process also loads the build kernels' code; a
    # second build of the same matrix (then freed) gives the plan's own cost.
    t0 = time.perf_counter()
    plan = A.plan(dev)
    torch.cuda.synchronize()
    plan_ms = (time.perf_counter() - t0) * 1e3
    info = plan.info()
    d_, i_, p_ = A.buffers(dev)
    t0 = time.perf_counter()
    again = _native.csr_plan(p_, m.shape[0], m.nnz, data=d_, indices=i_, n_cols=m.shape[1])
    torch.cuda.synchronize()
    rebuild_ms = (time.perf_counter() - t0) * 1e3
    del again, d_, i_, p_
    log(f"plan: {info} built in {plan_ms:.1f} ms (again: {rebuild_ms:.1f} ms)")

    nbytes = synthetic.compulsory_bytes(m.nnz, m.shape[0], m.shape[1], 4, 4)
    nflops = synthetic.flops(m.nnz)

    def step():
        return A @ x

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        y = step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / args.steps * 1e3
    value = nbytes / (wall / args.steps) / 1e9
    log(f"api step: {ms_per_step * 1e3:.1f} us  {value:.0f} GB/s")

    # kernel-only timing: SpMV calls on torch's current stream, replayed from
    # a HIP graph so that host overhead does not show between kernels
    data, indices, indptr = A.buffers(dev)

    def launch():
        return ext.csr_matvec(data, indices, indptr, x, m.shape[0], m.shape[1], plan=plan)

    kern_t, y_graph = _graph_time(launch)
    if not torch.equal(y_graph, y):
        raise RuntimeError("kernel-timing output differs from the API step output")
    kern_ms = kern_t.mean  # the average launch duration (the rocprofv3 average's twin)
    events_ms = _events_time(launch, args.steps)
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    log(f"kernel (graph replay): {kern_ms * 1e3:.1f} us  {achieved:.0f} GB/s  "
        f"{achieved / HBM_PEAK_GBS:.3f} of peak; back-to-back API calls {events_ms * 1e3:.1f} us")

    scratch = torch.empty(1 << 28, dtype=torch.float32, device=dev)  # 1 GiB
    cold_ms = _cold_time(launch, 30, scratch)
    cold_gbs = nbytes / (cold_ms * 1e-3) / 1e9
    clean_ms = _cold_time(launch, 30, scratch, clean=True)
    clean_gbs = nbytes / (clean_ms * 1e-3) / 1e9
    log(f"cold: {cold_ms * 1e3:.1f} us  {cold_gbs:.0f} GB/s; after a write and a read: "
        f"{clean_ms * 1e3:.1f} us")

    plan_kind = "panels" if info.get("n_panels") else ("slices" if info.get("n_slices") else "blocks")
    traffic = None
    tf = Path(args.traffic)
    if tf.exists():
        fields = dict(line.split(":", 1) for line in tf.read_text().splitlines()
                      if ":" in line and not line.startswith("#"))
        if fields.get("plan_kind", "").strip() == plan_kind and "hbm_bytes_per_call" in fields:
            traffic = int(fields["hbm_bytes_per_call"].strip())

    result = {
        "metric": "CSR SpMV effective HBM GB/s (% of peak) + SpMM GFLOP/s, fp32, 1xMI355X",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded): uniform random columns, N(0,1) values, x~U[-1,1]",
        "config": {"workload": "csr_spmv random16 n=4194304 nnz=67108864 f32/i32",
                   "n_rows": m.shape[0], "nnz": m.nnz, "index": "int32",
                   "compulsory_bytes": nbytes, "plan_build_ms": round(plan_ms, 3),
                   "plan_rebuild_ms": round(rebuild_ms, 3),
                   "plan": {"kind": plan_kind,
                            **{k: info[k] for k in ("block_nnz", "n_blocks", "n_long_rows",
                                                    "n_slices", "n_panels", "n_tiles",
                                                    "panel_values", "plan_bytes")}}},
        "gflops": round(nflops / (ms_per_step * 1e-3) / 1e9, 2),
        "pct_of_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "kernel": {"panels": "panel_products<F32> + panel_rows<F32,int>",
                                "slices": "spmv_sliced<F32> + slice_merge<F32>"}.get(
                                    plan_kind, f"spmv_blocks<F32,int,{info['block_nnz']}>"),
                     "kernel_us": round(kern_ms * 1e3, 2),
                     "kernel_us_median": round(float(kern_t) * 1e3, 2),
                     "frac_median": round(nbytes / (float(kern_t) * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "cold_kernel_us": round(cold_ms * 1e3, 2),
                     "cold_frac": round(cold_gbs / HBM_PEAK_GBS, 4),
                     "cold_clean_kernel_us": round(clean_ms * 1e3, 2),
                     "cold_clean_frac": round(clean_gbs / HBM_PEAK_GBS, 4),
                     "plan_bytes": info["plan_bytes"],
                     "footprint_bytes": {"matrix": m.nnz * 8 + (m.shape[0] + 1) * 4,
                                         "plan": info["plan_bytes"],
                                         "noalloc_scratch": NOALLOC_SCRATCH_BYTES},
                     "timing": ("HIP-graph replays of 20 calls, 50 replays each between "
                                "HIP events: kernel_us / achieved / frac use the mean per "
                                "call (the average launch duration), kernel_us_median the "
                                "median over replays; cold: median of 30 calls after a "
                                "1 GiB write; cold_clean: after a 1 GiB write and a 1 GiB "
                                "read (no dirty lines of the flush left to write back)")},
        "cold": {"kernel_us": round(cold_ms * 1e3, 2), "gbs": round(cold_gbs, 1),
                 "frac": round(cold_gbs / HBM_PEAK_GBS, 4)},
    }
    del y

    # ---- adjoint path on the headline matrix ---------------------------------------
    if not args.no_adjoint:
        result["adjoint"] = adjoint_leg(ext, A, m, x, nbytes)
        torch.cuda.empty_cache()

    # ---- SpMM k=64 on the 3D Poisson matrix --------------------------------------
    if not args.no_spmm:
        spmv_gflops_cfg2 = nflops / (kern_ms * 1e-3) / 1e9
        del A, x, data, indices, indptr, plan
        torch.cuda.empty_cache()
        p = synthetic.poisson_3d(128)
        P = ms.csr_array((p.data, p.indices, p.indptr), shape=p.shape)
        xp = torch.from_numpy(synthetic.uniform(p.shape[1], -1.0, 1.0, seed=1)).to(dev)
        Xp = torch.from_numpy(synthetic.normal(p.shape[1], seed=2, k=64)).to(dev)
        pd, pi, pp = P.buffers(dev)
        pplan = P.plan(dev)
        spmv_ms, _ = _graph_time(lambda: ext.csr_matvec(pd, pi, pp, xp, p.shape[0], p.shape[1],
                                                        plan=pplan))
        spmm_ms, _ = _graph_time(lambda: ext.csr_matmul(pd, pi, pp, Xp, p.shape[0], p.shape[1],
                                                        plan=pplan), calls=10)
        for _ in range(3):
            P @ Xp
        spmm_cold = _cold_time(lambda: ext.csr_matmul(pd, pi, pp, Xp, p.shape[0], p.shape[1],
                                                      plan=pplan), 15, scratch)
        f_spmv = synthetic.flops(p.nnz)
        f_spmm = synthetic.flops(p.nnz, 64)
        b_spmm = synthetic.compulsory_bytes(p.nnz, p.shape[0], p.shape[1], 4, 4, k=64)
        b_spmv = synthetic.compulsory_bytes(p.nnz, p.shape[0], p.shape[1], 4, 4)
        g_spmv = f_spmv / (spmv_ms * 1e-3) / 1e9
        g_spmm = f_spmm / (spmm_ms * 1e-3) / 1e9
        result["spmm"] = {
            "workload": "poisson3d 128^3 n=2097152 nnz=14581760, X n x 64 row-major, f32/i32",
            "k": 64, "kernel_us": round(spmm_ms * 1e3, 2), "gflops": round(g_spmm, 1),
            "gbs": round(b_spmm / (spmm_ms * 1e-3) / 1e9, 1),
            "frac": round(b_spmm / (spmm_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "cold_us": round(spmm_cold * 1e3, 2),
            "cold_frac": round(b_spmm / (spmm_cold * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "spmv_same_matrix_us": round(spmv_ms * 1e3, 2),
            "spmv_same_matrix_gflops": round(g_spmv, 1),
            "spmv_same_matrix_gbs": round(b_spmv / (spmv_ms * 1e-3) / 1e9, 1),
            "ratio_vs_spmv_same_matrix": round(g_spmm / g_spmv, 2),
            "ratio_vs_headline_spmv": round(g_spmm / spmv_gflops_cfg2, 2),
        }
        log(f"spmm k=64: {spmm_ms * 1e3:.1f} us {g_spmm:.0f} GFLOP/s; spmv same matrix "
            f"{spmv_ms * 1e3:.1f} us {g_spmv:.0f} GFLOP/s")

        # batched SpMV: 8 vectors through the native batched entry point
        # (transpose, one SpMM with k = 8, transpose back)
        B = 8
        Vb = torch.from_numpy(synthetic.normal(p.shape[1], seed=3, k=B).T.copy()).to(dev)
        # (events around back-to-back calls: the call takes stream-ordered
        # scratch, which this leg does not put under graph capture)
        bat_call = lambda: ext.csr_batched_matvec(pd, pi, pp, Vb, p.shape[0], p.shape[1])
        for _ in range(3):
            bat_call()
        bat_ms = _events_time(bat_call, 20)
        b_bat = p.nnz * 8 + (p.shape[0] + 1) * 4 + B * 4 * (p.shape[0] + p.shape[1])
        result["batched_spmv"] = {
            "workload": "poisson3d 128^3, 8 vectors (8 x n row-major), f32/i32",
            "batch": B, "kernel_us": round(bat_ms * 1e3, 2),
            "gbs": round(b_bat / (bat_ms * 1e-3) / 1e9, 1),
            "frac": round(b_bat / (bat_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "speedup_vs_8_spmv": round(B * spmv_ms / bat_ms, 2),
        }
        log(f"batched spmv x{B}: {bat_ms * 1e3:.1f} us ({B * spmv_ms * 1e3:.1f} us as {B} SpMVs)")
        del P, Xp, xp, pd, pi, pp, pplan, Vb

    # ---- a Matrix Market matrix, when given -------------------------------------
    if args.mtx:
        result["mtx"] = mtx_leg(ext, args.mtx, dev)
        torch.cuda.empty_cache()

    # ---- every benchmark configuration -------------------------------------------------
    if not args.no_configs:
        head = {"case": "cfg2 random16 n=2^22 f32/i32 (headline)", "nnz": m.nnz, "op": "spmv",
                "id": "cfg2", "plan": plan_kind, "plan_bytes": info["plan_bytes"],
                "block_nnz": info["block_nnz"], "window_rows": info["window_rows"],
                "long_rows": info["n_long_rows"], "compulsory_bytes": nbytes, "flops": nflops,
                "plan_build_ms": round(plan_ms, 2),
                "kernel_us": round(float(kern_t) * 1e3, 2),
                "kernel_us_mean": round(kern_ms * 1e3, 2),
                "gbs": round(nbytes / (float(kern_t) * 1e-3) / 1e9, 1),
                "frac": round(nbytes / (float(kern_t) * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "gflops": round(nflops / (float(kern_t) * 1e-3) / 1e9, 1),
                "cold_us": round(cold_ms * 1e3, 2),
                "cold_frac": round(cold_gbs / HBM_PEAK_GBS, 4),
                "cold_clean_us": round(clean_ms * 1e3, 2),
                "cold_clean_frac": round(clean_gbs / HBM_PEAK_GBS, 4)}
        result["configs"] = [head] + configs_leg(ext, dev, scratch)
        torch.cuda.empty_cache()

    # ---- conjugate gradients on the Poisson matrix --------------------------------
    if not args.no_cg:
        result["cg"] = cg_leg(dev)
        torch.cuda.empty_cache()

    # ---- BiCGSTAB and MINRES at the same size -----------------------------------------
    if not args.no_krylov:
        result["krylov"] = krylov_leg(dev)
        torch.cuda.empty_cache()

    # ---- CPU baseline (reference CPU kernel restated in C) -------------------------
    if not args.no_cpu:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(m, x_np)
        result["cpu_baseline"]["solvers"] = cpu_solver_baselines(result)
        log(f"cpu: {result['cpu_baseline']}")
    else:
        result["cpu_baseline"] = None

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
