"""Shared test helpers: dtype plumbing between numpy/torch/oracle and the
per-row parity tolerance of the path (|got - want| <= tol * sum|a_ij x_j|)."""

from __future__ import annotations

import numpy as np
import torch

TOL = {"float32": 1e-5, "complex64": 1e-5, "float16": 1e-2, "bfloat16": 1e-2}
TORCH = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16,
         "complex64": torch.complex64}


def storage(values: np.ndarray, vtype: str) -> np.ndarray:
    """float32/complex input -> numpy storage of `vtype` (bfloat16 as uint16
    bits, rounded to nearest even by torch)."""
    if vtype == "bfloat16":
        t = torch.from_numpy(np.ascontiguousarray(values, dtype=np.float32)).to(torch.bfloat16)
        return t.view(torch.int16).numpy().view(np.uint16)
    if vtype == "float16":
        return np.ascontiguousarray(values, dtype=np.float16)
    if vtype == "complex64":
        return np.ascontiguousarray(values, dtype=np.complex64)
    return np.ascontiguousarray(values, dtype=np.float32)


def to_torch(arr: np.ndarray, vtype: str | None = None, device="cpu") -> torch.Tensor:
    if vtype == "bfloat16":
        t = torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).view(torch.bfloat16)
    else:
        t = torch.from_numpy(np.ascontiguousarray(arr))
    return t.to(device)


def to_numpy(t: torch.Tensor) -> np.ndarray:
    """Tensor -> numpy storage (bfloat16 as uint16 bits)."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def widen(arr: np.ndarray, vtype: str) -> np.ndarray:
    """Storage -> float64 / complex128 values."""
    if vtype == "bfloat16":
        return (arr.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    if vtype == "complex64":
        return arr.astype(np.complex128)
    return arr.astype(np.float64)


def close_or_same_nonfinite(g: np.ndarray, w: np.ndarray, err: np.ndarray,
                            bound: np.ndarray) -> np.ndarray:
    """Entries that pass: ``err <= bound`` (False for a NaN error or bound),
    or both sides the same non-finite value (NaN and NaN, or infinities of one
    sign; for complex values, per component)."""
    ok = err <= bound
    if np.iscomplexobj(g) or np.iscomplexobj(w):
        g = np.asarray(g, dtype=np.complex128)
        w = np.asarray(w, dtype=np.complex128)
        same = (_same_nonfinite(g.real, w.real) & (_same_nonfinite(g.imag, w.imag)
                                                   | (g.imag == w.imag))) \
            | (_same_nonfinite(g.imag, w.imag) & (g.real == w.real))
    else:
        same = _same_nonfinite(g, w)
    return ok | same


def _same_nonfinite(g: np.ndarray, w: np.ndarray) -> np.ndarray:
    return (np.isnan(g) & np.isnan(w)) | (np.isinf(g) & (g == w))


def assert_rows_close(got: np.ndarray, want: np.ndarray, scale: np.ndarray, vtype: str,
                      what: str = "", exact: np.ndarray | None = None,
                      lengths: np.ndarray | None = None, min_len_exempt: int = 0) -> dict:
    """Per-row parity: |got - want| <= TOL[vtype] * scale (+ a denormal floor).

    With ``exact`` (float64 row sums), a row outside the bound still passes
    when it is at least as close to the exact sum as the oracle is AND the
    row holds at least ``min_len_exempt`` values: on such long rows the
    oracle's sequential float32 sum itself drifts past the tolerance (error
    ~ 2^-24 * sqrt(n) relative), and a GPU tree sum that is more accurate
    must not fail for that.  Such rows are counted in the returned report.
    """
    g = widen(got, vtype)
    w = widen(want, vtype)
    with np.errstate(invalid="ignore"):
        err = np.abs(g - w)
    bound = TOL[vtype] * scale + 1e-30
    bad = ~close_or_same_nonfinite(g, w, err, bound)
    report = {"rows_outside_tol_vs_oracle": int(bad.sum()), "exempt_rows": 0}
    if bad.any() and exact is not None:
        closer = np.abs(g - exact) <= np.abs(w - exact)
        long_enough = np.ones_like(bad) if lengths is None else (
            np.broadcast_to(lengths.reshape(-1, *([1] * (bad.ndim - 1))), bad.shape) >= min_len_exempt)
        exempt = bad & closer & long_enough
        report["exempt_rows"] = int(exempt.sum())
        if exempt.any():
            idx = np.argwhere(exempt)[0]
            report["example"] = {"row": idx.tolist(), "gpu_err_vs_exact": float(np.abs(g - exact)[tuple(idx)]),
                                 "oracle_err_vs_exact": float(np.abs(w - exact)[tuple(idx)]),
                                 "scale": float(scale[tuple(idx)])}
        bad = bad & ~exempt
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(
            f"{what}: {int(bad.sum())} entries outside {TOL[vtype]}*sum|a*x| "
            f"(first {idx.tolist()}: got {g[tuple(idx[0])]}, want {w[tuple(idx[0])]}, "
            f"scale {scale[tuple(idx[0])]})")
    with np.errstate(divide="ignore", invalid="ignore"):
        rel = np.where((scale > 0) & np.isfinite(err), err / np.maximum(scale, 1e-300), 0.0)
    report["max_rel_err"] = float(rel.max()) if rel.size else 0.0
    return report
