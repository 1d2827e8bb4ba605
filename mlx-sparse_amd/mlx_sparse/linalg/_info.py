"""Solver diagnostics (reference: mlx_sparse/linalg/utils/diagnostics/info.py:23-62,
status.py:54-88 ``status_reason``, callbacks.py:61-101 ``finish_solver_result``)."""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class SolverInfo:
    """Structured diagnostics of an iterative solve: status, true residual
    norm, iterations and a stable textual reason.  ``int(info)`` and
    ``info.info`` give the SciPy-style integer status."""

    solver: str
    status: int
    residual_norm: float
    iterations: int
    convergence_reason: str
    breakdown_reason: str | None
    message: str
    preconditioned_residual_norm: float | None = None
    rtol: float | None = None
    atol: float | None = None
    maxiter: int | None = None
    restart: int | None = None
    preconditioner: str | None = None

    @property
    def converged(self) -> bool:
        return self.status == 0

    @property
    def info(self) -> int:
        return self.status

    def __int__(self) -> int:
        return self.status


def status_reason(status: int) -> tuple[str, str | None, str]:
    """Stable diagnostic text for a native status code."""
    if status == 0:
        return "converged", None, "converged to the requested true-residual tolerance"
    if status > 0:
        return ("iteration_limit", None,
                "iteration budget exhausted before reaching the requested tolerance")
    if status == -1:
        return ("numerical_breakdown", "breakdown",
                "solver encountered a near-zero denominator or Krylov breakdown")
    if status == -2:
        return ("invalid_preconditioner_or_operator", "non_positive_preconditioned_inner_product",
                "solver encountered a non-positive preconditioned inner product")
    if status == -3:
        return ("non_finite", "non_finite",
                "solver encountered a non-finite scalar, vector, or preconditioner output")
    return ("numerical_breakdown", f"status_{status}",
            "solver reported an implementation-specific negative breakdown status")


def finish(x, status: int, residual: float, iterations: int, *, solver: str, return_info: bool,
           callback=None, callback_type: str | None = None, rtol=None, atol=None, maxiter=None,
           restart=None, preconditioner=None):
    """``(x, int)`` by default, ``(x, SolverInfo)`` with ``return_info``; a
    callback is called once after the solve, with ``x`` or, for
    ``callback_type`` "pr_norm" / "legacy", the final residual norm
    (reference: mlx_sparse/linalg/utils/diagnostics/callbacks.py:11-58)."""
    if return_info or callback is not None:
        reason, breakdown, message = status_reason(int(status))
        info = SolverInfo(solver=solver, status=int(status), residual_norm=float(residual),
                          iterations=int(iterations), convergence_reason=reason,
                          breakdown_reason=breakdown, message=message, rtol=rtol, atol=atol,
                          maxiter=maxiter, restart=restart, preconditioner=preconditioner)
        if callback is not None:
            if not callable(callback):
                raise TypeError(f"{solver} callback must be callable.")
            if callback_type in ("pr_norm", "legacy"):
                callback(info.preconditioned_residual_norm
                         if info.preconditioned_residual_norm is not None else info.residual_norm)
            else:
                callback(x)
        return x, info if return_info else info.status
    return x, int(status)
