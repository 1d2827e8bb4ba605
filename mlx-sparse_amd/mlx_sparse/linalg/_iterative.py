"""Krylov solvers on the path's SpMV (reference: mlx_sparse/linalg/_iterative.py:
69-323 ``cg``, :328-640 ``bicgstab``, :640-990 ``gmres``, :993-1145
``minres``; native loops src/linalg/cg/cg.cpp, src/preconditioners/pcg/pcg.cpp,
src/linalg/bicgstab/bicgstab.cpp, src/linalg/gmres/gmres.cpp,
src/linalg/minres/minres.cpp).

On the GPU each loop runs on the device (``msx_csr_cg``, ``msx_csr_bicgstab``,
``msx_csr_minres``): the path's SpMV with the matrix's cached plan, fused
vector passes, scalars on the device.  GMRES (``msx_csr_gmres``) runs each
Arnoldi step on the device and solves the small least-squares problem of a
restart cycle on the host, as the reference does.  With ``use_cpu()`` the
reference's sequential loops run natively.
"""

from __future__ import annotations

import torch

import mlx_sparse._native as _native
from mlx_sparse._csr import CSRArray
from mlx_sparse._device import default_torch_device
from mlx_sparse._validation import ensure_array
from mlx_sparse.linalg import preconditioners as _pc
from mlx_sparse.linalg._info import finish


def _float32_csr(A, solver: str = "cg") -> CSRArray:
    if not isinstance(A, CSRArray):
        if isinstance(A, torch.Tensor):
            raise TypeError("sparse iterative solvers expect a CSRArray; use torch.linalg for "
                            "dense arrays.")
        raise TypeError(f"sparse iterative solvers expect a CSRArray, got {type(A).__name__}.")
    if A.shape[0] != A.shape[1]:
        raise ValueError(f"{solver} requires a square matrix, got {A.shape}.")
    if A.dtype != torch.float32:
        if A.dtype.is_complex:
            raise TypeError("sparse iterative solvers currently use float32 values.")
        A = CSRArray(A.data.to(torch.float32), A.indices, A.indptr, A.shape,
                     A.sorted_indices, A.has_canonical_format)
    return A


def _float32_vector(x, device) -> torch.Tensor:
    t = ensure_array(x, device=device)
    if t.is_complex():
        raise TypeError("sparse iterative solvers currently use float32 values.")
    return t.to(torch.float32).contiguous()


def cg(A, b, *, x0=None, rtol: float = 1e-5, atol: float = 0.0, maxiter: int | None = None,
       M=None, callback=None, return_info: bool = False):
    """Solve a sparse SPD system ``A @ x = b`` with conjugate gradients.

    Stops when ``||r|| <= max(atol, rtol * ||b||)``.  ``maxiter`` defaults to
    ``10 * n``.  ``M``: ``None`` or ``preconditioners.identity`` (plain CG),
    ``preconditioners.diagonal`` / ``jacobi`` (Jacobi-preconditioned CG), or a
    rank-1 inverse diagonal.

    Returns ``(x, info)``: ``info`` 0 converged; > 0 the iteration count at
    which the budget ran out; < 0 breakdown (-1 near-zero denominator, -2
    non-positive preconditioned product, -3 non-finite).  With
    ``return_info=True`` a :class:`SolverInfo` replaces the integer.
    """
    csr = _float32_csr(A)
    device = default_torch_device()
    rhs = _float32_vector(b, device)
    if rhs.ndim != 1:
        raise ValueError(f"right-hand side must be rank-1, got {tuple(rhs.shape)}.")
    if rhs.shape[0] != csr.shape[0]:
        raise ValueError(f"b has length {rhs.shape[0]}, expected {csr.shape[0]}.")
    if x0 is None:
        guess = torch.zeros(csr.shape[1], dtype=torch.float32, device=device)
    else:
        guess = _float32_vector(x0, device)
        if guess.ndim != 1 or guess.shape[0] != csr.shape[1]:
            raise ValueError(f"x0 must have shape ({csr.shape[1]},), got {tuple(guess.shape)}.")
    maxiter_value = 10 * csr.shape[1] if maxiter is None else int(maxiter)
    if maxiter_value < 0:
        raise ValueError("maxiter must be non-negative.")
    data, indices, indptr = csr.buffers(device)
    plan = csr.plan(device)
    kind = None
    inv_diag = None
    if M is not None:
        pc = _pc.aspreconditioner(M, csr)
        kind = pc.kind
        if isinstance(pc, _pc.DiagonalPreconditioner):
            if pc.inverse_diagonal.shape[0] != csr.shape[0]:
                raise ValueError("preconditioner size does not match the matrix.")
            inv_diag = pc.inverse_diagonal.to(device=device, dtype=torch.float32).contiguous()
    if inv_diag is None:
        x, info, residual, iterations = _native.csr_cg(
            data, indices, indptr, rhs, guess, csr.shape, rtol=float(rtol), atol=float(atol),
            maxiter=maxiter_value, plan=plan)
    else:
        x, info, residual, iterations = _native.csr_pcg_jacobi(
            data, indices, indptr, rhs, guess, inv_diag, csr.shape, rtol=float(rtol),
            atol=float(atol), maxiter=maxiter_value, plan=plan)
    return finish(x, info, residual, iterations, solver="cg", return_info=bool(return_info),
                  callback=callback, rtol=float(rtol), atol=float(atol), maxiter=maxiter_value,
                  preconditioner=kind)


def _finite_scalar(name: str, value) -> float:
    scalar = float(value)
    if scalar != scalar or scalar in (float("inf"), float("-inf")):
        raise ValueError(f"{name} must be finite.")
    return scalar


def _normalize_tolerances(rtol, tol, atol) -> tuple[float, float]:
    """SciPy's ``tol`` alias of ``rtol`` (reference:
    mlx_sparse/linalg/_iterative.py:46-66)."""
    if rtol is None and tol is None:
        rtol_value = 1e-5
    elif rtol is None:
        rtol_value = _finite_scalar("tol", tol)
    else:
        rtol_value = _finite_scalar("rtol", rtol)
        if tol is not None and _finite_scalar("tol", tol) != rtol_value:
            raise ValueError("tol is a compatibility alias for rtol; do not set both.")
    atol_value = _finite_scalar("atol", atol)
    if rtol_value < 0.0:
        raise ValueError("rtol must be non-negative.")
    if atol_value < 0.0:
        raise ValueError("atol must be non-negative.")
    return float(rtol_value), float(atol_value)


def _system(A, b, x0, maxiter, solver: str):
    """(csr, rhs, guess, maxiter, device) of a square float32 system."""
    csr = _float32_csr(A, solver)
    device = default_torch_device()
    rhs = _float32_vector(b, device)
    if rhs.ndim != 1:
        raise ValueError(f"right-hand side must be rank-1, got {tuple(rhs.shape)}.")
    if rhs.shape[0] != csr.shape[0]:
        raise ValueError(f"b has length {rhs.shape[0]}, expected {csr.shape[0]}.")
    if x0 is None:
        guess = torch.zeros(csr.shape[1], dtype=torch.float32, device=device)
    else:
        guess = _float32_vector(x0, device)
        if guess.ndim != 1 or guess.shape[0] != csr.shape[1]:
            raise ValueError(f"x0 must have shape ({csr.shape[1]},), got {tuple(guess.shape)}.")
    maxiter_value = 10 * csr.shape[1] if maxiter is None else int(maxiter)
    if maxiter_value < 0:
        raise ValueError("maxiter must be non-negative.")
    return csr, rhs, guess, maxiter_value, device


# Solvers with a Jacobi-preconditioned loop (the reference's native
# diagonal paths: mlx_sparse/linalg/_iterative.py:437-461 csr_bicgstab_jacobi,
# :770-797 csr_gmres_jacobi, :1086-1110 csr_minres_jacobi).
_JACOBI_SOLVERS = {"bicgstab", "gmres", "minres"}


def _preconditioner(M, csr, solver: str, device):
    """(kind, pc, inverse diagonal or None) of ``M``: None or the identity
    run the plain loop; a diagonal/Jacobi preconditioner runs the solver's
    Jacobi loop; other kinds raise."""
    if M is None:
        return None, None, None
    minres_text = ("minres currently supports only identity, diagonal, and Jacobi "
                   "symmetric positive-definite native-backed preconditioners.")
    try:
        pc = _pc.aspreconditioner(M, csr)
    except TypeError:
        if solver == "minres" and not isinstance(M, CSRArray):
            raise TypeError(minres_text) from None  # the reference's text (:1118-1122)
        raise
    if isinstance(pc, _pc.IdentityPreconditioner):
        return pc.kind, pc, None
    if isinstance(pc, _pc.DiagonalPreconditioner) and solver in _JACOBI_SOLVERS:
        if pc.inverse_diagonal.shape[0] != csr.shape[0]:
            raise ValueError("preconditioner size does not match the matrix.")
        inv = pc.inverse_diagonal.to(device=device, dtype=torch.float32).contiguous()
        return pc.kind, pc, inv
    if solver == "minres":
        raise TypeError(minres_text)
    supported = "identity and diagonal/Jacobi" if solver in _JACOBI_SOLVERS else "identity"
    raise TypeError(f"{solver} in this build supports only the {supported} preconditioners; "
                    f"got {pc.kind}.")


def bicgstab(A, b, x0=None, *, rtol: float | None = None, atol: float = 0.0,
             tol: float | None = None, maxiter: int | None = None, M=None, callback=None,
             return_info: bool = False):
    """Solve a square (non-symmetric) sparse system ``A @ x = b`` with
    BiCGSTAB (reference: mlx_sparse/linalg/_iterative.py:328-640).

    Two SpMVs per iteration; convergence is confirmed on the true residual
    ``||b - A @ x|| <= max(rtol * ||b||, atol)``.  ``rtol`` defaults to
    ``1e-5``; ``tol`` is SciPy's alias for it (both may be given only when
    equal).  ``maxiter`` defaults to ``10 * n``.

    ``M``: ``None``, ``preconditioners.identity`` or a diagonal/Jacobi
    preconditioner (the reference's Jacobi loop: x advances along
    ``M @ p`` and ``M @ s``).

    Returns ``(x, info)``: ``info`` 0 converged, > 0 the iteration budget
    ran out, -1 breakdown (near-zero ``rho``, ``alpha`` denominator or
    ``omega``), -3 non-finite values.  With ``return_info=True`` a
    :class:`SolverInfo` replaces the integer.
    """
    rtol_value, atol_value = _normalize_tolerances(rtol, tol, atol)
    csr, rhs, guess, maxiter_value, device = _system(A, b, x0, maxiter, "bicgstab")
    kind, _, inv_diag = _preconditioner(M, csr, "bicgstab", device)
    data, indices, indptr = csr.buffers(device)
    if inv_diag is None:
        x, info, residual, iterations = _native.csr_bicgstab(
            data, indices, indptr, rhs, guess, csr.shape, rtol=rtol_value, atol=atol_value,
            maxiter=maxiter_value, plan=csr.plan(device))
    else:
        x, info, residual, iterations = _native.csr_bicgstab_jacobi(
            data, indices, indptr, rhs, guess, inv_diag, csr.shape, rtol=rtol_value,
            atol=atol_value, maxiter=maxiter_value, plan=csr.plan(device))
    return finish(x, info, residual, iterations, solver="bicgstab", return_info=bool(return_info),
                  callback=callback, rtol=rtol_value, atol=atol_value, maxiter=maxiter_value,
                  preconditioner=kind)


def minres(A, b, *, x0=None, rtol: float = 1e-5, atol: float = 0.0, shift: float = 0.0,
           maxiter: int | None = None, M=None, check_preconditioner: bool = True,
           callback=None, return_info: bool = False):
    """Solve a symmetric (possibly indefinite) sparse system
    ``(A - shift * I) @ x = b`` with MINRES (reference:
    mlx_sparse/linalg/_iterative.py:993-1145; SciPy's ``shift`` convention).

    Two SpMVs per iteration (the Lanczos step and the true residual the
    reference tests every iteration).  Stops when
    ``||b - (A - shift I) x|| <= max(rtol * ||b||, atol)``.  ``maxiter``
    defaults to ``10 * n``.  ``M``: ``None``, ``preconditioners.identity``
    or a diagonal/Jacobi preconditioner, which must be symmetric positive
    definite (checked unless ``check_preconditioner=False``; the loop then
    ends with -2 on a non-positive entry).  Returns ``(x, info)`` as
    :func:`bicgstab` does, plus -2: a non-positive preconditioned product.
    """
    csr, rhs, guess, maxiter_value, device = _system(A, b, x0, maxiter, "minres")
    shift_value = _finite_scalar("shift", shift)
    kind, pc, inv_diag = _preconditioner(M, csr, "minres", device)
    data, indices, indptr = csr.buffers(device)
    if inv_diag is None:
        x, info, residual, iterations = _native.csr_minres(
            data, indices, indptr, rhs, guess, csr.shape, rtol=float(rtol), atol=float(atol),
            maxiter=maxiter_value, shift=shift_value, plan=csr.plan(device))
    else:
        # reference: mlx_sparse/linalg/_iterative.py:1087-1096
        if check_preconditioner and (not pc.is_symmetric
                                     or not bool(torch.isfinite(inv_diag).all())
                                     or not bool((inv_diag > 0.0).all())):
            raise ValueError("minres requires a symmetric positive-definite preconditioner; "
                             "diagonal inverse entries must be finite and strictly positive.")
        x, info, residual, iterations = _native.csr_minres_jacobi(
            data, indices, indptr, rhs, guess, inv_diag, csr.shape, rtol=float(rtol),
            atol=float(atol), maxiter=maxiter_value, shift=shift_value, plan=csr.plan(device))
    return finish(x, info, residual, iterations, solver="minres", return_info=bool(return_info),
                  callback=callback, rtol=float(rtol), atol=float(atol), maxiter=maxiter_value,
                  preconditioner=kind)


def gmres(A, b, *, x0=None, rtol: float = 1e-5, atol: float = 0.0, restart: int | None = None,
          maxiter: int | None = None, M=None, callback=None, callback_type: str = "x",
          return_info: bool = False):
    """Solve a square (not necessarily symmetric) sparse system ``A @ x = b``
    with restarted GMRES (reference: mlx_sparse/linalg/_iterative.py:640-990).

    Each cycle builds an Arnoldi basis of ``restart`` vectors (default
    ``min(20, n)``; one SpMV per step) from the true residual and minimises
    the residual over it.  ``maxiter`` counts SpMVs over all cycles (default
    ``10 * n``).  Stops when ``||b - A x|| <= max(atol, rtol * ||b||)``,
    tested between cycles.  ``M``: ``None``, ``preconditioners.identity`` or
    a diagonal/Jacobi preconditioner (left preconditioning: the Arnoldi
    basis of ``M @ A``, each cycle from ``M @ r``).
    ``callback`` is called once after the solve, with ``x``
    (``callback_type="x"``) or the final residual norm ("pr_norm",
    "legacy").

    Returns ``(x, info)``: ``info`` 0 converged, > 0 the budget ran out, -1
    a failed least-squares solve, -3 non-finite values.  With
    ``return_info=True`` a :class:`SolverInfo` replaces the integer.
    """
    if callback_type not in {"x", "pr_norm", "legacy"}:
        raise ValueError("callback_type must be 'x', 'pr_norm', or 'legacy'.")
    csr, rhs, guess, maxiter_value, device = _system(A, b, x0, maxiter, "gmres")
    restart_value = min(20, csr.shape[0]) if restart is None else int(restart)
    if restart_value <= 0:
        raise ValueError("restart must be positive.")
    kind, _, inv_diag = _preconditioner(M, csr, "gmres", device)
    data, indices, indptr = csr.buffers(device)
    if inv_diag is None:
        x, info, residual, iterations = _native.csr_gmres(
            data, indices, indptr, rhs, guess, csr.shape, rtol=float(rtol), atol=float(atol),
            restart=restart_value, maxiter=maxiter_value, plan=csr.plan(device))
    else:
        x, info, residual, iterations = _native.csr_gmres_jacobi(
            data, indices, indptr, rhs, guess, inv_diag, csr.shape, rtol=float(rtol),
            atol=float(atol), restart=restart_value, maxiter=maxiter_value,
            plan=csr.plan(device))
    return finish(x, info, residual, iterations, solver="gmres", return_info=bool(return_info),
                  callback=callback, callback_type=callback_type, rtol=float(rtol),
                  atol=float(atol), maxiter=maxiter_value, restart=restart_value,
                  preconditioner=kind)
