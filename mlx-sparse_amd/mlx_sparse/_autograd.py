"""Differentiation rules of the CSR products, as torch autograd Functions
(reference: src/sparse/csr_matvec/csr_matvec.cpp:205-275 ``CSRMatVec::jvp``,
``::vjp``, ``::vmap``; src/sparse/csr_matmul/csr_matmul.cpp:302-380
``CSRMatMul::jvp``, ``::vjp``, ``::vmap``).

For ``y = A x`` with cotangent ``g``:

- gradient of the stored values: ``g[row(p)] * conj(x[col(p)])``
  (``csr_matvec_data_vjp``);
- gradient of ``x``: ``A^H g`` (``csr_matvec_transpose`` on ``conj(data)``).

For ``Y = A X`` the same with rows of ``X`` and ``G`` (``csr_matmul_data_vjp``,
``csr_matmul_transpose``).  Tangents: ``dA x + A dx``.  ``torch.func.vmap``
over the dense operand runs the batched kernels (sparse operands must stay
unmapped, as in the reference).

The ``A^H g`` products on the GPU take one of two routes, chosen by the
``gpu_adjoint`` runtime option: an atomic scatter over A's rows (one pass,
no set-up, the order of additions free) or a cached CSR of ``A^H`` built
once per matrix and multiplied with the forward kernels (deterministic).
"auto" scatters on a matrix's first adjoint product and caches the
transpose from the second one on.  On the CPU the reference's algorithm
runs (per-range partial outputs added in range order).
"""

from __future__ import annotations

import torch

import mlx_sparse._native as _native


def _conj(t: torch.Tensor) -> torch.Tensor:
    return t.conj().resolve_conj() if t.is_complex() else t


def _adjoint_csr(a, data: torch.Tensor):
    """CSR of A^H on data's device (None when the route is atomic): the
    array's cached (conjugate) transpose, which follows in-place updates of
    its values (``CSRArray._transpose_on``)."""
    from mlx_sparse import runtime

    device = data.device
    if device.type != "cuda":
        return None
    mode = runtime.get(runtime.RuntimeOption.GPU_ADJOINT)
    if mode == "atomic":
        return None
    if mode == "auto":
        seen = ("adjoint_calls", str(device))
        a._cache[seen] = a._cache.get(seen, 0) + 1
        if a._cache[seen] < 2:
            return None
    # real values: A^H is A^T, shared with the array's own cached transpose
    return a._transpose_on(device, conjugate=a.data.is_complex())


def _own_plan(a, data: torch.Tensor):
    """``a``'s plan when ``data`` is the very buffer the plan is bound to
    (``a``'s values, contiguous on their device), else None: values
    elsewhere run plan-free."""
    bufs = a.buffers(data.device)
    if data.data_ptr() != bufs[0].data_ptr() or not data.is_contiguous():
        return None
    return a.plan(data.device)


def rmatvec(a, data: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """A^H g for a vector g of length n_rows (native; plain tensors)."""
    _, indices, indptr = a.buffers(data.device)
    ah = _adjoint_csr(a, data)
    if ah is not None:
        d, i, p = ah.buffers(data.device)
        return _native.csr_matvec(d, i, p, g, ah.shape, plan=ah.plan(data.device))
    return _native.csr_matvec_transpose(_conj(data), indices, indptr, g, a.shape)


def rmatmat(a, data: torch.Tensor, G: torch.Tensor) -> torch.Tensor:
    """A^H G for G of shape (n_rows, k) (native; plain tensors)."""
    _, indices, indptr = a.buffers(data.device)
    ah = _adjoint_csr(a, data)
    if ah is not None:
        d, i, p = ah.buffers(data.device)
        return _native.csr_matmul(d, i, p, G, ah.shape, plan=ah.plan(data.device))
    return _native.csr_matmul_transpose(_conj(data), indices, indptr, G, a.shape)


_SECOND_ORDER = ("second-order derivatives of CSR products with respect to the stored values "
                 "are not supported.")


def _no_mapped_sparse(name, d_dim):
    if d_dim is not None:
        raise ValueError(
            f"{name} vmap supports batching only the dense RHS. Sparse data, indices, "
            "and indptr/coordinate axes must be unmapped.")


class CSRMatVec(torch.autograd.Function):
    """``y = A x`` with ``A``'s values ``data`` and ``x`` differentiable.
    ``planned``: ``data`` are ``a``'s own values, so ``a``'s plan applies."""

    @staticmethod
    def forward(data, x, a, planned=True):
        _, indices, indptr = a.buffers(data.device)
        plan = _own_plan(a, data) if planned else None
        return _native.csr_matvec(data, indices, indptr, x, a.shape, plan=plan)

    @staticmethod
    def setup_context(ctx, inputs, output):
        data, x, a, planned = inputs
        ctx.a = a
        ctx.planned = planned
        ctx.save_for_backward(data, x)
        ctx.save_for_forward(data, x)

    @staticmethod
    def backward(ctx, g):
        data, x = ctx.saved_tensors
        g_data = g_x = None
        if ctx.needs_input_grad[0]:
            g_data = MatVecDataVjp.apply(x, g, ctx.a)
        if ctx.needs_input_grad[1]:
            g_x = AdjointMatVec.apply(data, g, ctx.a, ctx.planned)
        return g_data, g_x, None, None

    @staticmethod
    def jvp(ctx, t_data, t_x, _a, _p):
        data, x = ctx.saved_tensors
        out = None
        if t_data is not None:
            out = CSRMatVec.apply(t_data, x, ctx.a, False)
        if t_x is not None:
            term = CSRMatVec.apply(data, t_x, ctx.a, ctx.planned)
            out = term if out is None else out + term
        return out

    @staticmethod
    def vmap(info, in_dims, data, x, a, planned=True):
        _no_mapped_sparse("CSRMatVec", in_dims[0])
        if in_dims[1] is None:
            raise ValueError("CSRMatVec vmap requires the dense RHS to have a mapped axis.")
        _, indices, indptr = a.buffers(data.device)
        out = _native.csr_batched_matvec(data, indices, indptr, x.movedim(in_dims[1], 0),
                                         a.shape)
        return out, 0


class CSRMatMul(torch.autograd.Function):
    """``Y = A X`` (X of shape (n_cols, k)) with ``data`` and ``X``
    differentiable."""

    @staticmethod
    def forward(data, X, a, planned=True):
        _, indices, indptr = a.buffers(data.device)
        plan = _own_plan(a, data) if planned else None
        return _native.csr_matmul(data, indices, indptr, X, a.shape, plan=plan)

    @staticmethod
    def setup_context(ctx, inputs, output):
        data, X, a, planned = inputs
        ctx.a = a
        ctx.planned = planned
        ctx.save_for_backward(data, X)
        ctx.save_for_forward(data, X)

    @staticmethod
    def backward(ctx, G):
        data, X = ctx.saved_tensors
        g_data = g_X = None
        if ctx.needs_input_grad[0]:
            g_data = MatMulDataVjp.apply(X, G, ctx.a)
        if ctx.needs_input_grad[1]:
            g_X = AdjointMatMul.apply(data, G, ctx.a, ctx.planned)
        return g_data, g_X, None, None

    @staticmethod
    def jvp(ctx, t_data, t_X, _a, _p):
        data, X = ctx.saved_tensors
        out = None
        if t_data is not None:
            out = CSRMatMul.apply(t_data, X, ctx.a, False)
        if t_X is not None:
            term = CSRMatMul.apply(data, t_X, ctx.a, ctx.planned)
            out = term if out is None else out + term
        return out

    @staticmethod
    def vmap(info, in_dims, data, X, a, planned=True):
        _no_mapped_sparse("CSRMatMul", in_dims[0])
        if in_dims[1] is None:
            raise ValueError("CSRMatMul vmap requires the dense RHS to have a mapped axis.")
        _, indices, indptr = a.buffers(data.device)
        out = _native.csr_batched_matmul(data, indices, indptr, X.movedim(in_dims[1], 0),
                                         a.shape)
        return out, 0


class AdjointMatVec(torch.autograd.Function):
    """``A^H g``; its derivative in ``g`` is ``A`` again.  ``cached``: the
    values are ``a``'s own, so a cached transpose of ``a`` may serve."""

    @staticmethod
    def forward(data, g, a, cached=True):
        if cached:
            return rmatvec(a, data, g.contiguous())
        _, indices, indptr = a.buffers(data.device)
        return _native.csr_matvec_transpose(_conj(data), indices, indptr, g.contiguous(), a.shape)

    @staticmethod
    def setup_context(ctx, inputs, output):
        data, g, a, cached = inputs
        ctx.a = a
        ctx.cached = cached
        ctx.save_for_backward(data)

    @staticmethod
    def backward(ctx, go):
        (data,) = ctx.saved_tensors
        if ctx.needs_input_grad[0]:
            raise NotImplementedError(_SECOND_ORDER)
        return None, CSRMatVec.apply(data, go, ctx.a, ctx.cached), None, None


class AdjointMatMul(torch.autograd.Function):
    """``A^H G``; its derivative in ``G`` is ``A`` again."""

    @staticmethod
    def forward(data, G, a, cached=True):
        if cached:
            return rmatmat(a, data, G.contiguous())
        _, indices, indptr = a.buffers(data.device)
        return _native.csr_matmul_transpose(_conj(data), indices, indptr, G.contiguous(), a.shape)

    @staticmethod
    def setup_context(ctx, inputs, output):
        data, G, a, cached = inputs
        ctx.a = a
        ctx.cached = cached
        ctx.save_for_backward(data)

    @staticmethod
    def backward(ctx, go):
        (data,) = ctx.saved_tensors
        if ctx.needs_input_grad[0]:
            raise NotImplementedError(_SECOND_ORDER)
        return None, CSRMatMul.apply(data, go, ctx.a, ctx.cached), None, None


class MatVecDataVjp(torch.autograd.Function):
    """Gradient of ``A x`` in the stored values: ``g[row(p)] * conj(x[col(p)])``."""

    @staticmethod
    def forward(x, g, a):
        _, indices, indptr = a.buffers(x.device)
        # the gradient does not read the values: the plan serves whatever
        # values it is bound to
        return _native.csr_matvec_data_vjp(indices, indptr, _conj(x), g.contiguous(), a.shape,
                                           plan=a.plan(x.device))

    @staticmethod
    def setup_context(ctx, inputs, output):
        pass

    @staticmethod
    def backward(ctx, go):
        raise NotImplementedError(_SECOND_ORDER)


class MatMulDataVjp(torch.autograd.Function):
    """Gradient of ``A X`` in the stored values:
    ``sum_q G[row(p), q] * conj(X[col(p), q])``."""

    @staticmethod
    def forward(X, G, a):
        _, indices, indptr = a.buffers(X.device)
        return _native.csr_matmul_data_vjp(indices, indptr, _conj(X.contiguous()),
                                           G.contiguous(), a.shape)

    @staticmethod
    def setup_context(ctx, inputs, output):
        pass

    @staticmethod
    def backward(ctx, go):
        raise NotImplementedError(_SECOND_ORDER)
