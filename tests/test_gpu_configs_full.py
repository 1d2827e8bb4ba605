"""Every benchmark configuration at its full size on the GPU, through the
drop-in API and the cached bound plan that AUTO builds - the same plan and
kernels bench.py times for that configuration.

Bar (against oracle/csr_oracle.c on the same seeded inputs):

- rows the kernels sum in stored order (row blocks of short rows when rows
  average at most 32 values; every short row of a panel plan) and every
  float32 / float16 SpMM: equal bit for bit;
- everything else: |gpu - oracle| <= tol * sum_j |a_ij x_j| per row (1e-5
  float32 / complex64, 1e-2 float16 / bfloat16), rows of 10,000 values or
  more exempt only where the GPU sum is closer to the float64 sum.

Configurations: cfg1 2D Laplacian 1024^2 f32/i32; cfg2
random 16 per row, n = 4,194,304, f32/i32; cfg3 power law Zipf(2), n =
2,097,152, f32/i64; cfg4 3D Poisson 128^3 f32/i32, SpMV and SpMM at k = 8,
64, 256; cfg5 banded n = 1,048,576, half-bandwidth 32, 65 % fill: bf16, f16,
f32 and complex64 SpMV, bf16 and f16 SpMM at k = 64.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import assert_rows_close, storage, to_numpy, to_torch
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda"
LONG_ROW_EXEMPT = 10_000


def _kind(info) -> str:
    return "panels" if info["n_panels"] else ("slices" if info["n_slices"] else "blocks")


def _array(ms, m, data, vtype):
    return ms.csr_array((to_torch(data, vtype, DEV), torch.from_numpy(m.indices),
                         torch.from_numpy(m.indptr)), shape=m.shape)


def serial_rows(plan, indptr) -> np.ndarray:
    """Rows a row-block plan sums one lane per row in stored order: the rows
    of short blocks that do not hold at most 32 rows averaging more than 32
    values (csr_spmv.hip, spmv_blocks phase 2)."""
    b = plan.export()[0].numpy().astype(np.int64)
    ip = np.asarray(indptr, dtype=np.int64)
    flag = np.int64(1) << 31
    long_entry = (b[:-1] & flag) != 0
    r0, r1 = b[:-1] & ~flag, b[1:] & ~flag
    m = r1 - r0
    tree = (ip[r1] - ip[r0] > 32 * m) & (m <= 32)
    out = np.repeat(~long_entry & ~tree, m)
    assert out.shape[0] == ip.shape[0] - 1
    return out


def _spmv_check(ms, m, data, x, vtype, what, exact_max_len=None):
    A = _array(ms, m, data, vtype)
    info = A.plan().info()
    y = to_numpy(A @ to_torch(x, vtype, DEV))
    y2 = to_numpy(A @ to_torch(x, vtype, DEV))
    np.testing.assert_array_equal(y, y2, err_msg=f"{what}: repeat call")
    n = m.shape[0]
    want = orc.csr_matvec(data, m.indices, m.indptr, x, n, vtype=vtype, n_threads=8)
    lengths = np.diff(m.indptr.astype(np.int64))
    if exact_max_len is not None:
        short = lengths <= exact_max_len
        if _kind(info) == "blocks":
            short &= serial_rows(A.plan(), m.indptr)
        g, w = y[short], want[short]
        if vtype == "complex64":
            g, w = g.view(np.float32), w.view(np.float32)
        np.testing.assert_array_equal(g, w, err_msg=f"{what}: stored-order rows")
    rep = assert_rows_close(
        y, want, orc.row_scale(data, m.indices, m.indptr, x, n, vtype=vtype), vtype, what,
        exact=orc.row_exact(data, m.indices, m.indptr, x, n, vtype=vtype), lengths=lengths,
        min_len_exempt=LONG_ROW_EXEMPT)
    print(f"{what}: plan {_kind(info)} W={info['block_nnz']} long={info['n_long_rows']} {rep}",
          flush=True)
    return info


def _spmm_check(ms, m, data, X, vtype, what, exact):
    A = _array(ms, m, data, vtype)
    info = A.plan().info()
    Y = to_numpy(A @ to_torch(X, vtype, DEV))
    want = orc.csr_matmul(data, m.indices, m.indptr, X, m.shape[0], vtype=vtype, n_threads=8)
    if exact:
        np.testing.assert_array_equal(Y, want, err_msg=what)
    else:
        assert_rows_close(Y, want, orc.row_scale(data, m.indices, m.indptr, X, m.shape[0],
                                                 vtype=vtype), vtype, what)
    print(f"{what}: plan {_kind(info)} window_rows={info['window_rows']} "
          f"{'bit-exact' if exact else 'within tol'}", flush=True)
    return info


@pytest.fixture(scope="module")
def poisson():
    from mlx_sparse import synthetic

    return synthetic.poisson_3d(128)


@pytest.fixture(scope="module")
def banded():
    from mlx_sparse import synthetic

    return synthetic.banded(1 << 20, 32, 0.65, 70.0, seed=0)


def test_cfg1_laplacian_1024(gpu):
    from mlx_sparse import synthetic

    m = synthetic.laplacian_2d(1024)
    x = synthetic.uniform(m.shape[1], -1.0, 1.0, seed=1)
    info = _spmv_check(gpu, m, m.data, x, "float32", "cfg1 laplacian 1024^2", exact_max_len=256)
    assert m.nnz == 5_238_784 and _kind(info) == "blocks"


def test_cfg2_random16_through_api(gpu):
    from mlx_sparse import synthetic

    m = synthetic.random_fixed_row(1 << 22, 16, seed=0)
    x = synthetic.uniform(m.shape[1], -1.0, 1.0, seed=1)
    info = _spmv_check(gpu, m, m.data, x, "float32", "cfg2 random16 4M", exact_max_len=256)
    assert _kind(info) == "panels"


@pytest.fixture(scope="module")
def power_law():
    from mlx_sparse import synthetic

    return synthetic.power_law(1 << 21, 2.0, 200_000, seed=0)


def test_cfg3_power_law_int64(gpu, power_law):
    """LDS panels with the long rows as 64-value virtual rows (AUTO's
    choice): every short row equal to the oracle."""
    from mlx_sparse import synthetic

    m = power_law
    assert m.indices.dtype == np.int64
    x = synthetic.uniform(m.shape[1], 0.0, 1.0, seed=1)
    info = _spmv_check(gpu, m, m.data, x, "float32", "cfg3 power law 2M", exact_max_len=256)
    assert _kind(info) == "panels" and info["n_long_rows"] > 1000


def test_cfg3_power_law_row_blocks(gpu, power_law):
    """The same matrix with the panel copy off: row blocks plus the
    XCD-sliced long rows in the same launch (x is 8 MB, every long row
    sorted); rows of blocks summed one lane per row in stored order equal."""
    from mlx_sparse import runtime, synthetic

    m = power_law
    x = synthetic.uniform(m.shape[1], 0.0, 1.0, seed=1)
    with runtime.context(gpu_slice="off"):
        info = _spmv_check(gpu, m, m.data, x, "float32", "cfg3 power law 2M blocks",
                           exact_max_len=256)
    assert _kind(info) == "blocks" and info["n_long_rows"] > 1000


def test_cfg4_poisson_spmv(gpu, poisson):
    from mlx_sparse import synthetic

    x = synthetic.uniform(poisson.shape[1], -1.0, 1.0, seed=1)
    info = _spmv_check(gpu, poisson, poisson.data, x, "float32", "cfg4 poisson 128^3",
                       exact_max_len=256)
    assert poisson.nnz == 14_581_760 and _kind(info) == "blocks"


@pytest.mark.parametrize("k", [8, 64, 256])
def test_cfg4_poisson_spmm(gpu, poisson, k):
    from mlx_sparse import synthetic

    X = synthetic.normal(poisson.shape[1], seed=2, k=k)
    _spmm_check(gpu, poisson, poisson.data, X, "float32", f"cfg4 poisson spmm k={k}", exact=True)


@pytest.mark.parametrize("vtype", ["bfloat16", "float16", "float32", "complex64"])
def test_cfg5_banded_spmv(gpu, banded, vtype):
    from mlx_sparse import synthetic

    x = synthetic.uniform(banded.shape[1], -1.0, 1.0, seed=1)
    if vtype == "complex64":
        data = synthetic.complex_values(banded, seed=3)
        xv = storage(x + 1j * synthetic.uniform(banded.shape[1], -1.0, 1.0, seed=5), vtype)
    else:
        data, xv = storage(banded.data, vtype), storage(x, vtype)
    info = _spmv_check(gpu, banded, data, xv, vtype, f"cfg5 banded {vtype}")
    assert 44_000_000 < banded.nnz < 45_500_000 and _kind(info) == "blocks"


@pytest.mark.parametrize("vtype", ["float16", "bfloat16"])
def test_cfg5_banded_spmm_k64(gpu, banded, vtype):
    """The column-window SpMM on the matrix cores (each 32-row tile's
    window densified in LDS, v_mfma_f32_16x16x32 with float32
    accumulation, one rounding): within the 16-bit tolerance of the
    oracle's stored-order sums."""
    from mlx_sparse import synthetic

    X = storage(synthetic.normal(banded.shape[1], seed=2, k=64), vtype)
    info = _spmm_check(gpu, banded, storage(banded.data, vtype), X, vtype,
                       f"cfg5 banded {vtype} spmm k=64", exact=False)
    assert 0 < info["window_rows"] <= 32 + 2 * 32


def test_cfg2_value_gradient_full_size(gpu):
    """The value gradient of y = A x through the headline's panel plan
    (pass A: x per copy entry; pass B: the tile's x placed by LDS word, the
    cotangent from each row's gap word, the gradient stored in position
    order), reached through autograd: equal to the oracle bit for bit on
    two backward passes in a row."""
    from mlx_sparse import synthetic

    ms = gpu
    m = synthetic.random_fixed_row(1 << 22, 16, seed=0)
    n_rows, n_cols = m.shape
    x = synthetic.uniform(n_cols, -1.0, 1.0, seed=1)
    g = synthetic.uniform(n_rows, -1.0, 1.0, seed=3)
    data = torch.from_numpy(m.data).to(DEV).requires_grad_()
    A = ms.csr_array((data, torch.from_numpy(m.indices), torch.from_numpy(m.indptr)),
                     shape=m.shape)
    assert _kind(A.plan().info()) == "panels"
    want = orc.csr_data_vjp(m.indices, m.indptr, x, g, n_rows, n_cols, m.nnz, vtype="float32")
    xt, gt = torch.from_numpy(x).to(DEV), torch.from_numpy(g).to(DEV)
    for k in range(2):
        data.grad = None
        (A @ xt).backward(gt)
        print(f"cfg2 value gradient, backward {k}", flush=True)
        np.testing.assert_array_equal(to_numpy(data.grad), want, err_msg=f"backward {k}")
