"""Runtime options for the path (reference: mlx_sparse/runtime.py:203-362,
mlx_sparse/_config.py:194-300,651-730).

Only the CPU worker budget reaches this path.  As in the reference, the
option is mirrored into ``MLX_SPARSE_CPU_THREADS`` in ``os.environ``, which
the native CPU path reads on every call.  ``GPU_PLAN`` (new) toggles the
cached row-block plan of the GPU SpMV; without it a plan-free kernel runs.
``GPU_SLICE`` (new) selects the reordered copy a plan may hold for scattered
gathers: "auto" (default: panels when the columns are scattered over an x of
more than 8 MB and the matrix qualifies, else XCD slices), "off", "on" (XCD
column slices) or "panels" (LDS column panels); it applies to plans built
while it is set.  ``GPU_ADJOINT`` (new) routes the A^H products of the
gradients on the GPU: "atomic" (scatter over A's rows), "transpose" (a
cached CSR of A^H, multiplied by the forward kernels) or "auto" (default:
scatter on a matrix's first adjoint product, cached transpose after).
"""

from __future__ import annotations

import contextlib
import enum
import os
from collections.abc import Iterator, Mapping
from typing import Any

_ENV = {"n_threads": "MLX_SPARSE_CPU_THREADS", "gpu_plan": "MLX_SPARSE_GPU_PLAN",
        "gpu_slice": "MLX_SPARSE_GPU_SLICE", "gpu_adjoint": "MLX_SPARSE_GPU_ADJOINT"}
_SLICE = {"auto": 0, "off": 1, "on": 2, "panels": 3}
_ADJOINT = ("auto", "atomic", "transpose")
_MISSING = object()


class RuntimeOption(str, enum.Enum):
    N_THREADS = "n_threads"
    GPU_PLAN = "gpu_plan"
    GPU_SLICE = "gpu_slice"  # "auto" | "off" | "on" | "panels": reordered copy of plans
    GPU_ADJOINT = "gpu_adjoint"  # "auto" | "atomic" | "transpose": route of A^H products


def _parse_threads(value: Any) -> int | str:
    if value is None or value == "auto":
        return "auto"
    if isinstance(value, bool):
        raise TypeError("n_threads must be a positive int or 'auto'.")
    count = int(value)
    if count <= 0:
        raise ValueError(f"n_threads must be positive, got {value!r}.")
    return count


def _parse_bool(value: Any) -> bool:
    if isinstance(value, str):
        v = value.strip().lower()
        if v in {"1", "true", "t", "yes", "y", "on"}:
            return True
        if v in {"0", "false", "f", "no", "n", "off"}:
            return False
        raise ValueError(f"expected a boolean, got {value!r}.")
    return bool(value)


def get(option: RuntimeOption | str) -> Any:
    key = _normalize_option(option)
    raw = os.environ.get(_ENV[key])
    if key == "n_threads":
        if raw is None or raw == "":
            alias = os.environ.get("MLX_SPARSE_N_THREADS")
            raw = alias if alias else None
        try:
            return _parse_threads(raw)
        except (TypeError, ValueError):
            return "auto"
    if key == "gpu_slice":
        return _SLICE.get((raw or "auto").strip().lower(), 0)
    if key == "gpu_adjoint":
        v = (raw or "auto").strip().lower()
        return v if v in _ADJOINT else "auto"
    return True if raw is None else _parse_bool(raw)


def _normalize_option(option) -> str:
    if isinstance(option, RuntimeOption):
        return option.value
    key = str(option).lower()
    if key not in _ENV:
        raise KeyError(f"unknown runtime option {option!r}.")
    return key


def _encode(key: str, value: Any) -> str | None:
    if key == "gpu_adjoint":
        v = str(value).strip().lower()
        if v not in _ADJOINT:
            raise ValueError(f"gpu_adjoint must be one of {list(_ADJOINT)}, got {value!r}.")
        return v
    if key == "gpu_slice":
        v = str(value).strip().lower()
        if v not in _SLICE:
            raise ValueError(f"gpu_slice must be one of {sorted(_SLICE)}, got {value!r}.")
        return v
    if key == "n_threads":
        parsed = _parse_threads(value)
        return None if parsed == "auto" else str(parsed)
    return "1" if _parse_bool(value) else "0"


def _hardware_concurrency() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):  # pragma: no cover
        return os.cpu_count() or 1


def resolve_n_threads() -> tuple[int, str]:
    """Effective CPU worker count and where it came from (reference
    runtime.py:203-215, cpu_parallel.cpp:97-123)."""
    configured = get(RuntimeOption.N_THREADS)
    if isinstance(configured, int):
        return configured, "configured"
    for name in ("OMP_NUM_THREADS", "SLURM_CPUS_PER_TASK", "PBS_NP", "LSB_DJOB_NUMPROC", "NSLOTS"):
        raw = os.environ.get(name, "")
        head = raw.split(",")[0]
        if head.isdigit() and int(head) > 0:
            return int(head), name
    return _hardware_concurrency(), "affinity"


@contextlib.contextmanager
def context(arg1: Any = None, arg2: Any = _MISSING, **kwargs: Any) -> Iterator[None]:
    """Temporarily patch runtime options: ``context(n_threads=4)``,
    ``context(RuntimeOption.N_THREADS, 4)`` or ``context({...: 4})``."""
    if arg1 is None:
        if arg2 is not _MISSING:
            raise TypeError("context(None, value) is not a valid call form.")
        updates = {_normalize_option(k): v for k, v in kwargs.items()}
    elif isinstance(arg1, Mapping):
        if arg2 is not _MISSING or kwargs:
            raise TypeError("Mapping context form does not accept other arguments.")
        updates = {_normalize_option(k): v for k, v in arg1.items()}
    else:
        if arg2 is _MISSING:
            raise TypeError("context(option, value) requires a value.")
        if kwargs:
            raise TypeError("Cannot combine two-argument context with keywords.")
        updates = {_normalize_option(arg1): arg2}
    encoded = {key: _encode(key, value) for key, value in updates.items()}
    saved = {key: os.environ.get(_ENV[key]) for key in encoded}
    try:
        for key, value in encoded.items():
            if value is None:
                os.environ.pop(_ENV[key], None)
            else:
                os.environ[_ENV[key]] = value
        yield
    finally:
        for key, value in saved.items():
            if value is None:
                os.environ.pop(_ENV[key], None)
            else:
                os.environ[_ENV[key]] = value


patch = context


def info() -> dict[str, Any]:
    """Structured runtime facts for reports (reference runtime.py:287-321)."""
    import torch

    from mlx_sparse._device import default_torch_device
    from mlx_sparse._ext_loader import extension_available

    threads, source = resolve_n_threads()
    gpu_name = None
    if torch.cuda.is_available():
        gpu_name = torch.cuda.get_device_name(0)
    return {
        "n_threads": threads,
        "n_threads_source": source,
        "gpu_plan": get(RuntimeOption.GPU_PLAN),
        "gpu_slice": get(RuntimeOption.GPU_SLICE),
        "gpu_adjoint": get(RuntimeOption.GPU_ADJOINT),
        "device": str(default_torch_device()),
        "extension": extension_available(),
        "gpu": gpu_name,
        "torch": torch.__version__,
        "hip": torch.version.hip,
    }
