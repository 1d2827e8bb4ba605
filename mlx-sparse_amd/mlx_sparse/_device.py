"""Execution-device selection (reference: mlx_sparse/_device.py:15-152).

``use_cpu()`` / ``use_gpu()`` / ``use_device(name)`` set the device that
mlx_sparse operations run on and that new CSR buffers are placed on, and
return a ``torch.device``.  ``use_gpu`` selects a HIP device (torch's
``"cuda"`` device type on ROCm) and probes it, as the reference probes its
Metal device.  Operands living elsewhere are copied to the selected device
when an operation runs (MLX's arrays are in unified memory; torch's are not).
"""

from __future__ import annotations

import torch

_DEFAULT = torch.device("cpu")
_CHOSEN = False


def default_torch_device() -> torch.device:
    """The device operations run on.  Until ``use_*`` is called: the GPU when
    one is available, else the CPU (the reference's MLX default)."""
    global _DEFAULT, _CHOSEN
    if not _CHOSEN:
        _CHOSEN = True
        try:
            if torch.cuda.is_available():
                _DEFAULT = torch.device("cuda", torch.cuda.current_device())
        except Exception:  # pragma: no cover - broken driver: stay on CPU
            _DEFAULT = torch.device("cpu")
    return _DEFAULT


def _set(device: torch.device) -> torch.device:
    global _DEFAULT, _CHOSEN
    _DEFAULT = device
    _CHOSEN = True
    return device


def use_cpu(index: int = 0, *, require_available: bool = True) -> torch.device:
    """Run subsequent mlx_sparse operations on the host CPU."""
    device = torch.device("cpu")
    if require_available:
        try:
            torch.zeros(1).add_(0)
        except Exception as exc:
            raise RuntimeError(
                f"CPU device {index} is not available to this Python process."
            ) from exc
    return _set(device)


def use_gpu(index: int = 0, *, require_available: bool = True) -> torch.device:
    """Run subsequent mlx_sparse operations on HIP device ``index``."""
    device = torch.device("cuda", index)
    if require_available:
        try:
            available = torch.cuda.is_available() and index < torch.cuda.device_count()
            if available:
                torch.zeros(1, device=device).add_(0)
                torch.cuda.synchronize(device)
        except Exception as exc:
            raise RuntimeError(
                f"GPU device {index} is not available to this Python process. "
                "Verify that PyTorch-ROCm can create a tensor on the GPU."
            ) from exc
        if not available:
            raise RuntimeError(
                f"GPU device {index} is not available. PyTorch-ROCm must be able to "
                "create tensors on the GPU before mlx_sparse GPU kernels can run."
            )
        torch.cuda.set_device(index)
    return _set(device)


def use_device(name: str, index: int = 0) -> torch.device:
    """Select ``"cpu"`` or ``"gpu"`` by name (case-insensitive)."""
    normalized = name.lower()
    if normalized == "cpu":
        return use_cpu(index)
    if normalized == "gpu":
        return use_gpu(index)
    raise ValueError(f"device must be 'cpu' or 'gpu', got {name!r}.")
