"""Loads the native module (reference: mlx_sparse/_ext_loader.py:15-36).

The reference falls back to NumPy when ``_ext`` is missing; this build has no
fallback, so callers get a RuntimeError naming the missing build instead.
"""

from __future__ import annotations

import torch  # noqa: F401 - loads torch's HIP runtime before the library binds to it

_EXT = None
_ERROR: Exception | None = None


def load_extension():
    global _EXT, _ERROR
    if _EXT is None and _ERROR is None:
        try:
            from mlx_sparse import _ext

            _EXT = _ext
        except ImportError as exc:  # not built
            _ERROR = exc
    return _EXT


def extension_available() -> bool:
    return load_extension() is not None


def extension():
    ext = load_extension()
    if ext is None:
        raise RuntimeError(
            "mlx_sparse native extension is not built (run `python mlx-sparse_amd/build.py`); "
            f"import error: {_ERROR}"
        )
    return ext
