"""Loader of the native extension ``_ext`` (gfx950 HIP kernels behind the C
ABI of ``include/lattice_hip.h``).

The product path has no CPU fallback: importing this module fails loudly when
the extension has not been built (``python mlx-lattice_amd/build.py``).
"""

from __future__ import annotations

import importlib
from pathlib import Path

_PKG = Path(__file__).resolve().parent


def _load():
    try:
        import torch  # noqa: F401  (loads libc10/libtorch for the extension)

        return importlib.import_module('mlx_lattice_amd._ext')
    except ImportError as exc:
        raise ImportError(
            'mlx_lattice_amd native extension is not built: run '
            '`python mlx-lattice_amd/build.py` (needs hipcc for gfx950). '
            f'Looked in {_PKG}. Cause: {exc}'
        ) from exc


ext = _load()

__all__ = ['ext']
