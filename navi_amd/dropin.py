"""Make ``import torch_sdf`` / ``import torch_sdf_backend`` resolve to this package.

Callers of the reference (``projects/environment/.../sdfdag_backend.py`` imports
``torch_sdf``; ``projects/torch-sdf/torch_sdf/backend.py:7-13`` imports
``torch_sdf_backend``) keep their import lines; one call at start-up swaps the
implementation::

    import navi_amd.dropin
    navi_amd.dropin.install()
    import torch_sdf            # -> navi_amd.torch_sdf
"""

from __future__ import annotations

import importlib
import sys


def install(*, force: bool = False) -> None:
    """Register the MI355X modules under the reference's module names.

    Raises ``ImportError`` if the HIP library is not built (no silent fallback).
    """
    backend = importlib.import_module("navi_amd.torch_sdf_backend")
    package = importlib.import_module("navi_amd.torch_sdf")
    for name, mod in (("torch_sdf_backend", backend), ("torch_sdf", package),
                      ("torch_sdf.backend", importlib.import_module("navi_amd.torch_sdf.backend"))):
        if force or name not in sys.modules:
            sys.modules[name] = mod
