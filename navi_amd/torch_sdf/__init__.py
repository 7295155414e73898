"""MI355X drop-in for the ``torch_sdf`` package (``projects/torch-sdf/torch_sdf/__init__.py``).

``navi_amd.dropin.install()`` registers this package as ``torch_sdf`` and
:mod:`navi_amd.torch_sdf_backend` as ``torch_sdf_backend`` so existing callers
(``SdfDagBackend``, the env CLI, tests) import it unchanged.
"""

from .backend import cast_rays, invalidate, prepare

__all__ = ["cast_rays"]
