"""navi_amd — MI355X-native batched sphere tracer for navi's ``.gmdag`` SDF DAGs.

Layers (top to bottom):

* :mod:`navi_amd.torch_sdf` / :mod:`navi_amd.torch_sdf_backend` — drop-in mirrors of
  the reference's ``torch_sdf.cast_rays`` API (11 positional arguments, zero-copy,
  caller-owned outputs, current-stream launch); :mod:`navi_amd.dropin` registers them
  under the reference's module names.
* :mod:`navi_amd._native` — ctypes binding of ``libnavi_trace.so`` (C ABI in
  ``include/navi_trace.h``), the hand-written HIP/gfx950 kernels in ``navi_amd/csrc``.

Importing this package does not load the HIP library; the submodules above do.
"""

__version__ = "0.3.0"
