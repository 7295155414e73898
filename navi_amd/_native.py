"""ctypes binding of ``libnavi_trace.so`` (the C ABI declared in ``include/navi_trace.h``).

Importing this module loads the HIP library and raises ``ImportError`` when it
has not been built — there is no fallback: the tracer runs on the GPU or not at
all (the reference's own stance, ``projects/torch-sdf/torch_sdf/backend.py:158-169``).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "_lib"
LIB_PATH = Path(os.environ.get("NAVI_TRACE_LIB", LIB_DIR / "libnavi_trace.so"))

NAVI_OK = 0
NAVI_E_ARG = -1
NAVI_E_LAUNCH = -2
NAVI_E_LAYOUT = -3
NAVI_E_NOMEM = -4

if not LIB_PATH.exists():
    raise ImportError(
        f"libnavi_trace.so not found at {LIB_PATH}; build it with "
        "`python -c 'import __graft_entry__ as g; g.build()'` (or `make -C navi_amd/csrc`)."
    )

_lib = ctypes.CDLL(str(LIB_PATH))

_vp = ctypes.c_void_p
_f3 = ctypes.POINTER(ctypes.c_float)

_lib.navi_last_error.restype = ctypes.c_char_p
_lib.navi_last_error.argtypes = []
_lib.navi_version.restype = ctypes.c_char_p
_lib.navi_version.argtypes = []

_lib.navi_cast_rays.restype = ctypes.c_int
_lib.navi_cast_rays.argtypes = [
    _vp, ctypes.c_uint64, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int32, ctypes.c_float,
    _f3, _f3, ctypes.c_int32, ctypes.c_float, _vp, _vp,
]


def lib() -> ctypes.CDLL:
    return _lib


def version() -> str:
    return _lib.navi_version().decode()


def last_error() -> str:
    return _lib.navi_last_error().decode(errors="replace")


def check(code: int) -> None:
    """Raise ``RuntimeError`` (the exception type TORCH_CHECK surfaces) for a failed call."""
    if code != NAVI_OK:
        raise RuntimeError(last_error() or f"navi_trace call failed with code {code}")


def float3(values) -> ctypes.Array:
    return (ctypes.c_float * 3)(*[float(v) for v in values])
