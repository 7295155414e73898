"""The drop-in boundary without a GPU: the validation contract of
projects/torch-sdf/torch_sdf/backend.py:28-197 and bindings.cpp:43-110 (messages pinned
by projects/torch-sdf/tests/test_sphere_tracing.py:294-680), the C ABI library exports,
and its host-side argument checks. No GPU kernel is launched here.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from navi_amd import _native, torch_sdf_backend
from navi_amd.torch_sdf import backend as backend_module

ROOT = Path(__file__).resolve().parents[1]


class _FakeTensor:
    def __init__(self, *, shape, dtype, is_cuda=True, contiguous=True):
        self.shape = shape
        self.dtype = dtype
        self.is_cuda = is_cuda
        self._contiguous = contiguous

    def dim(self):
        return len(self.shape)

    def size(self, idx):
        return self.shape[idx]

    def is_contiguous(self):
        return self._contiguous


def _inputs(**over):
    v = {
        "dag": _FakeTensor(shape=(8,), dtype=torch.int64),
        "origins": _FakeTensor(shape=(2, 3, 3), dtype=torch.float32),
        "dirs": _FakeTensor(shape=(2, 3, 3), dtype=torch.float32),
        "out_distances": _FakeTensor(shape=(2, 3), dtype=torch.float32),
        "out_semantics": _FakeTensor(shape=(2, 3), dtype=torch.int32),
    }
    v.update(over)
    return v["dag"], v["origins"], v["dirs"], v["out_distances"], v["out_semantics"]


@pytest.fixture
def fake_gpu(monkeypatch):
    monkeypatch.setattr(backend_module, "HAS_CUDA_BACKEND", True)
    monkeypatch.setattr(backend_module, "torch_sdf_backend", object())
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)


def test_native_call_has_eleven_arguments(monkeypatch):
    captured = {}

    class _Backend:
        def cast_rays(self, *args, **kw):
            captured["argc"] = len(args)
            captured["kw"] = kw
            captured["max_distance"] = args[6]

    monkeypatch.setattr(backend_module, "HAS_CUDA_BACKEND", True)
    monkeypatch.setattr(backend_module, "torch_sdf_backend", _Backend())
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    backend_module.cast_rays(*_inputs(), 64, 17.5, [0, 0, 0], [1, 1, 1], 128,
                             skip_direction_validation=True)
    assert captured["argc"] == 11 and captured["kw"] == {} and captured["max_distance"] == 17.5


@pytest.mark.parametrize("over,args,msg", [
    ({"dirs": _FakeTensor(shape=(2, 3, 3), dtype=torch.float32, contiguous=False)}, None, "dirs must be contiguous"),
    ({"dag": _FakeTensor(shape=(8,), dtype=torch.int64, is_cuda=False)}, None, "dag_tensor must be on CUDA"),
    ({"out_semantics": _FakeTensor(shape=(2, 3), dtype=torch.int32, is_cuda=False)}, None,
     "out_semantics must be a CUDA tensor"),
    ({"dirs": _FakeTensor(shape=(2, 3, 3), dtype=torch.float64)}, None, "dirs must have dtype"),
    ({"out_semantics": _FakeTensor(shape=(2, 4), dtype=torch.int32)}, None, "out_semantics must have shape"),
    ({}, (0, 30.0, [0, 0, 0], [1, 1, 1], 128), "max_steps must be a positive integer"),
    ({}, (64, 0.0, [0, 0, 0], [1, 1, 1], 128), "max_distance must be a finite positive float"),
    ({}, (64, 30.0, [1, 0, 0], [1, 1, 1], 128), r"bbox_min\[0\] must be strictly less than bbox_max\[0\]"),
    ({}, (64, 30.0, [0.0, float("nan"), 0.0], [1.0, 1.0, 1.0], 128), "must contain only finite floats"),
    ({}, (64, float("inf"), [0, 0, 0], [1, 1, 1], 128), "max_distance must be a finite positive float"),
    ({}, (64, 30.0, [0, 0, 0], [1, 1, 1], 0), "resolution must be a positive integer"),
])
def test_python_layer_rejections(fake_gpu, over, args, msg):
    args = args or (64, 30.0, [0, 0, 0], [1, 1, 1], 128)
    with pytest.raises(RuntimeError, match=msg):
        backend_module.cast_rays(*_inputs(**over), *args, skip_direction_validation=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_reduced_precision_distances_pass_the_python_layer(monkeypatch, dtype):
    """out_distances may be bfloat16 or float16 (the reference roadmap's T2 item,
    docs/FUTURE_HARDWARE_ROADMAP.md:157-176); the native call gets the tensor as is."""
    captured = {}

    class _Backend:
        def cast_rays(self, *args, **kw):
            captured["dtype"] = args[3].dtype

    monkeypatch.setattr(backend_module, "HAS_CUDA_BACKEND", True)
    monkeypatch.setattr(backend_module, "torch_sdf_backend", _Backend())
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    backend_module.cast_rays(*_inputs(out_distances=_FakeTensor(shape=(2, 3), dtype=dtype)), 64, 17.5,
                             [0, 0, 0], [1, 1, 1], 128, skip_direction_validation=True)
    assert captured["dtype"] == dtype


def test_other_distance_dtypes_are_rejected(fake_gpu):
    for dtype in (torch.float64, torch.int32):
        with pytest.raises(RuntimeError, match="out_distances must have dtype torch.float32"):
            backend_module.cast_rays(*_inputs(out_distances=_FakeTensor(shape=(2, 3), dtype=dtype)), 64, 30.0,
                                     [0, 0, 0], [1, 1, 1], 128, skip_direction_validation=True)
    # the native layer's message keeps the reference's prefix (bindings.cpp:71)
    with pytest.raises(RuntimeError, match="out_distances must be float32"):
        torch_sdf_backend.validate_cast_inputs(
            *[_FakeTensor(shape=t.shape, dtype=t.dtype, is_cuda=True) for t in _inputs()[:3]],
            _FakeTensor(shape=(2, 3), dtype=torch.float64), _FakeTensor(shape=(2, 3), dtype=torch.int32),
            64, 30.0, [0, 0, 0], [1, 1, 1], 128)


def test_direction_norm_checks():
    with pytest.raises(RuntimeError, match="normalized within tolerance"):
        backend_module._validate_direction_norms(torch.tensor([[[1.2, 0.0, 0.0]]]))
    with pytest.raises(RuntimeError, match="finite direction vectors"):
        backend_module._validate_direction_norms(torch.tensor([[[float("nan"), 0.0, 1.0]]]))
    backend_module._validate_direction_norms(torch.tensor([[[1.0, 5e-5, 0.0]]]))
    with pytest.raises(RuntimeError, match="normalized within tolerance"):
        torch_sdf_backend._validate_direction_norms(torch.tensor([[[0.5, 0.0, 0.0]]]))


def test_no_backend_means_no_fallback(monkeypatch):
    monkeypatch.setattr(backend_module, "HAS_CUDA_BACKEND", False)
    with pytest.raises(RuntimeError, match="torch_sdf_backend is not available"):
        backend_module.cast_rays(*_inputs(), 64, 30.0, [0, 0, 0], [1, 1, 1], 128)
    monkeypatch.setattr(backend_module, "HAS_CUDA_BACKEND", True)
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    with pytest.raises(RuntimeError, match="does not support CPU fallback"):
        backend_module.cast_rays(*_inputs(), 64, 30.0, [0, 0, 0], [1, 1, 1], 128)


def test_native_layer_checks_cpu_tensors_before_launch():
    """bindings.cpp:57-86 order: device first, then contiguity, dtype, shapes, params."""
    dag = torch.zeros(4, dtype=torch.int64)
    o = torch.zeros((1, 2, 3))
    with pytest.raises(RuntimeError, match="dag_tensor must be a CUDA tensor"):
        torch_sdf_backend.cast_rays(dag, o, o, torch.zeros(1, 2), torch.zeros(1, 2, dtype=torch.int32),
                                    4, 1.0, [0, 0, 0], [1, 1, 1], 1)


@pytest.mark.parametrize("max_steps,resolution,msg", [
    (2 ** 31, 128, "max_steps must be a positive integer"),
    (64, 2 ** 31, "resolution must be a positive integer"),
])
def test_native_layer_rejects_values_beyond_int32(max_steps, resolution, msg):
    """The native call takes int step counts and resolutions (bindings.cpp:49,53):
    larger values are rejected, not truncated."""
    with pytest.raises(RuntimeError, match=msg):
        torch_sdf_backend.validate_cast_inputs(*_inputs(), max_steps, 30.0, [0, 0, 0], [1, 1, 1], resolution)


def _declared_functions():
    names = []
    for h in sorted((ROOT / "include").glob("*.h")):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[\w]+\s*\**\s*(navi_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_every_declared_symbol_is_exported():
    declared = _declared_functions()
    assert "navi_cast_rays" in declared and "navi_trace_relaid" in declared
    libs = [ctypes.CDLL(str(ROOT / "navi_amd" / "_lib" / n)) for n in ("libnavi_trace.so", "libnavi_scene.so")]
    for name in declared:
        assert any(hasattr(lib, name) for lib in libs), f"{name} declared in include/ but not exported"
    assert re.fullmatch(r"\d+\.\d+\.\d+", _native.version())


def test_wide_min_rays_knob_without_a_gpu():
    """navi_set_wide_min_rays is host-only: it swaps the launch-shape threshold
    (default 2^19 rays) and returns the previous one."""
    prev = _native.set_wide_min_rays(12345)
    try:
        assert prev == 1 << 19
        assert _native.set_wide_min_rays(0) == 12345
        assert _native.set_wide_min_rays((1 << 64) - 1) == 0
    finally:
        _native.set_wide_min_rays(prev)
    with pytest.raises(ValueError):
        _native.set_wide_min_rays(-1)


def test_c_abi_rejects_bad_arguments_without_a_gpu():
    lib = _native.lib()
    f3 = _native.float3
    code = lib.navi_cast_rays(1, 1, None, None, None, None, 4, 0, 1.0, f3([0, 0, 0]), f3([1, 1, 1]), 1, 0.01,
                              None, None, None)
    assert code == _native.NAVI_E_ARG and "max_steps" in _native.last_error()
    code = lib.navi_cast_rays(1, 1, None, None, None, None, 4, 4, 1.0, f3([1, 0, 0]), f3([1, 1, 1]), 1, 0.01,
                              None, None, None)
    assert code == _native.NAVI_E_ARG and "strictly less" in _native.last_error()
    code = lib.navi_cast_rays(1, 1, None, None, None, None, 0, 4, 1.0, f3([0, 0, 0]), f3([1, 1, 1]), 1, 0.01,
                              None, None, None)
    assert code == _native.NAVI_OK  # empty batch: no launch
    code = lib.navi_trace_relaid(1, 1, 1, 1, 1, 6, None, None, 1 << 20, 1 << 20, 0, 1, 1, 1, 1, 4, 1.0, 0.01,
                                  None, None)
    assert code == _native.NAVI_E_ARG and "2^30" in _native.last_error()
    # one ray past the limit the drop-in's kernel choice uses, and a product that overflows int64
    over = torch_sdf_backend.RELAID_MAX_RAYS + 1
    for envs, rays in ((over, 1), (1, over), (1 << 62, 4)):
        code = lib.navi_trace_relaid(1, 1, 1, 1, 1, 6, None, None, envs, rays, 0, 1, 1, 1, 1, 4, 1.0, 0.01,
                                      None, None)
        assert code == _native.NAVI_E_ARG and "2^30" in _native.last_error()
    # 2^27 records would wrap the 32-bit byte size of the pool's buffer resource to 0
    code = lib.navi_trace_relaid(1, 1 << 27, 1, 1, 1, 6, None, None, 4, 4, 0, 1, 1, 1, 1, 4, 1.0, 0.01, None,
                                  None)
    assert code == _native.NAVI_E_ARG and "2^27" in _native.last_error()
    code = lib.navi_trace_relaid(1, 1, 1, 1, None, 6, None, None, 4, 4, 0, 1, 1, 1, 1, 4, 1.0, 0.01, None, None)
    assert code == _native.NAVI_E_ARG and "cell_tables" in _native.last_error()
    for depth in (3, 8):
        code = lib.navi_trace_relaid(1, 1, 1, 1, 1, depth, None, None, 4, 4, 0, 1, 1, 1, 1, 4, 1.0, 0.01, None,
                                      None)
        assert code == _native.NAVI_E_ARG and "table_depth" in _native.last_error()
    q = _native.PointQueries(records=1, n_records=1, scenes=1, n_scenes=1, cell_tables=1, table_depth=3,
                             points=1, n_points=1, out_distances=1, out_semantics=1)
    assert lib.navi_point_query(ctypes.byref(q), None) == _native.NAVI_E_ARG
    assert "table_depth" in _native.last_error()


@pytest.mark.parametrize("header", sorted(p.name for p in (ROOT / "include").glob("*.h")))
@pytest.mark.parametrize("lang", ["c", "c++"])
def test_headers_compile_on_their_own(tmp_path, header, lang):
    """The C ABI headers are self-contained plain C99 (and valid C++17), so a binding
    written in C, cgo or C++ can include them alone."""
    import shutil
    import subprocess

    compiler = {"c": "gcc", "c++": "g++"}[lang]
    if shutil.which(compiler) is None:
        pytest.skip(f"needs {compiler}")
    src = tmp_path / ("h.c" if lang == "c" else "h.cpp")
    src.write_text(f'#include "{header}"\nint main(void) {{ return 0; }}\n')
    std = "-std=c99" if lang == "c" else "-std=c++17"
    out = subprocess.run([compiler, std, "-Wall", "-Wextra", "-pedantic", "-Werror", "-fsyntax-only",
                          "-I", str(ROOT / "include"), str(src)], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr


def test_ctypes_structs_match_the_header(tmp_path):
    """Every struct the Python layer passes through the C ABI has the header's size and
    field offsets (gcc on include/navi_trace.h against ctypes), so a field added on one
    side only fails here rather than on the device."""
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("gcc not installed")
    structs = {"navi_relaid_launch": _native.RelaidLaunch, "navi_point_queries": _native.PointQueries,
               "navi_observation": _native.Observation, "navi_launch_info": _native.LaunchInfo}
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "navi_trace.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'  printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ['  printf("navi_relaid_scene size %zu\\n", sizeof(navi_relaid_scene));',
              '  printf("navi_scene_desc size %zu\\n", sizeof(navi_scene_desc));', "  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    got = {tuple(line.split()[:2]): int(line.split()[2]) for line in out if line}
    for cname, cls in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert got[(cname, field)] == getattr(cls, field).offset, (cname, field)
    assert got[("navi_relaid_scene", "size")] == 48 and got[("navi_scene_desc", "size")] == 40


def test_relaid_ex_rejects_bad_arguments_without_a_gpu():
    lib = _native.lib()
    assert lib.navi_trace_relaid_ex(None, None) == _native.NAVI_E_ARG
    assert "launch" in _native.last_error()
    base = dict(records=1, n_records=1, scenes=1, n_scenes=1, cell_tables=1, table_depth=6, n_envs=0,
                rays_per_env=4, max_steps=4, max_distance=1.0, hit_epsilon=0.01)
    # an empty batch is accepted, but not with an unknown distance type
    assert lib.navi_trace_relaid_ex(ctypes.byref(_native.RelaidLaunch(**base)), None) == _native.NAVI_OK
    for bad in (3, -1):
        L = _native.RelaidLaunch(**base, distance_dtype=bad)
        assert lib.navi_trace_relaid_ex(ctypes.byref(L), None) == _native.NAVI_E_ARG
        assert "distance_dtype" in _native.last_error()
    L = _native.RelaidLaunch(**dict(base, n_envs=1, out_distances=1, out_semantics=1))
    assert lib.navi_trace_relaid_ex(ctypes.byref(L), None) == _native.NAVI_E_ARG
    assert "origins and dirs" in _native.last_error()
    L = _native.RelaidLaunch(**dict(base, n_envs=1, out_distances=1, out_semantics=1, local_dirs=1))
    assert lib.navi_trace_relaid_ex(ctypes.byref(L), None) == _native.NAVI_E_ARG
    assert "env_pos" in _native.last_error()
