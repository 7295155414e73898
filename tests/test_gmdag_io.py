"""`.gmdag` format and loader (rows a10/a11), no GPU: header round trip and bbox_max
derivation (projects/torch-sdf/tests/test_gmdag_roundtrip.py:87-164), and the loader's
accept/reject gates with the reference messages
(projects/environment/tests/unit/test_voxel_dag_integration.py:28-268).
"""

from __future__ import annotations

import struct
from pathlib import Path

import numpy as np
import pytest

from navi_amd import gmdag
from navi_amd import scenes as S

H = struct.Struct("<4sIIffffI")


def _write(path: Path, header: bytes, words) -> Path:
    path.write_bytes(header + np.asarray(words, dtype="<u8").tobytes())
    return path


def test_round_trip(tmp_path):
    scene = S.box_room(resolution=32)
    words = scene.compile()
    p = gmdag.write_gmdag(tmp_path / "room.gmdag", words, 32, scene.bbox_min, scene.voxel_size)
    assert p.stat().st_size == 32 + 8 * words.size
    raw = p.read_bytes()
    magic, version, res, bx, by, bz, voxel, count = H.unpack(raw[:32])
    assert (magic, version, res, count) == (b"GDAG", 1, 32, words.size)
    asset = gmdag.load_gmdag_asset(p)
    assert np.array_equal(asset.nodes, words)
    assert asset.voxel_size == float(scene.voxel_size)
    for k in range(3):
        assert asset.bbox_min[k] == float(scene.bbox_min[k])
        assert asset.bbox_max[k] == pytest.approx(float(scene.bbox_min[k]) + float(scene.voxel_size) * 32, abs=1e-6)
    assert asset.bbox_max == tuple(scene.bbox_max)


def _hdr(magic=b"GDAG", version=1, res=2, bmin=(0.0, 0.0, 0.0), voxel=0.5, count=1):
    return H.pack(magic, version, res, *bmin, voxel, count)


LEAF = (1 << 63) | 0x3C00


@pytest.mark.parametrize("header,words,msg", [
    (_hdr(magic=b"NOPE"), [LEAF], "Unsupported gmdag magic"),
    (_hdr(version=2), [LEAF], "Unsupported gmdag version"),
    (_hdr(res=0), [LEAF], "Invalid gmdag resolution"),
    (_hdr(voxel=0.0), [LEAF], "Invalid gmdag voxel size"),
    (_hdr(count=0), [], "Invalid gmdag node count"),
    (_hdr(count=1), [LEAF, LEAF], "trailing bytes detected"),
    (_hdr(count=2), [LEAF], "expected 2 nodes"),
    (_hdr(bmin=(0.0, float("nan"), 0.0)), [LEAF], "non-finite bbox_min values"),
    (_hdr(count=1), [0], "empty child mask"),
    (_hdr(count=2), [(1 << 55) | 1, 9], r"child reference out of range"),
    (_hdr(count=2), [(1 << 55) | 5, 1], "child pointer table starts beyond payload"),
    (_hdr(count=2), [(0x3 << 55) | 1, 0], "child pointer table exceeds payload bounds"),
    (_hdr(count=3), [(1 << 55) | 1, 0, LEAF], "cycle detected"),
])
def test_loader_rejections(tmp_path, header, words, msg):
    p = _write(tmp_path / "bad.gmdag", header, words)
    with pytest.raises(RuntimeError, match=msg):
        gmdag.load_gmdag_asset(p)


def test_layout_validation_can_be_skipped(tmp_path):
    p = _write(tmp_path / "cyc.gmdag", _hdr(count=3), [(1 << 55) | 1, 0, LEAF])
    asset = gmdag.load_gmdag_asset(p, validate_layout=False)
    assert asset.nodes.size == 3


def test_missing_file(tmp_path):
    with pytest.raises(FileNotFoundError):
        gmdag.load_gmdag_asset(tmp_path / "none.gmdag")


def test_deep_chain_validates_without_recursion_limit():
    n = 5000
    words = [(1 << 55) | (2 * i + 1) if False else 0 for i in range(2 * n + 1)]
    for i in range(n):
        words[2 * i] = (1 << 55) | (2 * i + 1)
        words[2 * i + 1] = 2 * i + 2
    words[2 * n] = LEAF
    gmdag.validate_dag_layout(np.array(words, np.uint64))
