"""``.gmdag`` v1 asset I/O: header + u64 node words, host side.

Format (``docs/GMDAG.md:112-228``; ``projects/voxel-dag/src/compiler.hpp:19-31``):
a packed little-endian 32-byte header ``<4sIIffffI`` — magic ``b"GDAG"``, version 1,
resolution, bbox_min xyz (f32), voxel size (f32), node count — followed by exactly
``node_count`` u64 words and nothing else. ``bbox_max = bbox_min + voxel * resolution``
is derived in double precision by the loader.

:func:`load_gmdag_asset` applies the gates of the reference loader
(``projects/environment/src/navi_environment/integration/voxel_dag.py:193-259``) with
the same messages and, optionally, the DAG layout validation of ``voxel_dag.py:29-78``
(written iteratively here, so deep or long chains cannot exhaust Python's stack).
:func:`upload` puts the words on the GPU as the int64 tensor the tracer takes
(``sdfdag_backend.py:1897-1900``).
"""

from __future__ import annotations

import math
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HEADER = struct.Struct("<4sIIffffI")
MAGIC = b"GDAG"
VERSION = 1

__all__ = ["GmDagAsset", "HEADER", "load_gmdag_asset", "validate_dag_layout", "write_gmdag", "upload"]


@dataclass(frozen=True)
class GmDagAsset:
    path: Path
    version: int
    resolution: int
    bbox_min: tuple[float, float, float]
    bbox_max: tuple[float, float, float]
    voxel_size: float
    nodes: np.ndarray  # uint64 [node_count]


def write_gmdag(path: str | Path, words: np.ndarray, resolution: int, bbox_min, voxel_size: float) -> Path:
    """Write header + words (``compiler.cpp:680-697``)."""
    path = Path(path)
    w = np.ascontiguousarray(np.asarray(words).view(np.uint64).reshape(-1))
    bmin = [float(np.float32(v)) for v in bbox_min]
    with path.open("wb") as fh:
        fh.write(HEADER.pack(MAGIC, VERSION, int(resolution), bmin[0], bmin[1], bmin[2],
                             float(np.float32(voxel_size)), int(w.size)))
        fh.write(w.astype("<u8", copy=False).tobytes())
    return path


def validate_dag_layout(nodes: np.ndarray) -> None:
    """Reachability / range / cycle check from the root (``voxel_dag.py:29-78``).

    Raises ``RuntimeError`` with the reference's messages: internal node with an empty
    child mask, child table starting beyond or running past the payload, child
    reference out of range, or a cycle.
    """
    words = np.asarray(nodes).view(np.uint64).reshape(-1)
    n = int(words.size)
    WHITE, GREY, BLACK = 0, 1, 2
    state = np.zeros(n, np.uint8)
    if n == 0:
        raise RuntimeError("Invalid gmdag DAG layout: node index out of range: 0")
    # iterative DFS: stack of (node, next child offset)
    stack: list[list[int]] = []

    def enter(idx: int) -> None:
        if idx < 0 or idx >= n:
            raise RuntimeError(f"Invalid gmdag DAG layout: node index out of range: {idx}")
        if state[idx] == GREY:
            raise RuntimeError(f"Invalid gmdag DAG layout: cycle detected at node index {idx}")
        if state[idx] == BLACK:
            return
        word = int(words[idx])
        if (word >> 63) == 0:
            mask = (word >> 55) & 0xFF
            if mask == 0:
                raise RuntimeError(f"Invalid gmdag DAG layout: internal node {idx} has empty child mask")
            base = word & 0xFFFFFFFF
            count = mask.bit_count()
            if base >= n:
                raise RuntimeError(
                    f"Invalid gmdag DAG layout: child pointer table starts beyond payload at index {base}")
            if base + count > n:
                raise RuntimeError(
                    f"Invalid gmdag DAG layout: child pointer table exceeds payload bounds for node {idx}")
            state[idx] = GREY
            stack.append([idx, base, count, 0])
        else:
            state[idx] = BLACK

    enter(0)
    while stack:
        frame = stack[-1]
        idx, base, count, k = frame
        if k == count:
            state[idx] = BLACK
            stack.pop()
            continue
        frame[3] = k + 1
        child = int(words[base + k]) & 0xFFFFFFFFFFFFFFFF
        if child >= n:
            raise RuntimeError(
                f"Invalid gmdag DAG layout: child reference out of range ({child}) from node {idx}")
        enter(child)


def load_gmdag_asset(path: str | Path, *, validate_layout: bool = True) -> GmDagAsset:
    """Load and gate a ``.gmdag`` file (``voxel_dag.py:193-259``)."""
    path = Path(path).expanduser().resolve()
    if not path.exists():
        raise FileNotFoundError(f"gmdag asset does not exist: {path}")
    with path.open("rb") as fh:
        header = fh.read(HEADER.size)
        if len(header) != HEADER.size:
            raise RuntimeError(f"Invalid gmdag header in {path}")
        magic, version, resolution, bx, by, bz, voxel, count = HEADER.unpack(header)
        if magic != MAGIC:
            raise RuntimeError(f"Unsupported gmdag magic in {path}: {magic!r}")
        if version != VERSION:
            raise RuntimeError(f"Unsupported gmdag version in {path}: {version}")
        if resolution <= 0:
            raise RuntimeError(f"Invalid gmdag resolution in {path}: {resolution}")
        if not math.isfinite(voxel) or voxel <= 0.0:
            raise RuntimeError(f"Invalid gmdag voxel size in {path}: {voxel}")
        if count <= 0:
            raise RuntimeError(f"Invalid gmdag node count in {path}: {count}")
        if not all(math.isfinite(v) for v in (bx, by, bz)):
            raise RuntimeError(f"Invalid gmdag bounds in {path}: non-finite bbox_min values detected")
        nodes = np.fromfile(fh, dtype="<u8", count=count)
        if nodes.shape[0] != count:
            raise RuntimeError(
                f"Invalid gmdag node payload in {path}: expected {count} nodes, found {nodes.shape[0]}")
        if fh.read(1):
            raise RuntimeError(f"Invalid gmdag payload in {path}: trailing bytes detected")
    nodes = np.ascontiguousarray(nodes.astype(np.uint64, copy=False))
    if validate_layout:
        validate_dag_layout(nodes)
    bmin = (float(bx), float(by), float(bz))
    ext = float(voxel) * int(resolution)
    return GmDagAsset(path=path, version=int(version), resolution=int(resolution), bbox_min=bmin,
                      bbox_max=(bmin[0] + ext, bmin[1] + ext, bmin[2] + ext), voxel_size=float(voxel),
                      nodes=nodes)


def upload(asset_or_words, device="cuda"):
    """Words as a contiguous int64 device tensor (the ``dag_tensor`` of ``cast_rays``)."""
    import torch

    words = asset_or_words.nodes if isinstance(asset_or_words, GmDagAsset) else asset_or_words
    w = np.ascontiguousarray(np.asarray(words).view(np.uint64).reshape(-1))
    return torch.from_numpy(w.view(np.int64)).to(device)
