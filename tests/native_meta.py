"""Native mesh metadata files (CARL_ARENA_METADATA) for the tests.

The format is the one tools/arena_metadata.py writes and src/ArenaMesh.cu:69-99
reads: the triangle count, then per triangle of the arena mesh
`mesh order angle0 angle1 angle2 flags v0 v1 v2` with the native vertices in
Bullet units (0.02 uu).  Triangles lying in one of the arena planes (floor,
ceiling, side walls) are written as the exporter writes them: mesh and order
-1, boundary angles, no flags (tools/arena_metadata.py:58-66); the engine
skips them and adds the planes analytically.

RocketSim's own metadata cannot be produced here, so the files are
synthetic: `restating` keeps the arena's own triangles, edge angles and
triangle order (one native mesh); `synthetic` spreads the triangles over
several meshes in shuffled order, with random edge flags and the vertices
moved by a few parts per million, so that every piece of metadata changes
what the ball meets.
"""
from __future__ import annotations

import numpy as np

PLANES = ((2, 0.0), (2, 2048.0), (0, -4096.0), (0, 4096.0))
BOUNDARY = "6.2831853"


def plane_triangles(tv: np.ndarray) -> np.ndarray:
    """Triangles (rows of [n, 3, 3] vertices, uu) lying in an arena plane."""
    out = np.zeros(len(tv), bool)
    for axis, value in PLANES:
        out |= np.all(np.abs(tv[:, :, axis] - value) < 1e-3, axis=1)
    return out


def _fmt(x) -> str:
    return f"{float(x):.9g}"


def metadata_text(mesh, order, angles, flags, native) -> str:
    """The file text for per-triangle mesh, order, angles [n, 3], flags and
    native vertices [n, 3, 3]; triangles of mesh -1 are written as planes."""
    lines = [str(len(mesh))]
    for t in range(len(mesh)):
        v = " ".join(_fmt(x) for x in native[t].reshape(-1))
        if mesh[t] < 0:
            lines.append(f"-1 -1 {BOUNDARY} {BOUNDARY} {BOUNDARY} 0 {v}")
        else:
            a = " ".join(_fmt(x) for x in angles[t])
            lines.append(f"{int(mesh[t])} {int(order[t])} {a} {int(flags[t])} {v}")
    return "\n".join(lines) + "\n"


def native_vertices(tv: np.ndarray) -> np.ndarray:
    return (tv.astype(np.float32) * np.float32(0.02)).astype(np.float32)


def restating(verts, tris, angles):
    """One native mesh holding every non-plane triangle in triangle order,
    the arena's own edge angles and vertices: (mesh, order, angles, flags,
    native vertices)."""
    tv = verts[tris]
    plane = plane_triangles(tv)
    mesh = np.where(plane, -1, 0)
    order = np.arange(len(tris))
    return mesh, order, angles, np.zeros(len(tris), np.int64), native_vertices(tv)


def synthetic(verts, tris, angles, rng, n_meshes=5, jitter=4e-6):
    """Non-plane triangles spread over n_meshes meshes (n_meshes = 0: one
    mesh per triangle), each mesh in a shuffled order, random flags, and
    vertices moved by up to `jitter` of their size."""
    tv = verts[tris]
    n = len(tris)
    plane = plane_triangles(tv)
    mesh = np.arange(n) if n_meshes == 0 else rng.integers(0, n_meshes, n)
    order = np.zeros(n, np.int64)
    for m in np.unique(mesh):
        members = np.nonzero(mesh == m)[0]
        order[members] = rng.permutation(len(members))
    mesh = np.where(plane, -1, mesh)
    flags = rng.integers(0, 64, n)
    native = native_vertices(tv) * (1.0 + rng.uniform(-jitter, jitter, tv.shape)).astype(np.float32)
    return mesh, order, angles, flags, native.astype(np.float32)


def write(path, parts) -> str:
    """Write (mesh, order, angles, flags, native) to path; returns the path."""
    with open(path, "w") as f:
        f.write(metadata_text(*parts))
    return str(path)
