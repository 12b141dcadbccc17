"""The arena build's error path, without a GPU: a missing or malformed mesh
(bad OBJ lines, an index out of range, a degenerate triangle, a non-manifold
edge, inconsistent winding, two triangles folded onto each other) fails
environment creation with CARL_ERR_ARENA and the reference's message
(include/Arena/ObjLoader.cuh:17-126, TriMesh.cuh:26-44, EdgeInfo.cuh:60-93),
before any device work; the Python binding raises RuntimeError, as the
reference's std::runtime_error does, and the CPU oracle's loader reports the
same message.  A well-formed small mesh builds."""
import ctypes as C

import pytest

import carl
from abi import enum_values
from carl_amd import build
from oracle_py import OracleEnv

# a unit square of two triangles, consistently wound (counter-clockwise from +z);
# OBJ vertex lines store (y, x, z)
SQUARE_V = ["v 0 0 0", "v 0 1 0", "v 1 1 0", "v 1 0 0"]
GOOD = SQUARE_V + ["f 1 2 3", "f 1 3 4"]

BAD = {
    "invalid OBJ vertex": SQUARE_V[:3] + ["v 1 0"] + ["f 1 2 3"],
    "invalid OBJ triangle": SQUARE_V + ["f 1 2"],
    "OBJ triangle index is out of range": SQUARE_V + ["f 1 2 9"],
    "degenerate triangle in arena mesh": SQUARE_V + ["v 2 0 0", "f 1 4 5"],
    # a third triangle on the square's diagonal 1-3
    "non-manifold edge in arena mesh": SQUARE_V + ["v 0.5 0.5 1", "f 1 2 3", "f 1 3 4", "f 3 1 5"],
    # the second triangle runs the shared edge 3-1 in the same direction
    "inconsistent triangle winding in arena mesh": SQUARE_V + ["f 1 2 3", "f 3 1 4"],
    # the second triangle folded back onto the first across their shared edge
    "opposing triangle normals in arena mesh": SQUARE_V + ["v 0.2 0.9 0", "f 1 2 3", "f 1 3 5"],
}


def _write(tmp_path, lines, name="arena.obj"):
    p = tmp_path / name
    p.write_text("\n".join(lines) + "\n")
    return p


@pytest.fixture(scope="module")
def lib():
    L = C.CDLL(str(build.engine_path()))
    L.carl_last_error.restype = C.c_char_p
    return L


def _create(lib):
    handle = C.c_void_p()
    rc = lib.carl_env_create(1, 1, 1, 0, 1, 1, C.byref(handle))
    return rc, handle.value, lib.carl_last_error().decode()


@pytest.mark.parametrize("message", sorted(BAD))
def test_malformed_mesh_fails_creation_with_the_reference_message(tmp_path, monkeypatch, lib, message):
    path = _write(tmp_path, BAD[message])
    monkeypatch.setenv("CARL_ARENA_OBJ", str(path))
    rc, handle, err = _create(lib)
    assert rc == enum_values("CARL_")["CARL_ERR_ARENA"] and handle is None
    assert message in err
    with pytest.raises(RuntimeError, match=message):
        carl.Env(1, 1, 1, 0)
    with pytest.raises(RuntimeError, match=message):
        OracleEnv(1, 1, 1, 0, obj_path=path)


def test_missing_mesh(tmp_path, monkeypatch, lib):
    monkeypatch.setenv("CARL_ARENA_OBJ", str(tmp_path / "absent.obj"))
    rc, handle, err = _create(lib)
    assert rc == enum_values("CARL_")["CARL_ERR_ARENA"] and handle is None
    assert "failed to open" in err
    with pytest.raises(RuntimeError, match="failed to open"):
        OracleEnv(1, 1, 1, 0, obj_path=tmp_path / "absent.obj")


def test_well_formed_small_mesh_builds_on_the_oracle(tmp_path):
    env = OracleEnv(1, 1, 1, 0, obj_path=_write(tmp_path, GOOD))
    verts, tris, angles, prefix, cells = env.arena()
    assert len(verts) == 4 and len(tris) == 2
    # the diagonal is the one shared, flat edge; the rest are boundary edges
    assert sorted(float(a) for a in angles.reshape(-1)).count(0.0) == 2
    env.close()
