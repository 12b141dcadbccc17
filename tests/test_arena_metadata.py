"""Native arena-metadata mode (CARL_ARENA_METADATA), without a GPU.

The reader (src/ArenaMesh.cu:69-99): a count other than the mesh's triangle
count, and a file that does not open (read as count 0), fail environment
creation with CARL_ERR_ARENA and the reference's "CARL arena metadata
triangle count mismatch"; a file that ends early or holds a non-number fails
with "Invalid CARL arena metadata".  The C-ABI, the binding and the oracle
agree.

The oracle's native ball branch (BallArena/Contact.cuh:292-594) is pinned
against float64 brute force over the whole mesh: the contact triangles are
those whose native triangle comes within the native reach of the centre, in
order-key order, at most four per native mesh by Bullet's replacement rule
(a mesh of one triangle each keeps every contact), and the four arena planes
follow as closed-form contacts; the depths of the mesh contacts are the
uu-scale closest-point ones, and the native vertices, not the arena's, are
the ones tested.  The native internal-edge correction is pinned
on a small mesh by what it must do: a contact at the edge of a coplanar pair
takes the face normal, unless the ball is behind the face; a boundary edge or
a contact farther than 0.1 Bullet units from the edge leaves the normal
alone; a clamped normal is the raw one
turned about the edge axis until it sits at the edge's angle.
"""
import ctypes as C

import numpy as np
import pytest

import carl
import native_meta
from abi import enum_values
from ball_geometry import bullet_replacement, closest_on_triangles
from carl_amd import build
from oracle_py import OracleEnv

BALL_R, BREAK = 91.25, 1.905
SQUARE = ["v 0 0 0", "v 0 1 0", "v 1 1 0", "v 1 0 0", "f 1 2 3", "f 1 3 4"]


@pytest.fixture(scope="module")
def lib():
    L = C.CDLL(str(build.engine_path()))
    L.carl_last_error.restype = C.c_char_p
    return L


@pytest.fixture(scope="module")
def arena():
    env = OracleEnv(1, 1, 0, 0)
    verts, tris, angles, _, _ = env.arena()
    env.close()
    return verts, tris, angles


def _square(tmp_path, monkeypatch):
    obj = tmp_path / "square.obj"
    obj.write_text("\n".join(SQUARE) + "\n")
    monkeypatch.setenv("CARL_ARENA_OBJ", str(obj))
    return obj


def _line(mesh=0, order=0):
    return f"{mesh} {order} 6.2831853 6.2831853 0 0 0 0 0 0 0.02 0 0.02 0.02 0"


BAD = {
    "count": ("CARL arena metadata triangle count mismatch", ["3", _line(), _line(0, 1), _line(0, 2)]),
    "not a count": ("CARL arena metadata triangle count mismatch", ["two", _line(), _line(0, 1)]),
    "truncated": ("Invalid CARL arena metadata", ["2", _line()]),
    "short line": ("Invalid CARL arena metadata", ["2", _line(), "0 1 0 0 0 0 0 0 0"]),
    "non-number": ("Invalid CARL arena metadata", ["2", _line(), _line(0, 1).replace("0.02", "x", 1)]),
}


@pytest.mark.parametrize("case", sorted(BAD))
def test_malformed_metadata_fails_creation(tmp_path, monkeypatch, lib, case):
    obj = _square(tmp_path, monkeypatch)
    message, lines = BAD[case]
    meta = tmp_path / "arena.meta"
    meta.write_text("\n".join(lines) + "\n")
    monkeypatch.setenv("CARL_ARENA_METADATA", str(meta))
    handle = C.c_void_p()
    rc = lib.carl_env_create(1, 1, 1, 0, 1, 1, C.byref(handle))
    assert rc == enum_values("CARL_")["CARL_ERR_ARENA"] and handle.value is None
    assert lib.carl_last_error().decode() == message
    with pytest.raises(RuntimeError, match=message):
        carl.Env(1, 1, 1, 0)
    with pytest.raises(RuntimeError, match=message):
        OracleEnv(1, 1, 1, 0, obj_path=obj)


def test_missing_metadata_file_reads_as_count_zero(tmp_path, monkeypatch, lib):
    obj = _square(tmp_path, monkeypatch)
    monkeypatch.setenv("CARL_ARENA_METADATA", str(tmp_path / "absent.meta"))
    handle = C.c_void_p()
    assert lib.carl_env_create(1, 1, 1, 0, 1, 1, C.byref(handle)) == enum_values("CARL_")["CARL_ERR_ARENA"]
    assert lib.carl_last_error().decode() == "CARL arena metadata triangle count mismatch"
    with pytest.raises(RuntimeError, match="count mismatch"):
        OracleEnv(1, 1, 1, 0, obj_path=obj)


def test_well_formed_metadata_loads_on_the_oracle(tmp_path, monkeypatch):
    obj = _square(tmp_path, monkeypatch)
    meta = tmp_path / "arena.meta"
    # trailing text after the last triangle is not read
    meta.write_text("\n".join(["2", _line(), _line(0, 1), "trailing words"]) + "\n")
    monkeypatch.setenv("CARL_ARENA_METADATA", str(meta))
    env = OracleEnv(1, 1, 1, 0, obj_path=obj)
    env.close()


# ----------------------------------------------------------- brute force

def _expected(tv_native, mesh, key, center_uu):
    """Mesh contacts of the native branch by brute force, or None when a
    decision sits within rounding of its threshold.  Returns the kept
    (offset, depth uu, triangle, raw normal) in slot order."""
    c = center_uu * 0.02
    q = closest_on_triangles(c, tv_native[:, 0], tv_native[:, 1], tv_native[:, 2])
    dist = np.linalg.norm(c - q, axis=1)
    reach = (BALL_R + BREAK) * 0.02
    live = mesh >= 0
    if np.any(live & (np.abs(dist - reach) < 4e-5)):
        return None
    cand = np.nonzero(live & (dist < reach))[0]
    cand = cand[np.lexsort((cand, key[cand]))]
    room = 68 - len(_planes(center_uu))       # slots the planes leave
    out, kept, current = [], [], None
    for t in cand:
        if current is None or mesh[t] != current:
            out += kept
            kept, current = [], mesh[t]
        if len(kept) < 4 and len(out) + len(kept) == room:
            continue                           # no slot left: dropped
        entry = (-(c - q[t]) / dist[t] * BALL_R, BALL_R - dist[t] * 50.0, int(t), (c - q[t]) / dist[t])
        if len(kept) < 4:
            kept.append(entry)
            continue
        depths = sorted([k[1] for k in kept] + [entry[1]], reverse=True)
        if depths[0] - depths[1] < 2e-3:
            return None
        slot, tie = bullet_replacement([(k[0], k[1]) for k in kept], (entry[0], entry[1]))
        if tie:
            return None
        kept[slot] = entry
    return out + kept


def _planes(center):
    rows = []
    for n, off in (((0, 0, 1), 0.0), ((0, 0, -1), -2044.0), ((1, 0, 0), -4096.0), ((-1, 0, 0), -4096.0)):
        depth = BALL_R - (np.dot(n, center) - off)
        if depth > -BREAK:
            rows.append((np.array(n, float), depth))
    return rows


def _centres(verts, tris, rng, count):
    """Ball centres pressed up to 6 uu into random triangles, favouring the
    small triangles of the curved surfaces; every fourth from the back side
    of its triangle (outside the arena), where the face normal points away."""
    tv = verts[tris].astype(np.float64)
    n = np.cross(tv[:, 1] - tv[:, 0], tv[:, 2] - tv[:, 0])
    area = np.linalg.norm(n, axis=1)
    n /= area[:, None]
    weights = 1.0 / np.sqrt(np.maximum(area, 1.0))
    picks = rng.choice(len(tris), count, p=weights / weights.sum())
    side = np.where(np.arange(count) % 4 == 3, -1.0, 1.0)
    return [(tv[t].mean(0) + s * n[t] * (BALL_R - rng.uniform(0.0, 6.0))).astype(np.float32).astype(np.float64)
            for t, s in zip(picks, side)]


def _check_contacts(env, parts, centres):
    mesh, order, _, _, native = parts
    key = (mesh.astype(np.int64) * 10000 + order).astype(np.int64)
    tvn = native.astype(np.float64)
    checked = grouped = 0
    for center in centres:
        want = _expected(tvn, mesh, key, center)
        if want is None:
            continue
        tri, _, normal, depth, _ = env.ball_contacts(center)
        planes = _planes(center)
        assert list(tri) == [w[2] for w in want] + [-1] * len(planes), (center, list(tri), [w[2] for w in want])
        for i, w in enumerate(want):
            # depth back in uu; the normal a unit vector (internal edges may
            # correct it: the small-mesh tests below pin that)
            assert abs(depth[i] - w[1]) < 2e-3, (center, i, depth[i], w[1])
            assert abs(np.linalg.norm(normal[i]) - 1.0) < 1e-5
        for j, (n, d) in enumerate(planes):
            k = len(want) + j
            assert np.array_equal(normal[k], n.astype(np.float32)) and abs(depth[k] - d) < 1e-4
        checked += 1
        grouped += len({mesh[w[2]] for w in want}) > 1
    return checked, grouped


def _with_metadata(tmp_path, monkeypatch, parts):
    path = native_meta.write(tmp_path / "arena.meta", parts)
    monkeypatch.setenv("CARL_ARENA_METADATA", path)
    return OracleEnv(1, 1, 0, 0)


def test_restating_metadata_contacts_match_brute_force(tmp_path, monkeypatch, arena):
    verts, tris, angles = arena
    parts = native_meta.restating(verts, tris, angles)
    env = _with_metadata(tmp_path, monkeypatch, parts)
    checked, _ = _check_contacts(env, parts, _centres(verts, tris, np.random.default_rng(3), 400))
    env.close()
    assert checked >= 250


def test_floor_and_wall_contacts_are_the_analytic_planes(tmp_path, monkeypatch, arena):
    """Centres near the floor, ceiling and side walls: the plane triangles are
    skipped and each plane within reach adds one closed-form contact."""
    verts, tris, angles = arena
    env = _with_metadata(tmp_path, monkeypatch, native_meta.restating(verts, tris, angles))
    for center in ([0.0, 0.0, 90.0], [0.0, 0.0, 93.0], [0.0, 0.0, 1960.0], [4010.0, 0.0, 700.0],
                   [-4010.0, 200.0, 700.0], [0.0, 0.0, 400.0]):
        center = np.array(center)
        tri, _, normal, depth, _ = env.ball_contacts(center)
        planes = _planes(center)
        assert list(tri) == [-1] * len(planes), (center, list(tri))
        for k, (n, d) in enumerate(planes):
            assert np.array_equal(normal[k], n.astype(np.float32)) and abs(depth[k] - d) < 1e-4
    env.close()


@pytest.mark.parametrize("n_meshes,jitter", [(3, 0.0), (7, 1e-3)])
def test_meshes_group_contacts_in_order_key_order(tmp_path, monkeypatch, arena, n_meshes, jitter):
    """Shuffled orders over several meshes; with jitter the native vertices
    differ from the arena's by up to 0.1%, a few uu."""
    verts, tris, angles = arena
    rng = np.random.default_rng(20 + n_meshes)
    parts = native_meta.synthetic(verts, tris, angles, rng, n_meshes=n_meshes, jitter=jitter)
    env = _with_metadata(tmp_path, monkeypatch, parts)
    checked, grouped = _check_contacts(env, parts, _centres(verts, tris, rng, 400))
    env.close()
    assert checked >= 250 and grouped >= 20, (checked, grouped)


def test_one_mesh_per_triangle_keeps_every_contact(tmp_path, monkeypatch, arena):
    """One native mesh per triangle: no contact is reduced away, they come in
    key order, and where more reach the ball than the 68 slots less the
    planes (the goal's fine triangles) the later ones are dropped."""
    verts, tris, angles = arena
    rng = np.random.default_rng(31)
    parts = native_meta.synthetic(verts, tris, angles, rng, n_meshes=0, jitter=0.0)
    env = _with_metadata(tmp_path, monkeypatch, parts)
    mesh, order, _, _, native = parts
    key = mesh.astype(np.int64) * 10000 + order
    many = full = 0
    for center in _centres(verts, tris, rng, 600):
        want = _expected(native.astype(np.float64), mesh, key, center)
        if want is None:
            continue
        tri = env.ball_contacts(center)[0]
        assert list(tri[:len(want)]) == [w[2] for w in want]
        assert list(key[tri[:len(want)]]) == sorted(key[tri[:len(want)]])
        many += len(want) > 4
        full += len(want) + len(_planes(center)) == 68
    env.close()
    assert many >= 20 and full >= 1, (many, full)


# ------------------------------------------------------------ edge correction

# a square at z = 1000, clear of the analytic planes
Z0 = 1000.0
ROOF = ["v 0 0 1000", "v 0 100 1000", "v 100 100 1000", "v 100 0 1000", "f 1 2 3", "f 1 3 4"]


def _roof_env(tmp_path, monkeypatch, drop, angle, sign_bit=0, swap_bit=0):
    """Two triangles sharing the diagonal (0,0)-(100,100) (OBJ vertex lines
    store y, x, z), the second's far corner (0,100) lowered by `drop` (a
    ridge); the shared edge carries `angle` in the metadata and, in each
    triangle's own edge numbering, the side bit and the reversed-neighbour
    bit given."""
    lines = list(ROOF)
    lines[3] = f"v 100 0 {Z0 - drop}"
    obj = tmp_path / "roof.obj"
    obj.write_text("\n".join(lines) + "\n")
    monkeypatch.setenv("CARL_ARENA_OBJ", str(obj))
    monkeypatch.delenv("CARL_ARENA_METADATA", raising=False)
    env = OracleEnv(1, 1, 0, 0, obj_path=obj)
    verts, tris, _, _, _ = env.arena()
    env.close()
    tv = verts[tris].astype(np.float64)
    meta_angles = np.full((2, 3), 2.0 * np.pi, np.float32)
    flags = np.zeros(2, np.int64)
    edge = {}
    for t in range(2):
        for e in range(3):
            a, b = verts[tris[t][e]], verts[tris[t][(e + 1) % 3]]
            if {tuple(a[:2]), tuple(b[:2])} == {(0.0, 0.0), (100.0, 100.0)}:
                meta_angles[t, e] = angle
                flags[t] = (sign_bit << e) | (swap_bit << (e + 3))
                edge[t] = e
    parts = (np.zeros(2, np.int64), np.arange(2), meta_angles, flags, native_meta.native_vertices(tv))
    monkeypatch.setenv("CARL_ARENA_METADATA", native_meta.write(tmp_path / "roof.meta", parts))
    return OracleEnv(1, 1, 0, 0, obj_path=obj), tv, edge


def _raw_normal(tv, center):
    q = closest_on_triangles(center * 0.02, tv[:, 0] * 0.02, tv[:, 1] * 0.02, tv[:, 2] * 0.02)
    d = center * 0.02 - q
    return q, d / np.linalg.norm(d, axis=1)[:, None]


def test_coplanar_pair_contact_at_the_edge_takes_the_face_normal(tmp_path, monkeypatch):
    env, tv, _ = _roof_env(tmp_path, monkeypatch, 0.0, 0.0)
    # above the first triangle, 2 uu from the diagonal: the second
    # triangle's closest point is on the diagonal, its raw normal tilted
    center = np.array([51.4, 48.6, Z0 + 90.0])
    tri, _, normal, _, _ = env.ball_contacts(center)
    _, raw = _raw_normal(tv, center)
    assert sorted(tri) == [0, 1]
    assert max(abs(raw[0, 0]), abs(raw[1, 0])) > 1e-3        # one raw normal is tilted
    for k in range(2):
        assert np.array_equal(normal[k], np.array([0, 0, 1], np.float32)), normal
    # the same from below: behind the face the tilted raw normal stays
    center = np.array([51.4, 48.6, Z0 - 90.0])
    tri, _, normal, _, _ = env.ball_contacts(center)
    _, raw = _raw_normal(tv, center)
    assert sorted(tri) == [0, 1]
    for k, t in enumerate(tri):
        assert raw[t][2] < 0.0 and np.allclose(normal[k], raw[t], atol=1e-6), (normal[k], raw[t])
    env.close()


def test_boundary_edges_and_far_contacts_keep_the_raw_normal(tmp_path, monkeypatch):
    # the diagonal marked as a boundary edge: the tilted raw normal of the
    # contact on it stays
    env, tv, _ = _roof_env(tmp_path, monkeypatch, 0.0, 2.0 * np.pi)
    center = np.array([51.4, 48.6, Z0 + 90.0])
    tri, _, normal, _, _ = env.ball_contacts(center)
    _, raw = _raw_normal(tv, center)
    assert sorted(tri) == [0, 1]
    for k, t in enumerate(tri):
        assert np.allclose(normal[k], raw[t], atol=1e-6), (normal[k], raw[t])
    env.close()
    # a coplanar diagonal; the ball beside the outer edge x = 100 (a boundary
    # edge), so its contact sits on that edge with a tilted raw normal.  14 uu
    # from the diagonal the normal stays; 2.8 uu from it (within 0.1 Bullet
    # units) it becomes the face normal
    env, tv, _ = _roof_env(tmp_path, monkeypatch, 0.0, 0.0)
    far = np.array([101.0, 80.0, Z0 + 92.0])
    tri, _, normal, _, _ = env.ball_contacts(far)
    _, raw = _raw_normal(tv, far)
    assert list(tri) == [0] and abs(raw[0][0]) > 1e-3
    assert np.allclose(normal[0], raw[0], atol=1e-6), (normal[0], raw[0])
    near = np.array([101.0, 96.0, Z0 + 90.0])
    tri, _, normal, _, _ = env.ball_contacts(near)
    assert 0 in list(tri)
    for k in range(len(tri)):
        assert np.array_equal(normal[k], np.array([0, 0, 1], np.float32)), normal
    env.close()


@pytest.mark.parametrize("sign_bit,swap_bit", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_clamped_normal_is_turned_about_the_edge_to_its_angle(tmp_path, monkeypatch, sign_bit, swap_bit):
    """A ridge (the second triangle's far corner lowered): every contact
    normal the correction turns - it is neither the raw nor the face normal -
    keeps its length and its component along the edge axis, and sits at the
    edge's angle from the face normal on the flagged side."""
    drop = 20.0
    angle = float(np.arctan2(drop, 100.0 / np.sqrt(2.0)))
    turned = 0
    for edge_angle in (angle, -angle):
        env, tv, edge = _roof_env(tmp_path, monkeypatch, drop, edge_angle, sign_bit, swap_bit)
        # centres across the ridge, up to 8 uu either side, 84-97 uu above
        for off, h in np.stack(np.meshgrid(np.linspace(-8, 8, 17), np.linspace(84, 97, 14)), -1).reshape(-1, 2):
            center = np.array([50.0 + off / np.sqrt(2.0), 50.0 - off / np.sqrt(2.0), Z0 + h])
            tri, _, normal, _, _ = env.ball_contacts(center)
            _, raw = _raw_normal(tv, center)
            for k, t in enumerate(tri):
                n, r = normal[k].astype(np.float64), raw[t]
                a, b = tv[t][edge[t]], tv[t][(edge[t] + 1) % 3]
                axis = (a - b) / np.linalg.norm(a - b)
                face = np.cross(tv[t][1] - tv[t][0], tv[t][2] - tv[t][0])
                face /= np.linalg.norm(face)
                if np.allclose(n, r, atol=1e-5) or np.allclose(n, face, atol=1e-6):
                    continue
                turned += 1
                assert abs(np.linalg.norm(n) - 1.0) < 1e-5
                assert abs(np.dot(n, axis) - np.dot(r, axis)) < 1e-5
                side = face * (1.0 if sign_bit else -1.0)
                cur = np.arctan2(np.dot(n, np.cross(axis, side)), np.dot(n, side))
                assert abs(cur - edge_angle) < 1e-4, (sign_bit, swap_bit, edge_angle, cur)
        env.close()
    if sign_bit:
        # with the face side flagged the correction turns a quarter of them
        assert turned >= 20, turned
