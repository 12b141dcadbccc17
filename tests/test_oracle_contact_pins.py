"""The CPU oracle's car-mesh contact generation against brute-force geometry
(include/Physics/CarArena/Clip.cuh:163-377, Collision/Clip.cuh:5-35):

  face contacts   for a triangle whose SAT witness is a face axis, the
                  contacts are the vertices of the triangle cut by the four
                  side planes of the box face most aligned with the
                  separating axis.  Here that polygon is found by vertex
                  enumeration (triangle corners inside the slab, triangle
                  edges against the side planes, the slab's four edge lines
                  against the triangle's plane) rather than by clipping;
                  each contact sits at its vertex, moved onto the box face
                  along the separating axis, with depth = penetration of
                  the vertex through the face (clamped as the reference
                  clamps it), vertices farther than the contact break
                  distance left out
  car-car         for a face axis of two car boxes, the incident face of the
                  other box (the face most opposed to the reference face's
                  normal) cut by the reference box's side planes, each
                  vertex kept within the break distance with its depth below
                  the reference face; for an edge axis, each box's support
                  corner along the separating axis (a search over the eight
                  corners) (include/Physics/CarCar/Clip.cuh:25-197)
  edge contacts   for an edge axis, the one contact takes the box's support
                  edge toward the triangle (of the four box edges parallel
                  to the axis' car axis, the one farthest along the
                  separating axis turned toward the triangle); its
                  triangle point is the point of the triangle edge nearest
                  that box edge's line, and its box point the point of the
                  box edge nearest the triangle point (each found by a dense
                  search over the segment, so also where it falls at a
                  segment's end); where neither end is reached the two are
                  the edges' mutual closest points; depth = the SAT
                  penetration

The SAT verdicts, axes and depths themselves are pinned by linear
programming elsewhere (test_oracle_invariants.py); this file takes them as
given from the SAT probe.
"""
import ctypes as C
import itertools

import numpy as np
import pytest

from oracle_py import lib

HALF = np.array([60.186455, 43.282655, 19.262505])
BREAK = 2.03122735
FP = C.POINTER(C.c_float)
IP = C.POINTER(C.c_int)


def sat(tri: np.ndarray):
    t = np.ascontiguousarray(tri, np.float32).reshape(9)
    ov, ax, d, axis = C.c_int(), C.c_int(), C.c_float(), (C.c_float * 3)()
    lib().oracle_probe_box_tri_sat(t.ctypes.data_as(FP), C.byref(ov), C.byref(ax), C.byref(d), axis)
    return bool(ov.value), ax.value, float(d.value), np.array(axis[:], np.float64)


def contacts(tri: np.ndarray):
    t = np.ascontiguousarray(tri, np.float32).reshape(9)
    ax = C.c_int()
    cp, ap, nr, dp = (np.zeros((8, 3), np.float32), np.zeros((8, 3), np.float32), np.zeros((8, 3), np.float32),
                      np.zeros(8, np.float32))
    n = lib().oracle_probe_box_tri_contacts(t.ctypes.data_as(FP), C.byref(ax), cp.ctypes.data_as(FP),
                                            ap.ctypes.data_as(FP), nr.ctypes.data_as(FP), dp.ctypes.data_as(FP))
    return ax.value, cp[:n].astype(np.float64), ap[:n].astype(np.float64), nr[:n].astype(np.float64), \
        dp[:n].astype(np.float64)


# ------------------------------------------------------------------ geometry

def slab_polygon(poly: np.ndarray, face_axis: int) -> np.ndarray:
    """Vertices of {convex planar polygon} n {|p_a| <= HALF_a for both axes
    a != face_axis}, by enumeration of the candidate points (polygon corners
    inside the slab, polygon edges against the side planes, the slab's four
    edge lines against the polygon's plane) and a containment test."""
    others = [a for a in range(3) if a != face_axis]
    poly = np.asarray(poly, np.float64)
    k = len(poly)
    inside = lambda p, eps=1e-4: all(abs(p[a]) <= HALF[a] + eps for a in others)   # noqa: E731
    n = np.cross(poly[1] - poly[0], poly[2] - poly[0])
    cands = [v for v in poly if inside(v)]
    for i in range(k):
        a, b = poly[i], poly[(i + 1) % k]
        for ax in others:
            for side in (-1.0, 1.0):
                den = b[ax] - a[ax]
                if abs(den) < 1e-12:
                    continue
                t = (side * HALF[ax] - a[ax]) / den
                if 0.0 <= t <= 1.0:
                    p = a + t * (b - a)
                    if inside(p):
                        cands.append(p)
    for sx, sy in itertools.product((-1.0, 1.0), repeat=2):
        p = np.zeros(3)
        p[others[0]], p[others[1]] = sx * HALF[others[0]], sy * HALF[others[1]]
        if abs(n[face_axis]) < 1e-9 * np.linalg.norm(n):
            continue
        p[face_axis] = (n @ poly[0] - n[others[0]] * p[others[0]] - n[others[1]] * p[others[1]]) / n[face_axis]
        # inside the convex polygon: on the inner side of every edge
        if all(np.cross(poly[(i + 1) % k] - poly[i], p - poly[i]) @ n >= -1e-6 * (n @ n) for i in range(k)):
            cands.append(p)
    out = []
    for p in cands:
        if not any(np.linalg.norm(p - q) < 1e-3 for q in out):
            out.append(p)
    return np.array(out).reshape(-1, 3)


def closest_on_segments(p0, p1, q0, q1, grid=401):
    """Closest points of segments p0p1 and q0q1: dense grid, then refined."""
    s = np.linspace(0.0, 1.0, grid)
    P = p0 + s[:, None] * (p1 - p0)
    Q = q0 + s[:, None] * (q1 - q0)
    d = np.linalg.norm(P[:, None, :] - Q[None, :, :], axis=-1)
    i, j = np.unravel_index(np.argmin(d), d.shape)
    lo_s, hi_s = max(s[i] - 2.0 / grid, 0.0), min(s[i] + 2.0 / grid, 1.0)
    lo_t, hi_t = max(s[j] - 2.0 / grid, 0.0), min(s[j] + 2.0 / grid, 1.0)
    s2, t2 = np.linspace(lo_s, hi_s, grid), np.linspace(lo_t, hi_t, grid)
    P = p0 + s2[:, None] * (p1 - p0)
    Q = q0 + t2[:, None] * (q1 - q0)
    d = np.linalg.norm(P[:, None, :] - Q[None, :, :], axis=-1)
    i, j = np.unravel_index(np.argmin(d), d.shape)
    return P[i], Q[j], d[i, j]


def random_triangles(rng, n, kind, box_end=0.6, tri_end=False):
    """Triangles crossing the box: large ones lying across a face (face
    contacts) or slim ones cutting an edge (edge contacts).  For edge
    contacts `box_end` places the crossing along the box edge (beyond 1:
    past the box's corner) and `tri_end` starts the triangle edge just past
    the crossing, so the closest points clamp to segment ends."""
    out = []
    while len(out) < n:
        if kind == "face":
            axis = rng.integers(0, 3)
            normal = np.zeros(3)
            normal[axis] = rng.choice([-1.0, 1.0])
            normal = normal + rng.normal(scale=0.25, size=3)
            normal /= np.linalg.norm(normal)
            u = np.cross(normal, rng.normal(size=3))
            u /= np.linalg.norm(u)
            v = np.cross(normal, u)
            center = normal * (HALF[axis] - rng.uniform(0.2, 6.0)) + rng.normal(scale=15.0, size=3) * (1 - abs(normal))
            r = rng.uniform(40.0, 160.0)
            ang = rng.uniform(0, 2 * np.pi) + np.array([0.0, 2.1, 4.2]) + rng.normal(scale=0.2, size=3)
            tri = center + r * (np.cos(ang)[:, None] * u + np.sin(ang)[:, None] * v)
        else:
            edge_axis = rng.integers(0, 3)
            corner = HALF * rng.choice([-1.0, 1.0], size=3)
            corner[edge_axis] = rng.uniform(-box_end, box_end) * HALF[edge_axis]
            outward = corner / HALF
            outward[edge_axis] = 0.0
            outward /= np.linalg.norm(outward)
            tip = corner - outward * rng.uniform(0.5, 4.0)
            d = rng.normal(size=3)
            d[edge_axis] = 0.0
            d = np.cross(d, np.eye(3)[edge_axis]) + rng.normal(scale=0.3, size=3)
            d /= np.linalg.norm(d)
            away = outward * rng.uniform(30.0, 60.0)
            near = rng.uniform(1.0, 8.0) if tri_end else -rng.uniform(20, 60)
            tri = np.array([tip + d * near, tip + d * rng.uniform(20, 60),
                            tip + away + rng.normal(scale=10.0, size=3)])
        ok, ax, _, _ = sat(tri)
        if ok and ((kind == "face") == (ax < 4)):
            out.append(tri)
    return out


# ------------------------------------------------------------------ tests

def test_face_contacts_are_the_slab_polygon_moved_onto_the_face():
    rng = np.random.default_rng(31)
    checked = 0
    for tri in random_triangles(rng, 300, "face"):
        ok, ax, pen, sep = sat(tri)
        axis_idx, car_pos, arena_pos, normals, depths = contacts(tri)
        assert axis_idx == ax
        face = int(np.argmax(np.abs(sep)))
        face_normal = -np.sign(sep[face]) * np.eye(3)[face]
        poly = slab_polygon(np.asarray(tri, np.float32).astype(np.float64), face)
        dist = poly @ face_normal - HALF[face]
        keep = dist <= BREAK + 1e-4
        want = poly[keep]
        assert len(arena_pos) == len(want), (tri, arena_pos, want)
        for p in want:
            k = int(np.argmin(np.linalg.norm(arena_pos - p, axis=1)))
            assert np.linalg.norm(arena_pos[k] - p) < 2e-3, (p, arena_pos)
            d = max(p @ face_normal - HALF[face], -(pen + BREAK))
            assert abs(depths[k] + d) < 2e-3
            np.testing.assert_allclose(car_pos[k], p + sep * d, atol=3e-3)
            np.testing.assert_allclose(normals[k], sep, atol=1e-6)
        checked += len(want)
    assert checked > 600


def nearest_on_segment(p0, p1, target_fn, grid=4001):
    """Point of segment p0p1 minimising target_fn (dense search, refined)."""
    s = np.linspace(0.0, 1.0, grid)
    pts = p0 + s[:, None] * (p1 - p0)
    i = int(np.argmin(target_fn(pts)))
    s2 = np.linspace(max(s[i] - 2.0 / grid, 0.0), min(s[i] + 2.0 / grid, 1.0), grid)
    pts = p0 + s2[:, None] * (p1 - p0)
    return pts[int(np.argmin(target_fn(pts)))]


def check_edge_contact(tri32):
    ok, ax, pen, sep = sat(tri32)
    axis_idx, car_pos, arena_pos, normals, depths = contacts(tri32)
    assert axis_idx == ax >= 4 and len(car_pos) == 1
    car_axis, tri_edge = (ax - 4) // 3, (ax - 4) % 3
    on_car, on_tri = car_pos[0], arena_pos[0]
    assert abs(depths[0] - pen) < 1e-6
    others = [a for a in range(3) if a != car_axis]
    toward = sep if sep @ tri32.mean(0) > 0 else -sep
    support = None
    for sx, sy in itertools.product((-1.0, 1.0), repeat=2):
        mid = np.zeros(3)
        mid[others[0]], mid[others[1]] = sx * HALF[others[0]], sy * HALF[others[1]]
        if support is None or mid @ toward > support @ toward:
            support = mid
    p0, p1 = support.copy(), support.copy()
    p0[car_axis], p1[car_axis] = -HALF[car_axis], HALF[car_axis]
    a, b = tri32[tri_edge], tri32[(tri_edge + 1) % 3]
    axis_dir = np.eye(3)[car_axis]

    def to_line(q):
        rel = q - support
        return np.linalg.norm(rel - np.outer(rel @ axis_dir, axis_dir), axis=-1)

    want_tri = nearest_on_segment(a, b, to_line)
    want_car = nearest_on_segment(p0, p1, lambda q: np.linalg.norm(q - on_tri, axis=-1))
    scale = np.linalg.norm(b - a)
    np.testing.assert_allclose(on_tri, want_tri, atol=2e-3 + 1e-4 * scale)
    np.testing.assert_allclose(on_car, want_car, atol=2e-3)
    np.testing.assert_allclose(on_car[others], support[others], atol=1e-3)
    if np.linalg.norm(on_tri - on_car) > 1e-3:
        n = (on_tri - on_car) / np.linalg.norm(on_tri - on_car)
        want = -n if n @ tri32.mean(0) > 0 else n
        np.testing.assert_allclose(normals[0], want, atol=1e-4)
    return on_car, on_tri, (p0, p1, a, b)


@pytest.mark.parametrize("box_end,tri_end", [(0.6, False), (0.6, True)])
def test_edge_contact_points(box_end, tri_end):
    rng = np.random.default_rng(32 + tri_end)
    for tri in random_triangles(rng, 150, "edge", box_end, tri_end):
        on_car, on_tri, (p0, p1, a, b) = check_edge_contact(np.asarray(tri, np.float32).astype(np.float64))
        # away from the segment ends the two points are the edges' mutual closest points
        _, _, dmin = closest_on_segments(p0, p1, a, b)
        assert abs(np.linalg.norm(on_tri - on_car) - dmin) < 2e-3 + 1e-4 * dmin


def test_edge_contact_points_at_segment_ends():
    """Edge contacts whose triangle point or box point falls at a segment's
    end are rare (about 1 in 6,000 edge-axis contacts): triangles around a
    box corner are searched, with a fixed seed, until six of each kind are
    found."""
    rng = np.random.default_rng(11)
    at_tri_end = at_box_end = 0
    for _ in range(400_000):
        corner = HALF * rng.choice([-1.0, 1.0], size=3)
        tri = corner + rng.normal(scale=25.0, size=(3, 3))
        ok, ax, _, _ = sat(tri)
        if not ok or ax < 4:
            continue
        tri32 = np.asarray(tri, np.float32).astype(np.float64)
        _, cp, ap, _, _ = contacts(tri32)
        car_axis, tri_edge = (ax - 4) // 3, (ax - 4) % 3
        a, b = tri32[tri_edge], tri32[(tri_edge + 1) % 3]
        t = (ap[0] - a) @ (b - a) / ((b - a) @ (b - a))
        tri_clamped = t < 1e-5 or t > 1 - 1e-5
        box_clamped = abs(abs(cp[0][car_axis]) - HALF[car_axis]) < 1e-4
        if (tri_clamped and at_tri_end < 6) or (box_clamped and at_box_end < 3):
            check_edge_contact(tri32)
            at_tri_end += tri_clamped
            at_box_end += box_clamped
        if at_tri_end >= 6 and at_box_end >= 3:
            break
    assert at_tri_end >= 6 and at_box_end >= 3, (at_tri_end, at_box_end)


# ------------------------------------------------------------------ car-car

def box_box(cen_a, q_a, cen_b, q_b):
    f = lambda x: np.ascontiguousarray(x, np.float32)   # noqa: E731
    args = [f(cen_a), f(q_a), f(cen_b), f(q_b)]
    ax = C.c_int()
    pa, pb, nr, dp = (np.zeros((4, 3), np.float32), np.zeros((4, 3), np.float32), np.zeros((4, 3), np.float32),
                      np.zeros(4, np.float32))
    n = lib().oracle_probe_box_box_contacts(*[a.ctypes.data_as(FP) for a in args], C.byref(ax), pa.ctypes.data_as(FP),
                                            pb.ctypes.data_as(FP), nr.ctypes.data_as(FP), dp.ctypes.data_as(FP))
    return ax.value, pa[:n].astype(np.float64), pb[:n].astype(np.float64), nr[:n].astype(np.float64), \
        dp[:n].astype(np.float64)


def box_box_sat(cen_a, q_a, cen_b, q_b):
    f = lambda x: np.ascontiguousarray(x, np.float32)   # noqa: E731
    args = [f(cen_a), f(q_a), f(cen_b), f(q_b)]
    ov, ax, d = C.c_int(), C.c_int(), C.c_float()
    lib().oracle_probe_box_box_sat(*[a.ctypes.data_as(FP) for a in args], C.byref(ov), C.byref(ax), C.byref(d))
    return bool(ov.value), ax.value, float(d.value)


def _rot(q):
    x, y, z, w = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


CORNERS = np.array(list(itertools.product((-1.0, 1.0), repeat=3))) * HALF


def random_box_pairs(rng, n, want_edge):
    out = []
    while len(out) < n:
        q_a = rng.normal(size=4)
        q_a /= np.linalg.norm(q_a)
        q_b = rng.normal(size=4)
        q_b /= np.linalg.norm(q_b)
        cen_a = rng.uniform(-500, 500, 3)
        d = rng.normal(size=3)
        cen_b = cen_a + d / np.linalg.norm(d) * rng.uniform(40.0, 110.0)
        q_a, q_b = np.float32(q_a).astype(np.float64), np.float32(q_b).astype(np.float64)
        cen_a, cen_b = np.float32(cen_a).astype(np.float64), np.float32(cen_b).astype(np.float64)
        ok, ax, _ = box_box_sat(cen_a, q_a, cen_b, q_b)
        if ok and (ax >= 6) == want_edge:
            out.append((cen_a, q_a, cen_b, q_b))
    return out


def test_car_car_edge_contact_takes_the_support_corners():
    rng = np.random.default_rng(41)
    for cen_a, q_a, cen_b, q_b in random_box_pairs(rng, 300, True):
        _, ax, pen = box_box_sat(cen_a, q_a, cen_b, q_b)
        axis_idx, pa, pb, nr, dp = box_box(cen_a, q_a, cen_b, q_b)
        assert axis_idx == ax and len(pa) == 1 and abs(dp[0] - pen) < 1e-6
        n = nr[0]
        ra, rb = _rot(q_a), _rot(q_b)
        # A's corner farthest along -n, B's farthest along +n
        score_a, score_b = (CORNERS @ ra.T) @ -n, (CORNERS @ rb.T) @ n
        assert (ra @ pa[0]) @ -n >= score_a.max() - 1e-3
        assert (rb @ pb[0]) @ n >= score_b.max() - 1e-3
        assert min(np.abs(CORNERS - pa[0]).max(1)) < 1e-3 and min(np.abs(CORNERS - pb[0]).max(1)) < 1e-3
        # the separating axis points from B towards A
        assert n @ (cen_a - cen_b) >= -1e-3 * np.linalg.norm(cen_a - cen_b)


def test_car_car_face_contacts_are_the_clipped_incident_face():
    rng = np.random.default_rng(42)
    compared = 0
    for cen_a, q_a, cen_b, q_b in random_box_pairs(rng, 300, False):
        _, ax, pen = box_box_sat(cen_a, q_a, cen_b, q_b)
        axis_idx, pa, pb, nr, dp = box_box(cen_a, q_a, cen_b, q_b)
        assert axis_idx == ax
        ref_is_a = ax < 3
        (rc, rq), (ic, iq) = ((cen_a, q_a), (cen_b, q_b)) if ref_is_a else ((cen_b, q_b), (cen_a, q_a))
        rr, ri = _rot(rq), _rot(iq)
        faxis = ax if ref_is_a else ax - 3
        ref_n = rr[:, faxis] * (1.0 if rr[:, faxis] @ (ic - rc) >= 0 else -1.0)
        # incident face: the incident box's face whose outward normal opposes ref_n most
        normals = np.concatenate([ri.T, -ri.T])
        face = int(np.argmin(normals @ ref_n))
        iaxis, sign = face % 3, (1.0 if face < 3 else -1.0)
        u, v = [a for a in range(3) if a != iaxis]
        quad = []
        for su, sv in ((-1, -1), (1, -1), (1, 1), (-1, 1)):
            local = np.zeros(3)
            local[iaxis], local[u], local[v] = sign * HALF[iaxis], su * HALF[u], sv * HALF[v]
            quad.append(ic + ri @ local)
        quad_ref = (np.array(quad) - rc) @ rr                 # in the reference box's frame
        poly = slab_polygon(quad_ref, faxis)
        ref_n_local = rr.T @ ref_n
        depth = HALF[faxis] - poly @ ref_n_local if len(poly) else np.zeros(0)
        keep = depth >= -BREAK - 1e-4
        want, want_d = poly[keep], depth[keep]
        # points on the incident box and their projections on the reference face, in each box's frame
        inc_pts = pb if ref_is_a else pa
        ref_pts = pa if ref_is_a else pb
        if len(want) == 0:
            assert len(inc_pts) == 1 and abs(dp[0] - pen) < 1e-6
            continue
        # at most four are kept, the first in clipping order: with more
        # candidates every kept one must be among them
        assert len(inc_pts) == min(len(want), 4), (len(inc_pts), len(want))
        for k in range(len(inc_pts)):
            p = (ri @ inc_pts[k] + ic - rc) @ rr
            j = int(np.argmin(np.linalg.norm(want - p, axis=1)))
            assert np.linalg.norm(want[j] - p) < 3e-3, (p, want)
            assert abs(dp[k] - max(want_d[j], 0.0)) < 3e-3
            np.testing.assert_allclose(ref_pts[k], want[j] + ref_n_local * want_d[j], atol=3e-3)
            compared += 1
    assert compared > 300


# ------------------------------------------------------------------ manifold

def _manifold(env, car=0):
    cp, wp, nr, dp = (np.zeros((4, 3), np.float32), np.zeros((4, 3), np.float32), np.zeros((4, 3), np.float32),
                      np.zeros(4, np.float32))
    n = lib().oracle_probe_manifold(env.h, car, cp.ctypes.data_as(FP), wp.ctypes.data_as(FP), nr.ctypes.data_as(FP),
                                    dp.ctypes.data_as(FP))
    return cp[:n].astype(np.float64), wp[:n].astype(np.float64), nr[:n].astype(np.float64), dp[:n].astype(np.float64)


def _quat(axis, angle):
    axis = np.asarray(axis, float) / np.linalg.norm(axis)
    return np.concatenate([axis * np.sin(angle / 2), [np.cos(angle / 2)]])


def _qmul(a, b):
    ax, ay, az, aw = a
    bx, by, bz, bw = b
    return np.array([aw * bx + ax * bw + ay * bz - az * by, aw * by - ax * bz + ay * bw + az * bx,
                     aw * bz + ax * by - ay * bx + az * bw, aw * bw - ax * bx - ay * by - az * bz])


def test_manifold_keeps_the_deepest_mesh_contact_with_seam_normals():
    """A car pressed into the blue back wall above the goal (a grid of
    coplanar triangles, away from every analytic plane): the manifold holds
    one point, the deepest contact over every triangle of the car's cell
    (each triangle's contacts from the clip probe), and its normal is the
    wall's where the contact lies within 5 uu of a seam between coplanar
    triangles (the internal-edge adjustment, Clip.cuh:91-161) and the clip
    normal elsewhere."""
    from oracle_py import OracleEnv

    rng = np.random.default_rng(51)
    env = OracleEnv(1, 1, 0, 3)
    verts, tris, angles, prefix, cell_tris = env.arena()
    wall = np.array([0.0, 1.0, 0.0])
    seams = at_seam = 0
    for trial in range(120):
        facing = rng.choice([-np.pi / 2, 0.0, np.pi])           # nose, side or tail toward the wall
        q = _quat((0, 0, 1), facing + rng.normal(scale=0.08))
        q = _qmul(q, _quat(rng.normal(size=3), rng.normal(scale=0.06)))
        q = np.float32(q / np.linalg.norm(q)).astype(np.float64)
        pos = np.array([rng.uniform(-900.0, -100.0), -4900.0, rng.uniform(850.0, 1450.0)])
        env.set_car(pos[None, None], q[None, None], np.zeros((1, 1, 3)), np.zeros((1, 1, 3)), np.zeros((1, 1), bool))
        car, _, _ = env.export_state()
        cen = f32c(car, "CEN")
        r = _rot(q)
        world_corners = CORNERS @ r.T
        deepest = int(np.argmin(world_corners[:, 1]))
        pos[1] += -5120.0 - rng.uniform(0.3, 3.0) - (cen[1] + world_corners[deepest, 1])
        if trial % 2:
            # the deepest corner 0.6 to 4.5 uu beside a vertical seam of the 256 uu grid
            x = cen[0] + world_corners[deepest, 0]
            seam = 256.0 * np.round(x / 256.0)
            pos[0] += seam + rng.choice([-1.0, 1.0]) * rng.uniform(0.6, 4.5) - x
        env.set_car(pos[None, None], q[None, None], np.zeros((1, 1, 3)), np.zeros((1, 1, 3)), np.zeros((1, 1), bool))
        car, _, _ = env.export_state()
        cen, q = f32c(car, "CEN"), f32c(car, "ROT", 4)
        r = _rot(q)
        cell, count = env.broadphase()
        cell_list = cell_tris[prefix[cell[0]]:prefix[cell[0]] + count[0]]
        best = None
        for t in cell_list:
            local = ((verts[tris[t]].astype(np.float64) - cen) @ r).astype(np.float32).astype(np.float64)
            ax, cp, ap, nr, dp = contacts(local)
            for k in range(len(cp)):
                if best is None or dp[k] > best[3] + 1e-6:
                    best = (cp[k], ap[k], nr[k], dp[k], t)
        mp, wp, wn, md = _manifold(env)
        if best is None:
            assert len(mp) == 0
            continue
        assert len(mp) == 1, (len(mp), trial)
        np.testing.assert_allclose(mp[0], best[0], atol=2e-2)
        assert abs(md[0] + best[3]) < 2e-2
        # normal: the wall's near a seam between coplanar triangles, else the clip normal
        world_arena = r @ best[1] + cen
        near_seam = False
        t = best[4]
        for e in range(3):
            a, b = verts[tris[t][e]].astype(np.float64), verts[tris[t][(e + 1) % 3]].astype(np.float64)
            if abs(angles[t][e]) >= 2 * np.pi:
                continue
            s = np.clip((world_arena - a) @ (b - a) / ((b - a) @ (b - a)), 0.0, 1.0)
            if np.linalg.norm(world_arena - (a + s * (b - a))) < 5.0:
                near_seam |= angles[t][e] == 0.0
        clip_normal = r @ best[2]
        if near_seam and clip_normal @ wall >= 0.0:
            np.testing.assert_allclose(wn[0], wall, atol=1e-5)
            at_seam += 1
        else:
            np.testing.assert_allclose(wn[0], clip_normal, atol=1e-4)
        seams += near_seam
    assert at_seam >= 10, at_seam
    env.close()


def f32c(car, name, n=3):
    from abi import CAR_NAMES
    i = CAR_NAMES.index(f"CARL_CAR_{name}_0")
    return car[i:i + n, 0].astype(np.uint32).view(np.float32).astype(np.float64)


def _rotate_about(v, axis, angle):
    return v * np.cos(angle) + np.cross(axis, v) * np.sin(angle) + axis * (axis @ v) * (1.0 - np.cos(angle))


def _tri_normal(verts, tris, t):
    v = verts[tris[t]].astype(np.float64)
    n = np.cross(v[1] - v[0], v[2] - v[0])
    return n / np.linalg.norm(n)


def _seam_expected(n, N, Nb, E):
    """The normal a mesh contact keeps at a seam between two non-coplanar
    triangles (Bullet's internal-edge adjustment, Clip.cuh:91-161), stated on
    the edge's normal cone: N is the contact triangle's normal, Nb the
    neighbour's (from the mesh, not from the stored edge angle), E the edge.
    Angles are measured about E from N, positive toward E x N.
      concave seam (the neighbour turns toward the contact side, its angle
        below 0): a normal pointing out of both faces becomes N; any other
        normal stays
      convex seam (angle above 0): a normal pointing behind both faces
        stays; a normal beyond the neighbour's normal is turned about E onto
        the neighbour's angle (its E component kept), if it then still
        points out of the contact triangle; any other normal stays
    Returns (expected normal, branch name, distance of the inputs from a
    decision boundary)."""
    u = np.cross(E, N)
    beta = np.arctan2(Nb @ u, Nb @ N)
    if beta < 0.0:
        margin = min(abs(n @ N), abs(n @ Nb))
        if n @ N > 0.0 and n @ Nb > 0.0:
            return N, "concave: onto the face", margin
        return n, "concave: kept", margin
    if n @ N < 0.0 and n @ Nb < 0.0:
        return n, "convex: kept (behind both faces)", min(abs(n @ N), abs(n @ Nb))
    theta = np.arctan2(n @ u, n @ N)
    if theta > beta:
        turned = _rotate_about(n, E, beta - theta)
        margin = min(theta - beta, abs(turned @ N))
        if turned @ N > 0.0:
            return turned / np.linalg.norm(turned), "convex: turned onto the neighbour", margin
        return n, "convex: kept (turn rejected)", margin
    return n, "convex: kept (inside the cone)", beta - theta


def test_manifold_normals_at_seams_between_non_coplanar_triangles():
    """A car corner pressed 0.2-2.5 uu into the arena mesh within a few uu
    of a seam whose two triangles meet at an angle (the quarter pipes'
    facets, concave; the goal mouth's rounded edges, convex): the manifold's
    mesh point is the deepest clip contact over the car's cell, and its
    normal follows the edge's normal cone (`_seam_expected`), with the
    neighbour triangle's normal taken from the mesh.  Contacts farther than
    5 uu from every internal edge keep the clip normal."""
    from oracle_py import OracleEnv

    rng = np.random.default_rng(77)
    env = OracleEnv(1, 1, 0, 3)
    verts, tris, angles, prefix, cell_tris = env.arena()
    verts64 = verts.astype(np.float64)
    edges = {}
    for t in range(len(tris)):
        for e in range(3):
            a, b = int(tris[t][e]), int(tris[t][(e + 1) % 3])
            edges.setdefault((min(a, b), max(a, b)), []).append(t)

    def neighbour(t, e):
        a, b = int(tris[t][e]), int(tris[t][(e + 1) % 3])
        others = [x for x in edges[(min(a, b), max(a, b))] if x != t]
        return others[0] if len(others) == 1 else None

    # seams off the analytic planes (floor, ceiling, side walls)
    targets = {"concave": [], "convex": []}
    for t in range(len(tris)):
        c = verts64[tris[t]].mean(axis=0)
        if not 8.0 < c[2] < 2030.0 or abs(c[0]) > 4080.0:
            continue
        for e in range(3):
            if 0.0 < abs(angles[t][e]) < 2 * np.pi and neighbour(t, e) is not None:
                targets["convex" if angles[t][e] > 0 else "concave"].append((t, e))
    assert len(targets["concave"]) > 100 and len(targets["convex"]) > 20

    branches = {}
    checked = 0
    for trial in range(800):
        kind = "convex" if trial % 2 else "concave"
        t, e = targets[kind][rng.integers(len(targets[kind]))]
        N = _tri_normal(verts, tris, t)
        v0, v1 = verts64[tris[t][e]], verts64[tris[t][(e + 1) % 3]]
        E = (v1 - v0) / np.linalg.norm(v1 - v0)
        inward = np.cross(N, E)
        opp = verts64[tris[t][(e + 2) % 3]]
        if (opp - v0) @ inward < 0.0:
            inward = -inward
        target = v0 + (v1 - v0) * rng.uniform(0.15, 0.85) + inward * rng.uniform(-1.0, 6.0) \
            - N * rng.uniform(0.2, 2.5)
        if trial % 4 < 2:
            q = rng.normal(size=4)
        else:
            # a box face nearly parallel to the triangle (tilted up to ~0.2
            # rad), so that box-face axes separate and the clip normal
            # differs from the triangle's
            axis = np.zeros(3)
            axis[rng.integers(3)] = rng.choice([-1.0, 1.0])
            want_axis = -N
            c = np.cross(axis, want_axis)
            q = _quat(c, np.arccos(np.clip(axis @ want_axis, -1.0, 1.0))) if np.linalg.norm(c) > 1e-9 else \
                (np.array([0.0, 0.0, 0.0, 1.0]) if axis @ want_axis > 0 else _quat(np.cross(axis, [0.3, 0.5, 0.8]), np.pi))
            q = _qmul(_quat(N, rng.uniform(0, 2 * np.pi)), q)
            q = _qmul(_quat(rng.normal(size=3), abs(rng.normal(scale=0.1))), q)
        q = np.float32(q / np.linalg.norm(q)).astype(np.float64)
        pos = target + N * 60.0
        env.set_car(pos[None, None], q[None, None], np.zeros((1, 1, 3)), np.zeros((1, 1, 3)), np.zeros((1, 1), bool))
        car, _, _ = env.export_state()
        cen, r = f32c(car, "CEN"), _rot(f32c(car, "ROT", 4))
        corner = CORNERS[int(np.argmin((CORNERS @ r.T) @ N))]
        pos += target - (cen + r @ corner)
        env.set_car(pos[None, None], q[None, None], np.zeros((1, 1, 3)), np.zeros((1, 1, 3)), np.zeros((1, 1), bool))
        car, _, _ = env.export_state()
        cen, r = f32c(car, "CEN"), _rot(f32c(car, "ROT", 4))
        cell, count = env.broadphase()
        best, hits = None, 0
        for tt in cell_tris[prefix[cell[0]]:prefix[cell[0]] + count[0]]:
            local = ((verts[tris[tt]].astype(np.float64) - cen) @ r).astype(np.float32).astype(np.float64)
            ax, cp, ap, nr, dp = contacts(local)
            hits += len(cp) > 0
            for k in range(len(cp)):
                if best is None or dp[k] > best[3] + 1e-6:
                    best = (cp[k], ap[k], nr[k], dp[k], tt)
        if best is None or best[3] > 2.6 or hits > 32:
            continue                         # the car cuts the mesh elsewhere, or more SAT hits than the search keeps
        mp, wp, wn, md = _manifold(env)
        # the mesh point (an analytic plane's point may sit beside it, and
        # one at the same corner takes its place)
        mine = [i for i in range(len(mp)) if np.abs(mp[i] - best[0]).max() < 2e-2]
        if not mine:
            assert any(np.linalg.norm(mp[i] - best[0]) < BREAK for i in range(len(mp))), trial
            continue
        wn = wn[mine]
        # the nearest internal edge of the contact's triangle
        tb = best[4]
        arena_pt = r @ best[1] + cen
        n = r @ best[2]
        n = n / np.linalg.norm(n)
        dist = []
        for eb in range(3):
            if abs(angles[tb][eb]) >= 2 * np.pi:
                continue
            a, b = verts64[tris[tb][eb]], verts64[tris[tb][(eb + 1) % 3]]
            s = np.clip((arena_pt - a) @ (b - a) / ((b - a) @ (b - a)), 0.0, 1.0)
            dist.append((np.linalg.norm(arena_pt - (a + s * (b - a))), eb))
        dist.sort()
        if not dist or dist[0][0] >= 5.0:
            want, branch, margin = n, "no seam within 5 uu", 1.0
            margin = 1.0 if not dist else dist[0][0] - 5.0
        else:
            eb = dist[0][1]
            if len(dist) > 1 and dist[1][0] - dist[0][0] < 1e-3:
                continue
            Nt = _tri_normal(verts, tris, tb)
            nb = neighbour(tb, eb)
            if angles[tb][eb] == 0.0 or nb is None:
                continue                     # coplanar seams: the wall test above
            a, b = verts64[tris[tb][eb]], verts64[tris[tb][(eb + 1) % 3]]
            want, branch, margin = _seam_expected(n, Nt, _tri_normal(verts, tris, nb), (b - a) / np.linalg.norm(b - a))
            margin = min(margin, abs(dist[0][0] - 5.0))
        if margin < 2e-3:
            continue                         # too close to a decision boundary for float32
        np.testing.assert_allclose(wn[0], want, atol=2e-4, err_msg=f"trial {trial}: {branch}")
        branches[branch] = branches.get(branch, 0) + 1
        if np.abs(want - n).max() > 1e-3:
            branches["normal changed"] = branches.get("normal changed", 0) + 1
        checked += 1
    env.close()
    assert checked >= 200, (checked, branches)
    # ("concave: kept" needs a clip normal within 90 degrees of one face and
    # not of the other, and "convex: kept (turn rejected)" one turned past
    # the face's own plane: at these seams' angles neither occurs.  Clip
    # contacts whose normal is not the triangle's lie on a triangle edge, so
    # the 5 uu reach of the adjustment is not exercised either.)
    for branch in ("concave: onto the face", "convex: turned onto the neighbour", "convex: kept (inside the cone)",
                   "normal changed"):
        assert branches.get(branch, 0) >= 5, branches


def _wedge_obj(path, phi, theta, z=300.0, size=300.0):
    """A two-triangle mesh away from every analytic plane: T1 = (A, B, C)
    level at height z, its edges AB (along +x) and BC open (no neighbour),
    the angle at A between AB and AC phi; T2 shares CA and folds down across
    it by theta (a convex seam).  A point of AB at x = A.x + s lies
    s sin(phi) from the seam's line.  OBJ vertex lines list (y, x, z), as
    the arena file does."""
    a = np.array([0.0, 0.0, z])
    u = np.array([np.cos(phi), np.sin(phi), 0.0])      # along AC
    w = np.array([-np.sin(phi), np.cos(phi), 0.0])     # level, away from T1 across AC
    pts = [a, a + [size, 0.0, 0.0], a + size * u,
           a + 0.5 * size * u + 0.7 * size * (w * np.cos(theta) - np.array([0.0, 0.0, 1.0]) * np.sin(theta))]
    path.write_text("\n".join(f"v {p[1]:.6f} {p[0]:.6f} {p[2]:.6f}" for p in pts) + "\nf 1 2 3\nf 1 3 4\n")
    return a


def wedge_trials(obj, apex, theta_deg, trials, seed):
    """Random car poses pressed into the open edge AB of a wedge mesh
    (`_wedge_obj`) near its apex, from above or from below, run through the
    oracle.  Yields, for each pose whose deepest clip contact lies on T1 (and
    is deep enough and far enough from a tie with T2 to hold in float32):
    the car's position and rotation, the contact's distance from the seam,
    the normal the manifold should keep there (`_seam_expected` within 5 uu,
    the clip normal beyond), the manifold's normal, and a category."""
    from oracle_py import OracleEnv

    env = OracleEnv(1, 1, 0, 3, obj_path=obj)
    verts, tris, angles, _, _ = env.arena()
    assert len(tris) == 2
    seam = [e for e in range(3) if abs(angles[0][e]) < 2 * np.pi]
    assert len(seam) == 1 and 0.0 < angles[0][seam[0]] < np.pi
    a, b = verts[tris[0][seam[0]]].astype(np.float64), verts[tris[0][(seam[0] + 1) % 3]].astype(np.float64)
    E, N, Nb = (b - a) / np.linalg.norm(b - a), _tri_normal(verts, tris, 0), _tri_normal(verts, tris, 1)
    rng = np.random.default_rng(seed)
    for trial in range(trials):
        # the apex angle is 150 degrees: a point of AB at s lies s / 2 from the seam
        p = apex + [rng.uniform(6.0, 14.0) if theta_deg < 90 else rng.uniform(2.0, 25.0), 0.0, 0.0]
        q = rng.normal(size=4)
        q = np.float32(q / np.linalg.norm(q)).astype(np.float64)
        pos = p + [0.0, 0.0, 100.0]
        env.set_car(pos[None, None], q[None, None], np.zeros((1, 1, 3)), np.zeros((1, 1, 3)), np.zeros((1, 1), bool))
        car, _, _ = env.export_state()
        cen, r = f32c(car, "CEN"), _rot(f32c(car, "ROT", 4))
        heights = (CORNERS @ r.T)[:, 2]
        if trial % 2:      # from below: the highest corner just above the edge, the box under the open side
            corner, target = CORNERS[int(np.argmax(heights))], p + [0.0, rng.uniform(-5.0, 1.0), rng.uniform(0.2, 2.0)]
        else:              # from above: the lowest corner just below
            corner, target = CORNERS[int(np.argmin(heights))], p + [0.0, rng.uniform(-30.0, 5.0), -rng.uniform(0.2, 2.0)]
        pos = np.float32(pos + target - (cen + r @ corner)).astype(np.float64)
        env.set_car(pos[None, None], q[None, None], np.zeros((1, 1, 3)), np.zeros((1, 1, 3)), np.zeros((1, 1), bool))
        car, _, _ = env.export_state()
        cen, r = f32c(car, "CEN"), _rot(f32c(car, "ROT", 4))
        best, deepest = None, [-np.inf, -np.inf]
        for t in range(2):
            local = ((verts[tris[t]].astype(np.float64) - cen) @ r).astype(np.float32).astype(np.float64)
            _, cp, ap, nr, dp = contacts(local)
            for k in range(len(cp)):
                deepest[t] = max(deepest[t], dp[k])
                if best is None or dp[k] > best[3] + 1e-6:
                    best = (cp[k], ap[k], nr[k], dp[k], t)
        if best is None or best[4] != 0 or best[3] < 0.1 or deepest[1] > best[3] - 1e-3:
            continue          # none on T1, too shallow for its normal to hold in float32, or tied with T2's
        mp, _, wn, _ = _manifold(env)
        mine = [i for i in range(len(mp)) if np.abs(mp[i] - best[0]).max() < 2e-2]
        assert len(mine) == 1, trial
        n = r @ best[2]
        n /= np.linalg.norm(n)
        x = r @ best[1] + cen
        s = np.clip((x - a) @ (b - a) / ((b - a) @ (b - a)), 0.0, 1.0)
        dist = np.linalg.norm(x - (a + s * (b - a)))
        ruled, branch, margin = _seam_expected(n, N, Nb, E)
        if min(margin, abs(dist - 5.0)) < 2e-3:
            continue                         # too close to a decision boundary for float32
        changes = np.abs(ruled - n).max() > 1e-2
        key = (f"within 5 uu: {branch}" if dist < 5.0 else
               "beyond 5 uu, where the rule would turn it" if changes else "beyond 5 uu, inside the cone")
        yield dict(trial=trial, pos=pos, rot=q, dist=dist, want=ruled if dist < 5.0 else n, got=wn[mine[0]],
                   key=key, branch=branch)
    env.close()


@pytest.mark.parametrize("theta_deg", [8, 120])
def test_manifold_seam_reach_and_sharp_convex_seam_on_a_wedge_mesh(tmp_path, theta_deg):
    """The internal-edge adjustment's reach and its rejected convex turn
    (Clip.cuh:91-161), which the arena mesh does not exercise (its contacts
    off the face normal lie on the contact's own internal edge, and its
    sharpest convex seam folds 45 degrees): on a wedge mesh (`_wedge_obj`),
    a car corner or edge pressed 0.2-2 uu into the open edge AB, from above
    or from below, near the wedge's apex.  The manifold's mesh point is the
    deepest clip contact; where that lies on T1 within 5 uu of the seam its
    normal follows the seam's normal cone (`_seam_expected`), and beyond 5
    uu it keeps the clip normal.  With the seam folded 8 degrees the cone is
    narrow, so the rule turns most normals both within 5 uu and just beyond
    (there the reach alone keeps them); folded 120 degrees, a normal turned
    onto the neighbour's angle would point into T1, and the turn is
    rejected."""
    obj = tmp_path / "wedge.obj"
    apex = _wedge_obj(obj, np.radians(150.0), np.radians(theta_deg))
    seen = {}
    for c in wedge_trials(obj, apex, theta_deg, 6000, 150 + theta_deg):
        np.testing.assert_allclose(c["got"], c["want"], atol=2e-4,
                                   err_msg=f"trial {c['trial']}: {c['branch']}, {c['dist']:.2f} uu")
        seen[c["key"]] = seen.get(c["key"], 0) + 1
    if theta_deg == 8:
        need = ("within 5 uu: convex: turned onto the neighbour", "beyond 5 uu, where the rule would turn it")
    else:
        need = ("within 5 uu: convex: kept (turn rejected)",)
    for key in need:
        assert seen.get(key, 0) >= 10, seen
