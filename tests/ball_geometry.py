"""Float64 references for the ball-arena contact tests: Ericson's closest
point on a triangle and Bullet's four-point manifold replacement."""
import numpy as np


def closest_on_triangles(p, a, b, c):
    """Ericson, Real-Time Collision Detection 5.1.5, in float64, for every
    triangle (rows of a, b, c) at once."""
    ab, ac, ap, bp, cp = b - a, c - a, p - a, p - b, p - c
    d1, d2 = (ab * ap).sum(1), (ac * ap).sum(1)
    d3, d4 = (ab * bp).sum(1), (ac * bp).sum(1)
    d5, d6 = (ab * cp).sum(1), (ac * cp).sum(1)
    vc, vb, va = d1 * d4 - d3 * d2, d5 * d2 - d1 * d6, d3 * d6 - d5 * d4
    with np.errstate(divide="ignore", invalid="ignore"):
        inner = 1.0 / (va + vb + vc)
        out = a + ab * (vb * inner)[:, None] + ac * (vc * inner)[:, None]
        cases = [   # later entries take precedence (the first region of the text wins)
            ((va <= 0) & (d4 - d3 >= 0) & (d5 - d6 >= 0),
             b + (c - b) * ((d4 - d3) / ((d4 - d3) + (d5 - d6)))[:, None]),
            ((vb <= 0) & (d2 >= 0) & (d6 <= 0), a + ac * (d2 / (d2 - d6))[:, None]),
            ((d6 >= 0) & (d5 <= d6), c),
            ((vc <= 0) & (d1 >= 0) & (d3 <= 0), a + ab * (d1 / (d1 - d3))[:, None]),
            ((d3 >= 0) & (d4 <= d3), b),
            ((d1 <= 0) & (d2 <= 0), a),
        ]
    for cond, val in cases:
        out = np.where(cond[:, None], val, out)
    return out


def bullet_replacement(kept, cand):
    """Bullet's persistent-manifold point replacement (btPersistentManifold::
    sortCachedPoints): keep the deepest point (the candidate's own depth
    counts), replace the point whose removal leaves the largest quad."""
    deepest, depth = -1, cand[1]
    for i, (_, d) in enumerate(kept):
        if d > depth:
            deepest, depth = i, d
    p = [k[0] for k in kept]
    c = cand[0]
    area = [0.0] * 4
    if deepest != 0:
        area[0] = np.sum(np.cross(c - p[1], p[3] - p[2]) ** 2)
    if deepest != 1:
        area[1] = np.sum(np.cross(c - p[0], p[3] - p[2]) ** 2)
    if deepest != 2:
        area[2] = np.sum(np.cross(c - p[0], p[3] - p[1]) ** 2)
    if deepest != 3:
        area[3] = np.sum(np.cross(c - p[0], p[2] - p[1]) ** 2)
    best = max(range(4), key=lambda i: (area[i], -i))      # the first of equal maxima
    # any tie, exact ones included (float32 may split what float64 ties)
    gap = min(abs(area[best] - area[i]) for i in range(4) if i != best)
    tie = gap < 1e-4 * max(area[best], 1.0)
    return best, tie
