"""HIP engine vs CPU oracle where the internal-edge adjustment's reach and
its rejected convex turn decide the contact normal (Clip.cuh:91-161).

The arena mesh does not reach either case (its contacts off the face normal
lie on their own internal edge, and its sharpest convex seam folds 45
degrees), so the oracle's pins of them (test_oracle_contact_pins.py) run on a
wedge mesh given through CARL_ARENA_OBJ.  Here the engine runs on the same
mesh, from the poses those pins found (a car pressed into the wedge's open
edge within and beyond 5 uu of its seam, the seam folded 8 or 120 degrees),
with every car at rest and no input: the engine must match the oracle bit
for bit over every state field for 3 ticks, through the contacts, the seam
normals and the car-arena solve that follows.
"""
import numpy as np
import pytest

from gpu_harness import Pair
from test_oracle_contact_pins import _wedge_obj, wedge_trials

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("theta_deg", [8, 120])
def test_wedge_seams_match_the_oracle(gpu, tmp_path, monkeypatch, theta_deg):
    obj = tmp_path / "wedge.obj"
    apex = _wedge_obj(obj, np.radians(150.0), np.radians(theta_deg))
    poses = list(wedge_trials(obj, apex, theta_deg, 6000, 150 + theta_deg))
    keys = {}
    for c in poses:
        keys[c["key"]] = keys.get(c["key"], 0) + 1
    assert keys.get("within 5 uu: convex: turned onto the neighbour" if theta_deg == 8
                    else "within 5 uu: convex: kept (turn rejected)", 0) >= 10, keys
    n = len(poses)
    print(f"wedge {theta_deg} deg: {n} poses {keys}", flush=True)
    monkeypatch.setenv("CARL_ARENA_OBJ", str(obj))
    p = Pair(n, 1, 0, seed=5, frameskip=1, obj_path=obj)
    f32 = lambda x: np.ascontiguousarray(x, dtype=np.float32)  # noqa: E731
    ball = np.tile([2500.0, 2500.0, 500.0], (n, 1))
    p.apply_reset_state({
        "ball_position": f32(ball), "ball_velocity": f32(np.zeros((n, 3))),
        "ball_angular_velocity": f32(np.zeros((n, 3))),
        "car_position": f32(np.stack([c["pos"] for c in poses])[:, None]),
        "car_rotation": f32(np.stack([c["rot"] for c in poses])[:, None]),
        "car_velocity": f32(np.zeros((n, 1, 3))), "car_angular_velocity": f32(np.zeros((n, 1, 3))),
        "car_demoed": np.zeros((n, 1), dtype=np.bool_), "car_boost": f32(np.zeros((n, 1))),
    })
    report = p.state_mismatches()
    assert not report, "after the reset:\n  " + "\n  ".join(report)
    for tick in range(3):
        p.step_continuous(np.zeros((n, 1, 7), np.float32))
        report = p.state_mismatches()
        assert not report, f"after tick {tick + 1}:\n  " + "\n  ".join(report)
    p.close()
