"""CPU checks of the Python layer's own code: the forward/up -> quaternion
conversion, the observation column map for every team size, and the action
availability mask."""
import math

import numpy as np
import pytest
import torch

import carl
from carl.gymnasium.action import CARLActionCodec
from carl.gymnasium.state import CARLObservation, CarlState
from carl.gymnasium.torch import _forward_up_to_quat, _ticks


def _rotate(q: np.ndarray, v: np.ndarray) -> np.ndarray:
    """v rotated by unit quaternions q (xyzw), in float64."""
    xyz, w = q[..., :3], q[..., 3:]
    t = 2.0 * np.cross(xyz, v)
    return v + w * t + np.cross(xyz, t)


def _check_frames(q, forward, up, tol):
    q = q.double().numpy()
    np.testing.assert_allclose(np.linalg.norm(q, axis=-1), 1.0, atol=1e-6)
    assert (q[..., 3] >= 0).all()
    np.testing.assert_allclose(_rotate(q, np.array([1.0, 0, 0])), forward, atol=tol)
    np.testing.assert_allclose(_rotate(q, np.array([0, 0, 1.0])), up, atol=tol)


# The conversion takes each component's magnitude from the square root of a
# float32 diagonal combination of the rotation matrix (the reference's copysign
# form): a component whose exact value is 0 comes out as the square root of
# that sum's rounding residue, a few float32 ulps of 1, so components (and
# the axes they rebuild) are exact to about sqrt(8 * 2^-24) / 2 = 3.5e-4.
RESIDUE = 3.6e-4


def test_quaternion_of_random_frames_reproduces_the_axes():
    rng = np.random.default_rng(0)
    q = rng.normal(size=(4096, 4))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    forward, up = _rotate(q, np.array([1.0, 0, 0])), _rotate(q, np.array([0, 0, 1.0]))
    out = _forward_up_to_quat(torch.tensor(forward, dtype=torch.float32), torch.tensor(up, dtype=torch.float32))
    _check_frames(out, forward, up, 4 * RESIDUE)
    # the same rotation as the generating quaternion, up to the sign of q
    canon = q * np.where(q[:, 3:] < 0, -1.0, 1.0)
    err = np.abs(out.double().numpy() - canon)
    assert err.max() < RESIDUE, err.max()
    # components well away from 0 carry no residue: float32 rounding only
    far = np.abs(canon) > 0.05
    assert err[far].max() < 2e-6, err[far].max()


@pytest.mark.parametrize("yaw", [0.0, 0.3, 1.0, math.pi / 2, 2.5, -0.7, -math.pi / 2, -3.0])
def test_quaternion_of_yaw_only_frames(yaw):
    """A car on its wheels (up = +z) turned by `yaw`: z and w are the half
    angle's sine and cosine; x and y, exactly 0, come out as the residue of
    1 + R00 - R11 - R22 and 1 - R00 + R11 - R22, at most RESIDUE (the reference
    conversion's behaviour)."""
    forward = torch.tensor([[math.cos(yaw), math.sin(yaw), 0.0]], dtype=torch.float32)
    up = torch.tensor([[0.0, 0.0, 1.0]], dtype=torch.float32)
    out = _forward_up_to_quat(forward, up).double().numpy()[0]
    exact = np.array([0.0, 0.0, math.sin(yaw / 2), math.cos(yaw / 2)])
    exact *= 1.0 if exact[3] >= 0 else -1.0
    assert np.abs(out[:2]).max() <= RESIDUE, out
    assert np.abs(out[2:] - exact[2:]).max() < 1e-6, (out, exact)


@pytest.mark.parametrize("axis,angle", [((1, 0, 0), math.pi), ((0, 1, 0), math.pi), ((0, 0, 1), math.pi),
                                        ((1, 1, 0), math.pi), ((0, 0, 1), 0.0), ((0, 0, 1), -math.pi / 2),
                                        ((1, 0, 0), 3.0), ((1, 0, 0), -3.0)])
def test_quaternion_of_half_turns_and_axis_rotations(axis, angle):
    """Rotations with w = 0 (half turns) and near it, where a conversion that
    divides by w fails."""
    a = np.array(axis, dtype=np.float64) / np.linalg.norm(axis)
    q = np.concatenate([a * math.sin(angle / 2), [math.cos(angle / 2)]])[None]
    forward, up = _rotate(q, np.array([1.0, 0, 0])), _rotate(q, np.array([0, 0, 1.0]))
    out = _forward_up_to_quat(torch.tensor(forward, dtype=torch.float32), torch.tensor(up, dtype=torch.float32))
    _check_frames(out, forward, up, 4 * RESIDUE)


def test_quaternion_renormalises_and_orthogonalises_the_basis():
    forward = torch.tensor([[2.0, 0.0, 0.0], [0.0, 3.0, 0.0]])
    up = torch.tensor([[0.2, 0.0, 5.0], [0.0, 0.3, 1.0]])   # not orthogonal to forward
    out = _forward_up_to_quat(forward, up)
    f = forward.double().numpy() / np.linalg.norm(forward.numpy(), axis=-1, keepdims=True)
    _check_frames(out, f, np.array([[0.0, 0, 1], [0.0, 0, 1]]), 4 * RESIDUE)


@pytest.mark.parametrize("forward,up,message", [
    ([[float("nan"), 0, 0]], [[0, 0, 1.0]], "finite"),
    ([[0.0, 0, 0]], [[0, 0, 1.0]], "define a rotation"),
    ([[1.0, 0, 0]], [[2.0, 0, 0]], "define a rotation"),
])
def test_quaternion_rejects_degenerate_frames(forward, up, message):
    with pytest.raises(ValueError, match=message):
        _forward_up_to_quat(torch.tensor(forward), torch.tensor(up))
    _forward_up_to_quat(torch.tensor(forward), torch.tensor(up), validate=False)   # masked path: no host check


def test_timeouts_in_ticks_or_seconds():
    assert _ticks(None, None, 7) == 7
    assert _ticks(5, None, 7) == 5
    assert _ticks(None, 1.0, None) == carl.PHYS_TICKS_PER_SECOND
    assert _ticks(None, 0.001, None) == 1          # rounded up to whole ticks
    for bad in ((1, 1.0), (0, None), (None, 0.0), (None, float("inf"))):
        with pytest.raises(ValueError):
            _ticks(*bad, 7)


@pytest.mark.parametrize("n_cars,previous", [(n, p) for n in range(1, 9) for p in (False, True)])
def test_observation_blocks_tile_the_row(n_cars, previous):
    """The named blocks of an observation row, in row order, tile the row
    exactly (widths of include/Cuda/DLPack.h:95-107).  Float views are read
    on a row holding each column's own index; flag views on one-hot rows."""
    dim = (carl.OBS_BALL + carl.OBS_PER_CAR * n_cars + carl.OBS_BOOST_PADS + carl.OBS_RELATIVE_EGO_BALL
           + carl.OBS_RELATIVE_PER_OTHER_CAR * (n_cars - 1) + carl.OBS_RELATIVE_GOALS + carl.OBS_EGO_DODGE
           + carl.OBS_EGO_CONTROLLER + (carl.OBS_PREVIOUS_CONTROLS if previous else 0))
    index_row = CARLObservation.from_tensor(torch.arange(dim, dtype=torch.float32).repeat(2, 1), n_cars)

    def cols_of(view):
        return view[0].reshape(-1).long().tolist()

    def flag_cols(name, width):
        found = []
        for c in range(dim):
            one_hot = torch.zeros(1, dim)
            one_hot[0, c] = 1.0
            v = getattr(CARLObservation.from_tensor(one_hot, n_cars), name).reshape(-1)
            found += [c] if v.any() else []
            assert int(v.sum()) <= 1
        assert len(found) == width, (name, found)
        return found

    order = (cols_of(index_row.ball) + cols_of(index_row.cars)
             + flag_cols("boost_pad_active", carl.NUM_BOOST_PADS) + cols_of(index_row.boost_pad_distance)
             + cols_of(index_row.ego_ball_relative) + cols_of(index_row.ego_other_relative)
             + cols_of(index_row.own_goal_relative) + cols_of(index_row.opponent_goal_relative)
             + flag_cols("ego_has_flip_or_jump", 1) + cols_of(index_row.ego_flip_window_remaining[..., None])
             + cols_of(index_row.ego_controller))
    if previous:
        order += cols_of(index_row.ego_previous_controls)
    assert order == list(range(dim))
    assert index_row.car_end == carl.OBS_BALL + carl.OBS_PER_CAR * n_cars
    controller = cols_of(index_row.ego_controller)
    assert cols_of(index_row.ego_flip_time[..., None]) == [controller[3]]
    assert cols_of(index_row.ego_demo_respawn_time[..., None]) == [controller[4]]
    assert cols_of(index_row.car_boost) == [carl.OBS_BALL + k * carl.OBS_PER_CAR + carl.OBS_BOOST
                                            for k in range(n_cars)]
    assert cols_of(index_row.cars.ego_up) == list(range(carl.OBS_BALL + carl.OBS_UP, carl.OBS_BALL + carl.OBS_BOOST))
    if not previous:
        with pytest.raises(ValueError, match="previous controls"):
            index_row.ego_previous_controls
    with pytest.raises(ValueError, match="controller v3"):
        CARLObservation.from_tensor(index_row[:, :-1], n_cars).ego_controller


def test_canonical_state_views():
    n = 3
    width = carl.OBS_BALL + carl.STATE_PER_CAR * n + carl.NUM_BOOST_PADS
    raw = torch.arange(2 * width, dtype=torch.float32).reshape(2, width)
    st = CarlState.from_raw(raw, n, torch.zeros(34, 3), torch.ones(n))
    assert torch.equal(st.ball_angular_velocity, raw[:, 6:9])
    assert torch.equal(st.car_values[:, 1], raw[:, 9 + carl.STATE_PER_CAR:9 + 2 * carl.STATE_PER_CAR])
    assert torch.equal(st.car_ball_touches, raw[:, 9 + carl.STATE_BALL_TOUCH::carl.STATE_PER_CAR][:, :n].bool())
    assert torch.equal(st.boost_pad_values, raw[:, width - 34:])
    with pytest.raises(ValueError, match="raw state shaped"):
        CarlState.from_raw(raw[:, 1:], n, torch.zeros(34, 3), torch.ones(n))


@pytest.mark.parametrize("previous", [False, True])
def test_action_mask_rules(previous):
    """Powerslide only on the ground, boost only with boost left, jump on the
    ground or with the dodge window open for more than one tick; every other
    logit always available (python/carl/gymnasium/action.py:17-38)."""
    n_cars = 2
    dim = 9 + 21 * n_cars + 68 + 6 + 6 + 6 + 2 + 5 + (8 if previous else 0)
    tail = 8 if previous else 0
    rng = np.random.default_rng(1)
    rows = []
    for on_ground in (0.0, 1.0):
        for boost in (0.0, 0.5):
            for flip in (0.0, 1.0):
                for window in (0.0, carl.PHYS_DT, 2 * carl.PHYS_DT, 1.0):
                    o = rng.normal(size=dim).astype(np.float32)
                    o[carl.OBS_EGO_ON_GROUND_INDEX] = on_ground
                    o[carl.OBS_EGO_BOOST_INDEX] = boost
                    o[dim + carl.OBS_EGO_FLIP_INDEX - tail] = flip
                    o[dim + carl.OBS_EGO_DODGE_TIME_INDEX - tail] = np.float32(window)
                    rows.append((o, on_ground, boost, flip, np.float32(window)))
    mask = CARLActionCodec(previous).mask(torch.tensor(np.stack([r[0] for r in rows])))
    assert mask.shape == (len(rows), carl.ACTION_LOGITS) and mask.dtype == torch.bool
    special = {carl.ACTION_POWERSLIDE_LOGIT, carl.ACTION_BOOST_LOGIT, carl.ACTION_JUMP_LOGIT}
    for m, (_, on_ground, boost, flip, window) in zip(mask.numpy(), rows):
        assert m[carl.ACTION_POWERSLIDE_LOGIT] == bool(on_ground)
        assert m[carl.ACTION_BOOST_LOGIT] == (boost > 0)
        assert m[carl.ACTION_JUMP_LOGIT] == (bool(on_ground) or (bool(flip) and window > np.float32(carl.PHYS_DT)))
        assert all(m[i] for i in range(carl.ACTION_LOGITS) if i not in special)
