"""The EnvIO pack entry points through the C-ABI: a step composed by a C++
host from carl_env_tick and the pack calls, in the order of
python/carl.cu:359-367, leaves every output buffer and the whole state bit
for bit equal to the fused carl_env_step, over episodes short enough that
simulations finish and reset on most steps."""
import ctypes as C

import numpy as np
import pytest
import torch

from carl_amd import build, workloads

pytestmark = pytest.mark.gpu

CONTINUOUS, DISCRETE = 1, 0
PARAM_MAX_TICKS, PARAM_NO_TOUCH = 0, 2
DTYPES = {0: torch.float32, 1: torch.int32, 2: torch.bool}


class _Device:
    """A device buffer viewed as a tensor (no copy)."""

    def __init__(self, ptr, shape, dtype):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": {torch.float32: "<f4", torch.int32: "<i4",
                                                                            torch.bool: "|b1"}[dtype],
                                         "data": (ptr, False), "version": 3}


@pytest.fixture(scope="module")
def lib():
    L = C.CDLL(str(build.engine_path()))
    L.carl_last_error.restype = C.c_char_p
    vp = C.c_void_p
    for name, args in {
        "carl_env_create": [C.c_int] * 6 + [C.POINTER(vp)], "carl_env_destroy": [vp],
        "carl_env_step": [vp, C.c_int, vp], "carl_env_tick": [vp, C.c_int, vp, C.c_int],
        "carl_env_reset_dones": [vp], "carl_env_pack_rewards_dones": [vp],
        "carl_env_pack_transition_state": [vp, C.c_int], "carl_env_pack_transition_obs": [vp],
        "carl_env_pack_match_state": [vp, vp], "carl_env_pack_obs": [vp, vp], "carl_env_pack_state": [vp, vp],
        "carl_env_set_actions": [vp, C.c_int, vp], "carl_env_synchronize": [vp],
        "carl_env_set_param": [vp, C.c_int, C.c_int],
        "carl_env_buffer": [vp, C.c_int, C.POINTER(vp), C.POINTER(C.c_int64), C.POINTER(C.c_int), C.POINTER(C.c_int)],
        "carl_env_export_state": [vp, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.POINTER(C.c_int)],
    }.items():
        getattr(L, name).argtypes = args
    return L


def _ok(lib, rc):
    assert rc == 0, lib.carl_last_error()


def _buffers(lib, env):
    out = {}
    for bid in range(14):
        ptr, shape, nd, dt = C.c_void_p(), (C.c_int64 * 3)(), C.c_int(), C.c_int()
        _ok(lib, lib.carl_env_buffer(env, bid, C.byref(ptr), shape, C.byref(nd), C.byref(dt)))
        t = torch.as_tensor(_Device(ptr.value, shape[:nd.value], DTYPES[dt.value]), device="cuda:0")
        out[bid] = t.clone()
    return out


def _state(lib, env, n_cars_total, n_sim):
    car = np.zeros(81 * n_cars_total, np.uint32)
    sim = np.zeros(67 * n_sim, np.uint32)
    tick = C.c_int()
    _ok(lib, lib.carl_env_export_state(env, car.ctypes.data_as(C.POINTER(C.c_uint32)),
                                       sim.ctypes.data_as(C.POINTER(C.c_uint32)), C.byref(tick)))
    return car, sim, tick.value


@pytest.mark.parametrize("n_blue,frameskip,discrete", [(1, 8, False), (2, 1, True), (3, 4, False)])
def test_composed_step_matches_the_fused_step(gpu, lib, n_blue, frameskip, discrete):
    n_sim, nc = 96, 2 * n_blue
    envs = []
    for _ in range(2):
        h = C.c_void_p()
        _ok(lib, lib.carl_env_create(n_sim, n_blue, n_blue, 5, frameskip, 1 | 4, C.byref(h)))
        _ok(lib, lib.carl_env_set_param(h, PARAM_MAX_TICKS, 3 * frameskip + 1))
        _ok(lib, lib.carl_env_set_param(h, PARAM_NO_TOUCH, 5 * frameskip))
        envs.append(h)
    fused, composed = envs
    rng = np.random.default_rng(70 + n_blue)
    kind = DISCRETE if discrete else CONTINUOUS
    finished = 0
    try:
        for step in range(14):
            a = (workloads.random_discrete_actions(rng, n_sim, nc) if discrete
                 else workloads.random_continuous_actions(rng, n_sim, nc))
            actions = torch.from_numpy(a).to("cuda:0")
            torch.cuda.synchronize()
            ptr = C.c_void_p(actions.data_ptr())
            _ok(lib, lib.carl_env_step(fused, kind, ptr))
            _ok(lib, lib.carl_env_set_actions(composed, kind, ptr))
            _ok(lib, lib.carl_env_tick(composed, kind, ptr, frameskip))
            _ok(lib, lib.carl_env_pack_rewards_dones(composed))
            _ok(lib, lib.carl_env_pack_transition_state(composed, frameskip))
            _ok(lib, lib.carl_env_pack_transition_obs(composed))
            _ok(lib, lib.carl_env_reset_dones(composed))
            _ok(lib, lib.carl_env_pack_match_state(composed, None))
            _ok(lib, lib.carl_env_pack_obs(composed, None))
            _ok(lib, lib.carl_env_pack_state(composed, None))
            for h in envs:
                _ok(lib, lib.carl_env_synchronize(h))
            bf, bc = _buffers(lib, fused), _buffers(lib, composed)
            for bid in range(14):
                same = torch.equal(bf[bid].view(torch.int32) if bf[bid].dtype == torch.float32 else bf[bid],
                                   bc[bid].view(torch.int32) if bc[bid].dtype == torch.float32 else bc[bid])
                assert same, f"buffer {bid} differs after step {step}"
            finished += int(bf[6].sum().item())
            sf, sc = _state(lib, fused, n_sim * nc, n_sim), _state(lib, composed, n_sim * nc, n_sim)
            assert sf[2] == sc[2]
            np.testing.assert_array_equal(sf[0], sc[0], err_msg=f"car state after step {step}")
            np.testing.assert_array_equal(sf[1], sc[1], err_msg=f"simulation state after step {step}")
        assert finished > n_sim      # the packs of finished simulations (transition rows, resets) ran
    finally:
        for h in envs:
            lib.carl_env_destroy(h)
