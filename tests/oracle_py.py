"""ctypes wrapper of the CPU oracle (oracle/liboracle.so).

Test infrastructure: the oracle is the checker the HIP engine is compared
against.  Buffers are numpy arrays; ids and field indices come from
include/carl_amd.h (mirrored in carl_amd/abi.py).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
LIB_PATH = ROOT / "oracle" / "liboracle.so"
ARENA_OBJ = ROOT / "carl_amd" / "assets" / "arena.obj"

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run __graft_entry__.build())")
        L = C.CDLL(str(LIB_PATH))
        vp, ip, fp, i64p, u8p, u32p = (C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_float),
                                       C.POINTER(C.c_int64), C.POINTER(C.c_uint8), C.POINTER(C.c_uint32))
        L.oracle_create.restype = vp
        L.oracle_create.argtypes = [C.c_int] * 6 + [C.c_char_p, C.c_char_p, C.c_int]
        L.oracle_destroy.argtypes = [vp]
        L.oracle_step.argtypes = [vp, C.c_int, vp]
        L.oracle_tick.argtypes = [vp, C.c_int, vp, C.c_int]
        L.oracle_reset.argtypes = [vp]
        L.oracle_reset_dones.argtypes = [vp]
        L.oracle_set_ball.argtypes = [vp, vp, vp, vp, vp, C.c_int]
        L.oracle_set_car.argtypes = [vp, vp, vp, vp, vp, vp, C.c_int, vp, vp, vp, C.c_int]
        L.oracle_apply_reset.argtypes = [vp] + [vp] * 8 + [C.c_int] + [vp] * 6 + [C.c_int, vp]
        L.oracle_set_match.argtypes = [vp, vp, vp, vp, vp, C.c_int]
        L.oracle_reset_pads.argtypes = [vp, vp, C.c_int]
        L.oracle_set_param.argtypes = [vp, C.c_int, C.c_int]
        L.oracle_get_param.argtypes = [vp, C.c_int]
        L.oracle_buffer.restype = C.c_long
        L.oracle_buffer.argtypes = [vp, C.c_int, C.POINTER(C.c_void_p)]
        L.oracle_export.argtypes = [vp, u32p, u32p, ip]
        L.oracle_import.argtypes = [vp, u32p, u32p, C.c_int]
        L.oracle_arena_counts.argtypes = [vp, ip, ip, ip]
        L.oracle_arena_copy.argtypes = [vp, fp, ip, fp, ip, ip]
        L.oracle_cell_of.argtypes = [C.c_float, C.c_float, C.c_float, ip]
        L.oracle_broadphase.argtypes = [vp, ip, ip]
        L.oracle_raycast.argtypes = [vp, fp, fp, ip]
        L.oracle_ball_contacts.argtypes = [vp, fp, ip, fp, fp, fp, fp]
        L.oracle_ball_hit_prev_tick.argtypes = [C.c_int, C.c_int]
        L.oracle_probe_ball_floor_split.restype = C.c_float
        L.oracle_probe_ball_floor_split.argtypes = [C.c_float, C.c_float, C.c_int]
        L.oracle_probe_dodge.argtypes = [C.c_float] * 3 + [ip, ip, fp]
        L.oracle_probe_autoflip.argtypes = [fp, C.c_int, C.c_int, fp, ip, fp, fp]
        L.oracle_probe_steer_stage.argtypes = [C.c_float, fp, fp]
        L.oracle_kickoff_perm.argtypes = [C.c_int, C.c_int]
        L.oracle_probe_box_tri_sat.argtypes = [fp, ip, ip, fp, fp]
        L.oracle_probe_box_tri_contacts.argtypes = [fp, ip, fp, fp, fp, fp]
        L.oracle_probe_box_box_contacts.argtypes = [fp, fp, fp, fp, ip, fp, fp, fp, fp]
        L.oracle_probe_manifold.argtypes = [vp, C.c_int, fp, fp, fp, fp]
        L.oracle_probe_box_box_sat.argtypes = [fp, fp, fp, fp, ip, ip, fp]
        L.oracle_hash32.restype = C.c_uint32
        L.oracle_hash32.argtypes = [C.c_uint32]
        L.oracle_sincos.argtypes = [C.c_float, fp, fp]
        L.oracle_atan2.restype = C.c_float
        L.oracle_atan2.argtypes = [C.c_float, C.c_float]
        L.oracle_integrate_quat.argtypes = [fp, fp, fp]
        L.oracle_cpu_throughput.restype = C.c_double
        L.oracle_cpu_throughput.argtypes = [C.c_char_p, C.c_int, C.c_int, C.c_int]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# buffer ids / dtypes (include/carl_amd.h)
BUFFERS = {
    "obs": (0, np.float32), "transition_obs": (1, np.float32), "state": (2, np.float32),
    "transition_state": (3, np.float32), "actions": (4, np.int32), "rewards": (5, np.float32),
    "dones": (6, np.bool_), "score_difference": (7, np.int32), "episode_ticks": (8, np.int32),
    "transition_score_difference": (9, np.int32), "transition_episode_ticks": (10, np.int32),
    "overtime": (11, np.bool_), "transition_overtime": (12, np.bool_),
    "continuous_actions": (13, np.float32),
}
CAR_FIELDS = 81
SIM_FIELDS = 67


class OracleEnv:
    """CPU oracle environment with the carl._carl.Env call sequencing."""

    def __init__(self, n_sim, n_blue, n_orange, seed, frameskip=1, invert_orange=True,
                 normalize=False, previous_controls=False, obj_path=ARENA_OBJ):
        flags = (1 if invert_orange else 0) | (2 if normalize else 0) | (4 if previous_controls else 0)
        err = C.create_string_buffer(256)
        h = lib().oracle_create(n_sim, n_blue, n_orange, seed, frameskip, flags,
                                str(obj_path).encode(), err, 256)
        if not h:
            raise RuntimeError(err.value.decode())
        self.h = C.c_void_p(h)
        self.n_sim, self.n_blue, self.n_orange = n_sim, n_blue, n_orange
        self.n_cars = n_blue + n_orange

    def close(self):
        if getattr(self, "h", None):
            lib().oracle_destroy(self.h)
            self.h = None

    __del__ = close

    # -- parameters
    def param(self, p):
        return lib().oracle_get_param(self.h, p)

    def set_param(self, p, v):
        if lib().oracle_set_param(self.h, p, int(v)) != 0:
            raise ValueError(f"invalid value {v} for parameter {p}")

    @property
    def obs_dim(self):
        return self.param(6)

    @property
    def tick_count(self):
        return self.param(9)

    # -- stepping
    def step(self, actions: np.ndarray):
        a = np.ascontiguousarray(actions)
        kind = 0 if a.dtype == np.int32 else 1
        lib().oracle_step(self.h, kind, _p(a))

    def step_continuous(self, actions):
        self.step(np.ascontiguousarray(actions, dtype=np.float32))

    def tick(self, actions, kind, n=1):
        a = np.ascontiguousarray(actions)
        lib().oracle_tick(self.h, kind, _p(a), n)

    def reset(self):
        lib().oracle_reset(self.h)

    def reset_dones(self):
        lib().oracle_reset_dones(self.h)

    # -- setters
    def set_ball(self, pos, vel, ang, idx=None):
        n = self.n_sim if idx is None else len(idx)
        arrs = [np.ascontiguousarray(x, dtype=np.float32) for x in (pos, vel, ang)]
        ii = None if idx is None else np.ascontiguousarray(idx, dtype=np.int64)
        lib().oracle_set_ball(self.h, *map(_p, arrs), _p(ii), n)

    def set_car(self, pos, rot, vel, ang, demoed, boost=None, internal=None, idx=None):
        n = self.n_sim if idx is None else len(idx)
        f = [np.ascontiguousarray(x, dtype=np.float32) for x in (pos, rot, vel, ang)]
        d = np.ascontiguousarray(demoed)
        byte = d.dtype == np.bool_
        d = d.astype(np.uint8) if byte else d.astype(np.int32)
        b = None if boost is None else np.ascontiguousarray(boost, dtype=np.float32)
        it = None if internal is None else np.ascontiguousarray(internal, dtype=np.float32)
        ii = None if idx is None else np.ascontiguousarray(idx, dtype=np.int64)
        lib().oracle_set_car(self.h, *map(_p, f), _p(d), int(byte), _p(b), _p(it), _p(ii), n)

    def apply_reset_state(self, ball_position, ball_velocity, ball_angular_velocity, car_position,
                          car_rotation, car_velocity, car_angular_velocity, car_demoed, car_boost=None,
                          car_internal_state=None, blue_score=None, orange_score=None,
                          episode_ticks=None, simulation_indices=None, reset_mask=None):
        f = [np.ascontiguousarray(x, dtype=np.float32) for x in (
            ball_position, ball_velocity, ball_angular_velocity, car_position, car_rotation,
            car_velocity, car_angular_velocity)]
        d = np.ascontiguousarray(car_demoed)
        byte = d.dtype == np.bool_
        d = d.astype(np.uint8) if byte else d.astype(np.int32)
        opt = lambda x, t: None if x is None else np.ascontiguousarray(x, dtype=t)
        b, it = opt(car_boost, np.float32), opt(car_internal_state, np.float32)
        bl, orr, tk = opt(blue_score, np.int32), opt(orange_score, np.int32), opt(episode_ticks, np.int32)
        ii = opt(simulation_indices, np.int64)
        m = None if reset_mask is None else np.ascontiguousarray(reset_mask, dtype=np.uint8)
        n = len(ii) if ii is not None else self.n_sim
        lib().oracle_apply_reset(self.h, *map(_p, f), _p(d), int(byte), _p(b), _p(it), _p(bl),
                                 _p(orr), _p(tk), _p(ii), n, _p(m))

    def set_match_state(self, blue, orange, ticks, idx=None):
        n = self.n_sim if idx is None else len(idx)
        arr = [np.ascontiguousarray(x, dtype=np.int32) for x in (blue, orange, ticks)]
        ii = None if idx is None else np.ascontiguousarray(idx, dtype=np.int64)
        lib().oracle_set_match(self.h, *map(_p, arr), _p(ii), n)

    def reset_boost_pads(self, idx=None):
        n = self.n_sim if idx is None else len(idx)
        ii = None if idx is None else np.ascontiguousarray(idx, dtype=np.int64)
        lib().oracle_reset_pads(self.h, _p(ii), n)

    # -- outputs
    def get(self, name) -> np.ndarray:
        bid, dt = BUFFERS[name]
        ptr = C.c_void_p()
        n = lib().oracle_buffer(self.h, bid, C.byref(ptr))
        itemsize = np.dtype(dt).itemsize
        raw = (C.c_ubyte * (n * itemsize)).from_address(ptr.value)
        out = np.frombuffer(raw, dtype=np.uint8 if dt == np.bool_ else dt).copy()
        if dt == np.bool_:
            out = out.astype(np.bool_)
        if name in ("obs", "transition_obs"):
            return out.reshape(self.n_sim, self.n_cars, -1)
        if name in ("state", "transition_state"):
            return out.reshape(self.n_sim, -1)
        if name in ("actions", "continuous_actions"):
            return out.reshape(self.n_sim, self.n_cars, 7)
        return out

    def export_state(self):
        car = np.zeros(CAR_FIELDS * self.n_sim * self.n_cars, np.uint32)
        sim = np.zeros(SIM_FIELDS * self.n_sim, np.uint32)
        tick = C.c_int()
        lib().oracle_export(self.h, car.ctypes.data_as(C.POINTER(C.c_uint32)),
                            sim.ctypes.data_as(C.POINTER(C.c_uint32)), C.byref(tick))
        return car.reshape(CAR_FIELDS, -1), sim.reshape(SIM_FIELDS, -1), tick.value

    def import_state(self, car, sim, tick):
        car = np.ascontiguousarray(car, dtype=np.uint32)
        sim = np.ascontiguousarray(sim, dtype=np.uint32)
        lib().oracle_import(self.h, car.ctypes.data_as(C.POINTER(C.c_uint32)),
                            sim.ctypes.data_as(C.POINTER(C.c_uint32)), int(tick))

    def arena(self):
        nv, nt, nr = C.c_int(), C.c_int(), C.c_int()
        ncell = lib().oracle_arena_counts(self.h, C.byref(nv), C.byref(nt), C.byref(nr))
        verts = np.zeros((nv.value, 3), np.float32)
        tris = np.zeros((nt.value, 3), np.int32)
        ang = np.zeros((nt.value, 3), np.float32)
        prefix = np.zeros(ncell + 1, np.int32)
        cell_tris = np.zeros(max(nr.value, 1), np.int32)
        fpp, ipp = C.POINTER(C.c_float), C.POINTER(C.c_int)
        lib().oracle_arena_copy(self.h, verts.ctypes.data_as(fpp), tris.ctypes.data_as(ipp),
                                ang.ctypes.data_as(fpp), prefix.ctypes.data_as(ipp),
                                cell_tris.ctypes.data_as(ipp))
        return verts, tris, ang, prefix, cell_tris[:nr.value]

    def ball_contacts(self, center):
        """Ball-arena contacts gathered for a ball centred at `center`, in
        slot order: (triangles, points, normals, depths, reduction offsets)."""
        tri = np.zeros(68, np.int32)
        pt, nrm, red = np.zeros((68, 3), np.float32), np.zeros((68, 3), np.float32), np.zeros((68, 3), np.float32)
        dep = np.zeros(68, np.float32)
        c = np.ascontiguousarray(center, np.float32)
        fp = C.POINTER(C.c_float)
        n = lib().oracle_ball_contacts(self.h, c.ctypes.data_as(fp), tri.ctypes.data_as(C.POINTER(C.c_int)),
                                       pt.ctypes.data_as(fp), nrm.ctypes.data_as(fp), dep.ctypes.data_as(fp),
                                       red.ctypes.data_as(fp))
        return tri[:n], pt[:n], nrm[:n], dep[:n], red[:n]

    def broadphase(self):
        n = self.n_sim * self.n_cars
        cell, cnt = np.zeros(n, np.int32), np.zeros(n, np.int32)
        ipp = C.POINTER(C.c_int)
        lib().oracle_broadphase(self.h, cell.ctypes.data_as(ipp), cnt.ctypes.data_as(ipp))
        return cell, cnt

    def raycast(self):
        n = self.n_sim * self.n_cars
        d, nrm, s = np.zeros((n, 4), np.float32), np.zeros((n, 4, 3), np.float32), np.zeros((n, 4), np.int32)
        lib().oracle_raycast(self.h, d.ctypes.data_as(C.POINTER(C.c_float)),
                             nrm.ctypes.data_as(C.POINTER(C.c_float)), s.ctypes.data_as(C.POINTER(C.c_int)))
        return d, nrm, s


def cell_of(x, y, z):
    out = (C.c_int * 3)()
    lib().oracle_cell_of(x, y, z, out)
    return tuple(out)
