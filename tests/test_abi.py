"""The C-ABI library without a GPU: it loads, exports every function that
include/carl_amd.h declares, and its host-only entry points (widths, argument
validation, error text) behave as documented.  No call here launches work."""
import ctypes as C

import pytest

from abi import CAR_NAMES, SIM_NAMES, abi_header_text, declared_functions, enum_values
from carl_amd import build


@pytest.fixture(scope="module")
def lib():
    path = build.engine_path()
    if not path.is_file():
        pytest.fail(f"{path} is missing: run __graft_entry__.build()")
    L = C.CDLL(str(path))
    L.carl_last_error.restype = C.c_char_p
    return L


def test_every_declared_function_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 24
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_widths_match_the_reference_formulas(lib):
    """include/Cuda/DLPack.h:95-107: obs = 9 + 21n + 68 + 6 + 6(n-1) + 6 + 2 + 5 (+8)."""
    for n in range(1, 9):
        base = 9 + 21 * n + 68 + 6 + 6 * (n - 1) + 6 + 2 + 5
        assert lib.carl_observation_dim(n, 0) == base
        assert lib.carl_observation_dim(n, 1) == base + 8
        assert lib.carl_state_dim(n) == 9 + 22 * n + 34


def test_state_layout_is_dense():
    codes = enum_values("CARL_")
    assert len(CAR_NAMES) == codes["CARL_CAR_FIELDS"] and all(CAR_NAMES)
    assert len(SIM_NAMES) == codes["CARL_SIM_FIELDS"] and all(SIM_NAMES)


@pytest.mark.parametrize("args,message", [
    ((0, 1, 1, 0, 1, 0), "n_sim must be at least 1"),
    ((4, 0, 0, 0, 1, 0), "need at least one car"),
    ((4, 5, 1, 0, 1, 0), "at most 4 cars per team"),
    ((4, 1, 1, 0, 0, 0), "frameskip must be at least 1"),
])
def test_create_rejects_invalid_arguments_before_touching_the_device(lib, args, message):
    handle = C.c_void_p()
    rc = lib.carl_env_create(*[C.c_int(a) for a in args], C.byref(handle))
    assert rc == enum_values("CARL_")["CARL_ERR_VALUE"]
    assert handle.value is None
    assert message in lib.carl_last_error().decode()


def _max_cars() -> int:
    """The largest car count whose state the 32-bit buffer offsets reach: the
    car block, 4 * CARL_CAR_FIELDS bytes per car in whole tiles of 64 cars,
    stays below 2^31 bytes."""
    return ((2 ** 31 - 1) // (4 * enum_values("CARL_")["CARL_CAR_FIELDS"])) & ~63


def test_documented_size_limit_is_the_offset_limit():
    import re

    text = abi_header_text()
    m = re.search(r"must be at most ([\d,]+) cars", text)
    assert m and int(m.group(1).replace(",", "")) == _max_cars()


@pytest.mark.parametrize("n_sim,blue,orange", [
    (_max_cars() // 2 + 1, 1, 1),      # one 1v1 simulation past the limit
    (_max_cars() // 8 + 1, 4, 4),      # 4v4
    (_max_cars() + 1, 1, 0),           # one car per simulation
    (2 ** 31 - 1, 4, 4),               # the car count itself overflows 32 bits
])
def test_create_rejects_sizes_past_the_32bit_offsets_before_any_allocation(lib, n_sim, blue, orange):
    """Sizes whose state the engine's 32-bit buffer offsets cannot address fail
    with CARL_ERR_VALUE and a message naming the limit; the check comes before
    the arena build and any device call (none exists in this container)."""
    handle = C.c_void_p()
    rc = lib.carl_env_create(n_sim, blue, orange, 0, 1, 0, C.byref(handle))
    assert rc == enum_values("CARL_")["CARL_ERR_VALUE"]
    assert handle.value is None
    err = lib.carl_last_error().decode()
    assert f"at most {_max_cars()}" in err and str(n_sim * (blue + orange)) in err


def test_null_handles_are_value_errors(lib):
    err = enum_values("CARL_")["CARL_ERR_VALUE"]
    assert lib.carl_env_step(None, 0, None) == err
    assert lib.carl_env_reset(None) == err
    assert lib.carl_env_synchronize(None) == err
    assert "null environment handle" in lib.carl_last_error().decode()


def test_boost_pad_cylinders_are_disjoint():
    """The window kernel splits a simulation's boost pads over several threads,
    which gives the serial result only if no car position can lie in two pads'
    cylinders: every pair of pad circles in the engine's table is apart."""
    import itertools
    import re
    from pathlib import Path

    import numpy as np

    text = (Path(__file__).resolve().parents[1] / "carl_amd" / "csrc" / "constants.h").read_text()
    body = text[text.index("kPadPos[kPads][3] = {"):]
    body = body[:body.index("};")]
    pads = [tuple(float(v) for v in m) for m in re.findall(r"\{\s*(-?[\d.]+)f,\s*(-?[\d.]+)f,\s*(-?[\d.]+)f\s*\}", body)]
    big = float(re.search(r"kBigPadRadius = ([\d.]+)f", text).group(1))
    small = float(re.search(r"kSmallPadRadius = ([\d.]+)f", text).group(1))
    n_big = 6  # big pads come first in the table
    assert len(pads) == 34
    radius = [big] * n_big + [small] * (len(pads) - n_big)
    gaps = [np.hypot(pads[i][0] - pads[j][0], pads[i][1] - pads[j][1]) - radius[i] - radius[j]
            for i, j in itertools.combinations(range(len(pads)), 2)]
    assert min(gaps) > 0.0, min(gaps)
    # the big pads are the six at |x| >= 3072 (corners and mid-field sides)
    assert all(abs(p[0]) >= 3072 for p in pads[:n_big])


def test_boost_pad_table_is_point_symmetric():
    """An orange observer sees pad slot p as pad mirroredPad(p); the packing
    kernels take that pad's position as pad p's with x and y negated, which is
    the same position only if the table is symmetric through the field centre
    under the engine's mirror map."""
    import re
    from pathlib import Path

    text = (Path(__file__).resolve().parents[1] / "carl_amd" / "csrc" / "constants.h").read_text()
    body = text[text.index("kPadPos[kPads][3] = {"):]
    body = body[:body.index("};")]
    pads = [tuple(float(v) for v in m) for m in re.findall(r"\{\s*(-?[\d.]+)f,\s*(-?[\d.]+)f,\s*(-?[\d.]+)f\s*\}", body)]
    fn = text[text.index("HDI int mirroredPad(int p)"):]
    fn = fn[:fn.index("}\n") + 1]
    # the map as written: p >= 6 -> 39 - p, p < 2 -> 1 - p, else 7 - p
    assert "if (p >= 6) return 39 - p;" in fn and "return p < 2 ? 1 - p : 7 - p;" in fn
    mirror = [39 - p if p >= 6 else (1 - p if p < 2 else 7 - p) for p in range(34)]
    assert sorted(mirror) == list(range(34))
    for p, q in enumerate(mirror):
        assert pads[q] == (-pads[p][0], -pads[p][1], pads[p][2]), (p, q)
