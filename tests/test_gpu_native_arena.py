"""Native arena meshes (CARL_ARENA_METADATA) on the GPU.

With a metadata file the engine's ball meets the arena through the native
branch (BallArena/Contact.cuh:292-594): native triangles in Bullet units,
visited in order-key order, at most four contacts per native mesh, the arena
planes as analytic contacts, and up to 68 contacts in the averaged solve.
These tests run the engine and the oracle on the same synthetic metadata
(tests/native_meta.py: the arena restated as one mesh; five shuffled meshes
with random edge flags and moved vertices; one mesh per triangle, where balls
among the goal's fine triangles fill all 68 contact slots) from balls and cars placed in the densest
geometry (half of the simulations placed there again before every step),
and require the whole state and every output to agree bit for bit
after every step, on the window kernel and on the phase kernels.
"""
import numpy as np
import pytest

import native_meta
from carl_amd import workloads
from gpu_harness import Pair, dense_geometry_reset_state
from abi import enum_values
from oracle_py import OracleEnv

pytestmark = pytest.mark.gpu
BALL_POS = enum_values("CARL_SIM_")["CARL_SIM_BALL_POS"]

CASES = {
    "restating": lambda a, rng: native_meta.restating(*a),
    "five meshes": lambda a, rng: native_meta.synthetic(*a, rng, n_meshes=5),
    "mesh per triangle": lambda a, rng: native_meta.synthetic(*a, rng, n_meshes=0),
}


@pytest.fixture(scope="module")
def arena():
    env = OracleEnv(1, 1, 0, 0)
    verts, tris, angles, _, _ = env.arena()
    env.close()
    return verts, tris, angles


@pytest.mark.parametrize("window", [64, 0])
@pytest.mark.parametrize("case", sorted(CASES))
def test_native_arena_matches_the_oracle(gpu, tmp_path, monkeypatch, arena, case, window):
    rng = np.random.default_rng(sorted(CASES).index(case) * 10 + (window > 0))
    monkeypatch.setenv("CARL_ARENA_METADATA", native_meta.write(tmp_path / "arena.meta", CASES[case](arena, rng)))
    n_sim, n_blue, frameskip = 192, 2, 4
    pair = Pair(n_sim, n_blue, n_blue, seed=61, frameskip=frameskip)
    try:
        assert pair.gpu.native_arena
        pair.gpu.tick_window = window
        pair.apply_reset_state(dense_geometry_reset_state(rng, n_sim, 2 * n_blue))
        touching = grouped = full = 0
        for step in range(16):
            # half the simulations start again in the densest geometry
            mask = rng.uniform(size=n_sim) < 0.5
            pair.apply_reset_state(dense_geometry_reset_state(rng, n_sim, 2 * n_blue), reset_mask=mask)
            # balls with native mesh contacts (not only planes) at the step's start
            pos = pair.cpu.export_state()[1][BALL_POS:BALL_POS + 3].view(np.float32).T
            for p in pos:
                tri = pair.cpu.ball_contacts(p)[0]
                touching += int(np.any(tri >= 0))
                grouped += int(np.count_nonzero(tri >= 0) >= 8)
                full += int(len(tri) == 68)
            pair.step_continuous(workloads.random_continuous_actions(rng, n_sim, 2 * n_blue))
            report = pair.state_mismatches() + pair.output_mismatches()
            assert not report, f"{case}, window {window}, after step {step}:\n  " + "\n  ".join(report)
        assert touching >= 16 * n_sim // 8, touching
        if case != "restating":
            assert grouped >= 100, grouped      # several native meshes at once
        if case == "mesh per triangle":
            assert full >= 5, full              # all 68 slots taken, later contacts dropped
    finally:
        pair.close()


def test_without_metadata_the_default_branch_runs(gpu, monkeypatch):
    monkeypatch.delenv("CARL_ARENA_METADATA", raising=False)
    pair = Pair(8, 1, 1)
    try:
        assert not pair.gpu.native_arena
    finally:
        pair.close()


def test_stage_profile_refuses_the_native_branch(gpu, tmp_path, monkeypatch, arena):
    monkeypatch.setenv("CARL_ARENA_METADATA", native_meta.write(tmp_path / "arena.meta",
                                                                native_meta.restating(*arena)))
    pair = Pair(8, 1, 1)
    try:
        with pytest.raises(ValueError, match="native arena"):
            pair.gpu.enable_tick_timing(True, stages=True)
        pair.gpu.enable_tick_timing(True)      # whole-launch timing still works
        pair.gpu.enable_tick_timing(False)
    finally:
        pair.close()
