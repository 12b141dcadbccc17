"""The arena is built once per process and shared per device: a second
environment on the same mesh neither rebuilds the host arena nor uploads a
device copy (the reference builds its host mesh once per process in static
locals, src/ArenaMesh.cu:17-28), and an environment keeps working, bit for bit
against the oracle, after the one that first uploaded the arena is destroyed."""
import gc
import time

import numpy as np
import pytest

import carl_amd
from carl_amd import workloads
from gpu_harness import Pair

pytestmark = pytest.mark.gpu


def test_second_environment_reuses_the_arena(gpu):
    import torch

    first = carl_amd.Env(16, 1, 1, 0)
    first.synchronize()
    torch.cuda.synchronize()
    free_before, _ = torch.cuda.mem_get_info()
    t0 = time.perf_counter()
    second = carl_amd.Env(16, 1, 1, 1)
    second.synchronize()
    seconds = time.perf_counter() - t0
    free_after, _ = torch.cuda.mem_get_info()
    # the arena's device data is about 134 MB; 16 1v1 simulations need well under a megabyte
    assert free_before - free_after < (32 << 20), (free_before - free_after) / 2 ** 20
    assert seconds < 0.05, seconds
    del first, second
    gc.collect()


def test_environment_outlives_the_one_that_uploaded_the_arena(gpu):
    first = carl_amd.Env(8, 1, 1, 3)
    pair = Pair(8, 1, 1, seed=5, frameskip=8)
    del first
    gc.collect()
    rng = np.random.default_rng(11)
    for _ in range(3):
        pair.step_continuous(workloads.random_continuous_actions(rng, 8, 2))
    report = pair.state_mismatches() + pair.output_mismatches()
    pair.close()
    assert not report, report


def test_last_environment_frees_the_arena_and_a_new_one_uploads_it_again(gpu):
    import torch

    gc.collect()
    torch.cuda.synchronize()
    env = carl_amd.Env(8, 1, 1, 0)
    env.synchronize()
    free_with, _ = torch.cuda.mem_get_info()
    del env
    gc.collect()
    torch.cuda.synchronize()
    free_without, _ = torch.cuda.mem_get_info()
    assert free_without - free_with > (100 << 20), (free_without - free_with) / 2 ** 20
    pair = Pair(8, 1, 1, seed=9, frameskip=8)
    rng = np.random.default_rng(12)
    for _ in range(2):
        pair.step_continuous(workloads.random_continuous_actions(rng, 8, 2))
    report = pair.state_mismatches() + pair.output_mismatches()
    pair.close()
    assert not report, report
