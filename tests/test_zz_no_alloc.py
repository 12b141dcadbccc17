"""carl_exclusive_scan_i32_noalloc, the scan that allocates nothing, against
carl_exclusive_scan_i32 through the C-ABI: bit-equal results on two calls in
a row on one stream (the second one shorter, so it runs over the first
call's leftover tile sums), the known answer of tests/direct_controls.cu:15-33,
the maximum length, and the rejection of longer inputs."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

MAX_ITEMS = 1 << 26


@pytest.fixture(scope="module")
def lib():
    from carl_amd import build

    L = ctypes.CDLL(str(build.engine_path()))
    for name in ("carl_exclusive_scan_i32", "carl_exclusive_scan_i32_noalloc"):
        getattr(L, name).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    L.carl_last_error.restype = ctypes.c_char_p
    return L


def _scan_both(lib, x: np.ndarray, stream: torch.cuda.Stream) -> tuple[np.ndarray, np.ndarray]:
    src = torch.from_numpy(x).to("cuda:0")
    a = torch.full_like(src, -7)
    b = torch.full_like(src, -9)
    torch.cuda.synchronize()
    h = ctypes.c_void_p(stream.cuda_stream)
    assert lib.carl_exclusive_scan_i32(src.data_ptr(), a.data_ptr(), len(x), h) == 0, lib.carl_last_error()
    assert lib.carl_exclusive_scan_i32_noalloc(src.data_ptr(), b.data_ptr(), len(x), h) == 0, lib.carl_last_error()
    stream.synchronize()
    return a.cpu().numpy(), b.cpu().numpy()


@pytest.mark.parametrize("sizes", [(3_000_000, 100_000), (MAX_ITEMS, 4_194_305), (2049, 4)])
def test_noalloc_scan_matches_the_allocating_scan_twice(gpu, lib, sizes):
    rng = np.random.default_rng(sizes[0] % 1000)
    stream = torch.cuda.Stream()
    for n in sizes:
        x = rng.integers(0, 30, n).astype(np.int32)
        a, b = _scan_both(lib, x, stream)
        np.testing.assert_array_equal(b, a, err_msg=f"n={n}")
        expect = np.concatenate([[0], np.cumsum(x[:-1], dtype=np.int64)]).astype(np.int32)
        np.testing.assert_array_equal(b, expect, err_msg=f"n={n}")


def test_noalloc_scan_known_answer(gpu, lib):
    a, b = _scan_both(lib, np.array([3, 1, 4, 2], np.int32), torch.cuda.Stream())
    assert b.tolist() == [0, 3, 4, 8] and a.tolist() == [0, 3, 4, 8]


def test_noalloc_scan_rejects_more_than_the_maximum(gpu, lib):
    src = torch.zeros(4, dtype=torch.int32, device="cuda:0")
    rc = lib.carl_exclusive_scan_i32_noalloc(src.data_ptr(), src.data_ptr(), MAX_ITEMS + 1, None)
    assert rc == -1
    assert b"no-allocation maximum" in lib.carl_last_error()
    assert lib.carl_exclusive_scan_i32_noalloc(src.data_ptr(), src.data_ptr(), 0, None) == 0
