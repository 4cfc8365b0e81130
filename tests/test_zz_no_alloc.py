"""nc_hip_reduce_fwd_noalloc, the reduction entry point that allocates nothing (called through the
C ABI), against nc_hip_reduce_fwd with a caller's workspace: the same bits for every kind and plan (a
full sum split into chunk partials, few long rows, column scans with chunk partials, short rows with
no partials), two calls in a row on the shared scratch, the second on a smaller input; the device's
free memory is unchanged across calls that need partials."""

import ctypes
from ctypes import c_int, c_int64, c_void_p

import numpy as np
import pytest

from newch_amd import abi
from tests.test_gpu_parity import assert_bits, dev, empty, sync

pytestmark = pytest.mark.gpu

# (outer, R, inner) pairs: the first call, then a smaller one of the same plan kind
PAIRS = [((1, 1 << 22, 1), (1, 100_003, 1)),       # full sums: chunk partials, then fewer of them
         ((3, 300_000, 1), (2, 9_000, 1)),          # few long rows
         ((7, 3000, 130), (2, 500, 40)),            # column scans split into chunk partials
         ((4096, 1024, 1), (100, 64, 1))]           # one wave per row, no partials


@pytest.fixture(scope="module")
def libs():
    lib = ctypes.CDLL(str(abi.LIB_PATH))
    fn = lib.nc_hip_reduce_fwd_noalloc
    fn.restype = c_int
    fn.argtypes = [c_int, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p]
    lib.nc_hip_last_error.restype = ctypes.c_char_p
    from newch_amd.hip import RED, Kernels
    return lib, Kernels(), RED


@pytest.mark.parametrize("kind", ["sum", "mean", "max", "argmax"])
def test_reduce_noalloc_matches_workspace_entry(libs, kind):
    lib, K, RED = libs
    for shape in PAIRS:
        for outer, R, inner in shape:
            print(f"reduce_fwd_noalloc {kind} outer={outer} R={R} inner={inner}", flush=True)
            rng = np.random.default_rng(outer + R + inner)
            x = (rng.standard_normal((outer, R, inner)) * 2).astype(np.float32)
            x[:, R // 3, :] = x.max(axis=1)  # ties for max / argmax
            X = dev(x)
            n = outer * inner
            want_y = kind != "argmax"
            want_a = kind in ("max", "argmax")
            Y1, A1, Y2, A2 = empty(4 * n), empty(4 * n), empty(4 * n), empty(4 * n)
            rc = lib.nc_hip_reduce_fwd_noalloc(RED[kind], outer, R, inner, X.ptr, Y1.ptr if want_y else None,
                                               A1.ptr if want_a else None, None)
            assert rc == 0, lib.nc_hip_last_error().decode()
            wsb = K.reduce_workspace(kind, outer, R, inner)
            ws = empty(max(wsb, 8))
            K.reduce_fwd(kind, outer, R, inner, X.ptr, Y2.ptr if want_y else None, A2.ptr if want_a else None,
                         ws.ptr, wsb)
            sync()
            if want_y:
                assert_bits(Y1.to_numpy(np.float32, n), Y2.to_numpy(np.float32, n), f"{kind} values")
            if want_a:
                assert_bits(A1.to_numpy(np.int32, n), A2.to_numpy(np.int32, n), f"{kind} indices")


def test_reduce_noalloc_takes_no_device_memory(libs):
    """After a first call (which looks up the scratch address), calls that need partials leave the
    device's free memory as it was: the partials live in the static scratch."""
    from newch_amd import hipmem as hm
    lib, K, RED = libs
    outer, R, inner = 7, 3000, 130  # column scans with chunk partials
    print(f"reduce_fwd_noalloc sum outer={outer} R={R} inner={inner}: free memory around 5 calls", flush=True)
    assert K.reduce_workspace("sum", outer, R, inner) > 0
    x = np.random.default_rng(5).standard_normal((outer, R, inner)).astype(np.float32)
    X, Y = dev(x), empty(4 * outer * inner)
    assert lib.nc_hip_reduce_fwd_noalloc(RED["sum"], outer, R, inner, X.ptr, Y.ptr, None, None) == 0
    sync()
    free0, _ = hm.mem_info()
    for _ in range(5):
        rc = lib.nc_hip_reduce_fwd_noalloc(RED["sum"], outer, R, inner, X.ptr, Y.ptr, None, None)
        assert rc == 0, lib.nc_hip_last_error().decode()
    sync()
    free1, _ = hm.mem_info()
    assert free1 == free0, (free0, free1)
