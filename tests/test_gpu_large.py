"""Broadcast forwards past the 32-bit index range.

The kernels index with 32-bit work items and (in the fast path) 32-bit operand offsets; larger outputs
are cut along their outermost coalesced dim into launches of at most 2^30 outputs.  Each case below
crosses 2^31 outputs or offsets in ONE call and is checked two ways:
  * against the same result computed by separate calls of at most 2^30 outputs made here, with the
    operand pointers advanced by the test (the form the configuration's chunked workload uses): every
    element, compared on the device as sum((x - y)^2) == 0 over 2^28-element slices;
  * against a + b (or the op) on the host at the first and last elements and around every 2^30-output
    boundary, so an error shared by both device paths still shows.
Cases: the configuration's full broadcast a[256,512,1,64] + b[1,1,512,64] (2^32 outputs, 16 GiB; the
reference's binary_fwd, engine/src/ops/ops_elementwise.c:108-127), an odd innermost dim with no
128-bit path ([40000,1] * [1,54001], 2,160,040,000 outputs) and a flat subtraction of 2^31 + 6
elements whose last piece is 6 elements long.  Flat operands are periodic patterns expanded on the
device (a strided copy with a zero stride), so the host never holds a whole operand.
"""

import numpy as np
import pytest

from tests.test_gpu_parity import dev, empty, sync

pytestmark = pytest.mark.gpu

SLICE = 1 << 28
PIECE = 1 << 30
WIN = 1 << 16


@pytest.fixture(scope="module")
def K():
    from newch_amd.hip import Kernels
    return Kernels()


def device_equal(K, X, Y, total, what):
    D = empty(4 * SLICE)
    SS = dev(np.zeros(1, np.float64))
    wsb = K.sumsq_workspace(SLICE)
    ws = empty(max(wsb, 8))
    for s0 in range(0, total, SLICE):
        n = min(SLICE, total - s0)
        K.binary_fwd("sub", (n,), X.ptr + 4 * s0, [1], Y.ptr + 4 * s0, [1], D.ptr, [1])
        K.sumsq(n, D.ptr, SS.ptr, s0 > 0, ws.ptr, wsb)
    sync()
    ss = SS.to_numpy(np.float64, 1)[0]
    assert ss == 0.0, f"{what}: one call and the pieces differ (sum of squared differences {ss})"


def host_windows(O, total, expect, what):
    starts = {0, max(total - WIN, 0)}
    for b in range(PIECE, total, PIECE):
        starts.update({b - WIN, b})
    for s0 in sorted(starts):
        n = min(WIN, total - s0)
        got = O.to_numpy(np.float32, n, offset=4 * s0)
        want = expect(np.arange(s0, s0 + n, dtype=np.int64))
        bad = got.view(np.uint32) != want.view(np.uint32)
        assert not bad.any(), f"{what}: element {s0 + int(np.flatnonzero(bad)[0])} differs from the host"


def test_full_config_broadcast_in_one_call(K):
    print("binary_fwd add a[256,512,1,64] + b[1,1,512,64] -> 2^32 outputs, one call", flush=True)
    rng = np.random.default_rng(3)
    a = rng.standard_normal((256, 512, 1, 64)).astype(np.float32)
    b = rng.uniform(0.5, 2.0, (1, 1, 512, 64)).astype(np.float32)
    total = 1 << 32
    A, B, O, R = dev(a), dev(b), empty(4 * total), empty(4 * total)
    K.binary_fwd("add", (256, 512, 512, 64), A.ptr, [32768, 64, 0, 1], B.ptr, [0, 0, 64, 1], O.ptr,
                 [1 << 24, 1 << 15, 64, 1])
    for k in range(4):  # the configuration's chunks: a[64k : 64k + 64] -> 2^30 outputs each
        K.binary_fwd("add", (64, 512, 512, 64), A.ptr + 4 * k * 64 * 32768, [32768, 64, 0, 1], B.ptr,
                     [0, 0, 64, 1], R.ptr + 4 * k * PIECE, [1 << 24, 1 << 15, 64, 1])
    device_equal(K, O, R, total, "full broadcast add")
    af, bf = a.ravel(), b.ravel()

    def expect(i):
        i0, i1, i2, i3 = i >> 24, (i >> 15) & 511, (i >> 6) & 511, i & 63
        return af[(i0 * 512 + i1) * 64 + i3] + bf[i2 * 64 + i3]

    host_windows(O, total, expect, "full broadcast add")


def test_odd_inner_dim_past_2_31(K):
    print("binary_fwd mul [40000,1] * [1,54001] -> 2,160,040,000 outputs, one call", flush=True)
    rng = np.random.default_rng(4)
    M, N = 40000, 54001
    a = rng.standard_normal((M, 1)).astype(np.float32)
    b = rng.standard_normal((1, N)).astype(np.float32)
    total = M * N
    assert total > 1 << 31
    A, B, O, R = dev(a), dev(b), empty(4 * total), empty(4 * total)
    K.binary_fwd("mul", (M, N), A.ptr, [1, 0], B.ptr, [0, 1], O.ptr, [N, 1])
    rows = 8000
    for r0 in range(0, M, rows):
        K.binary_fwd("mul", (rows, N), A.ptr + 4 * r0, [1, 0], B.ptr, [0, 1], R.ptr + 4 * r0 * N, [N, 1])
    device_equal(K, O, R, total, "outer product")
    af, bf = a.ravel(), b.ravel()
    host_windows(O, total, lambda i: af[i // N] * bf[i % N], "outer product")


def test_flat_same_shape_past_2_31(K):
    n = (1 << 31) + 6
    print(f"binary_fwd sub, two flat operands of {n} elements, one call", flush=True)
    rng = np.random.default_rng(5)
    pa, pb = 1_000_003, 999_983  # periods of the two operand patterns
    a_pat = rng.standard_normal(pa).astype(np.float32)
    b_pat = rng.standard_normal(pb).astype(np.float32)

    def expand(pat):
        period = pat.size
        reps = (n + period - 1) // period
        P, X = dev(pat), empty(4 * reps * period)
        K.copy_strided(4, (reps, period), P.ptr, [0, 1], X.ptr)
        return X

    A, B = expand(a_pat), expand(b_pat)
    O, R = empty(4 * n), empty(4 * n)
    K.binary_fwd("sub", (n,), A.ptr, [1], B.ptr, [1], O.ptr, [1])
    for s0 in range(0, n, SLICE):
        m = min(SLICE, n - s0)
        K.binary_fwd("sub", (m,), A.ptr + 4 * s0, [1], B.ptr + 4 * s0, [1], R.ptr + 4 * s0, [1])
    device_equal(K, O, R, n, "flat sub")
    host_windows(O, n, lambda i: a_pat[i % pa] - b_pat[i % pb], "flat sub")
