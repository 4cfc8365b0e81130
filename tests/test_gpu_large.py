"""Broadcasts, their gradients and strided copies past the 32-bit index range.

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

The configuration's full-shape backward (2^32-element gradient, the reference's binary_bwd,
engine/src/ops/ops_elementwise.c:129-186, and reduce_bwd, engine/src/ops/ops_reduce.c:118-163) is
checked at the kernel layer -- one call against the four 2^30-element chunk calls, bit for bit, and
against the fp64 sums -- and through nc.h: forward, sum and nc_backward over 2^32 outputs.
"""

import numpy as np
import pytest

from newch_amd import abi
from tests.ncdrive import Engine
from tests.test_gpu_parity import assert_bits, assert_close64, dev, empty, sync

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


FULL = (256, 512, 512, 64)
S_G = [1 << 24, 1 << 15, 64, 1]
S_A = [32768, 64, 0, 1]  # a[256,512,1,64] over the output
S_B = [0, 0, 64, 1]      # b[1,1,512,64]


def _config_inputs(seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((256, 512, 1, 64)).astype(np.float32)
    b = rng.uniform(0.5, 2.0, (1, 1, 512, 64)).astype(np.float32)
    g1 = rng.standard_normal((512, 512, 64)).astype(np.float32)  # g[p0] = g1 for every p0
    return a, b, g1


def _truth(op, a, b, g1):
    """fp64 sums of the gradient terms for g[p0, p1, h, w] = g1[p1, h, w]: grad_a (the same for every
    p0) and grad_b, with the magnitudes of their terms."""
    G = g1.astype(np.float64)
    a64 = a[:, :, 0, :].astype(np.float64)  # [256, 512, 64]
    b64 = b[0, 0].astype(np.float64)        # [512, 64]
    if op == "add":
        ga, ta = G.sum(axis=1), np.abs(G).sum(axis=1)
        gb, tb = 256 * G.sum(axis=0), 256 * np.abs(G).sum(axis=0)
    else:  # mul: grad_a = sum_h g b, grad_b = sum_{p0, p1} g a
        ga, ta = (G * b64).sum(axis=1), (np.abs(G) * b64).sum(axis=1)
        A1, A1abs = a64.sum(axis=0), np.abs(a64).sum(axis=0)  # [512, 64]
        gb = np.einsum("phw,pw->hw", G, A1)
        tb = np.einsum("phw,pw->hw", np.abs(G), A1abs)
    return ga, ta, gb, tb


@pytest.mark.parametrize("op", ["add", "mul"])
def test_full_config_backward_in_one_call(K, op):
    """nc_hip_binary_bwd2 over the configuration's full g[256,512,512,64] (2^32 elements) in one call:
    grad_a and grad_b bit-equal to the four 2^30-element chunk calls (grad_a written by each, grad_b
    stored by the first and added to by the others), and within the reductions' bar of fp64."""
    print(f"binary_bwd2 {op}: g[256,512,512,64] -> grad a[256,512,1,64], grad b[1,1,512,64], one call", flush=True)
    a, b, g1 = _config_inputs(6)
    total = 1 << 32
    A, B, G1 = dev(a), dev(b), dev(g1)
    G = empty(4 * total)
    K.copy_strided(4, (256, 1 << 24), G1.ptr, [0, 1], G.ptr)  # a 2^32-element gather in one call
    nws = K.binary_bwd2_workspace(FULL, S_A, S_B)
    WS = empty(max(nws, 8))
    GA, GB = empty(4 * a.size), empty(4 * b.size)
    K.binary_bwd2(op, FULL, G.ptr, S_G, A.ptr, S_A, B.ptr, S_B, GA.ptr, S_A, GB.ptr, S_B, WS.ptr, nws,
                  accumulate=False)
    # the chunk calls take one accumulate flag for both gradients: grad_a accumulates into zeros
    # (0 + x is x) so that grad_b can be stored by the first chunk and added to by the others
    GA2, GB2 = dev(np.zeros(a.size, np.float32)), empty(4 * b.size)
    chunk = (64, 512, 512, 64)
    for k in range(4):
        nk = K.binary_bwd2_workspace(chunk, S_A, S_B)
        assert nk <= nws
        K.binary_bwd2(op, chunk, G.ptr + 4 * k * PIECE, S_G, A.ptr + 4 * k * 64 * 32768, S_A, B.ptr, S_B,
                      GA2.ptr + 4 * k * 64 * 32768, S_A, GB2.ptr, S_B, WS.ptr, nk, accumulate=k > 0)
    sync()
    ga, gb = GA.to_numpy(np.float32, a.shape), GB.to_numpy(np.float32, b.shape)
    assert_bits(ga, GA2.to_numpy(np.float32, a.shape), "grad_a: one call vs four chunks")
    assert_bits(gb, GB2.to_numpy(np.float32, b.shape), "grad_b: one call vs four chunks")
    ga64, ta, gb64, tb = _truth(op, a, b, g1)
    for p0 in (0, 63, 64, 127, 128, 255):
        assert_close64(ga[p0, :, 0, :], ga64, ta, f"grad_a[{p0}]")
    assert_close64(gb[0, 0], gb64, tb, "grad_b")


def test_full_config_backward_through_engine():
    """The configuration's full broadcast through nc.h: y = a + b over 2^32 outputs, loss =
    sum(y * g1) with g1[1,512,512,64], nc_backward.  The backward walks a 2^32-element sum gradient,
    a 2^32-element unreduced mul gradient and the fused add gradient; grad a and grad b are checked
    against the fp64 sums."""
    print("engine: a[256,512,1,64] + b[1,1,512,64] -> 2^32 outputs, sum(y * g1), nc_backward", flush=True)
    a, b, g1 = _config_inputs(7)
    with Engine(lib=abi.load(abi.LIB_PATH)) as eng:
        L = eng.lib
        pa, pb = eng.param(a), eng.param(b)
        y = L.nc_add(pa, pb)
        eng.check()
        assert eng.shape(y) == FULL
        loss = L.nc_sum(L.nc_mul(y, eng.tensor(g1.reshape(1, 512, 512, 64))), abi.ALL_AXES, 0)
        eng.check()
        assert L.nc_backward(loss) == 0, L.nc_error(eng.ctx)
        ga, gb = eng.grad(pa), eng.grad(pb)
        ga64, ta, gb64, tb = _truth("add", a, b, g1)
        for p0 in (0, 63, 64, 127, 128, 255):
            assert_close64(ga[p0, :, 0, :], ga64, ta, f"grad_a[{p0}]")
        assert_close64(gb[0, 0], gb64, tb, "grad_b")
        eng.step_end()
