"""Results do not depend on the device's compute-unit count.

The reference guarantees bit-identical results for any thread count: elementwise chunk edges are
multiples of 16 elements and the serial reductions have one order (engine/src/runtime/threadpool.c:182-186,
tested at engine/tests/test_main.c:1169-1246).  The GPU counterpart: every split of a reduction into
partials is a function of the problem shape only, and the CU count sizes nothing but the grids of
grid-stride kernels.  nc_hip_set_grid_cus makes the kernels size their grids for another CU count (as
on a part with fewer or more CUs, or another partition mode); each case below is run at the device's
own count, at 32, 100 and 1024 CUs, and must give the same bits every time.
"""

import numpy as np
import pytest

from oracle import pyoracle as O
from tests.test_gpu_parity import assert_bits, bcast_strides, dev, empty, strides_of, sync

pytestmark = pytest.mark.gpu

GRID_CUS = [0, 32, 100, 1024]  # 0 = the device's own count


@pytest.fixture(scope="module")
def K():
    from newch_amd.hip import Kernels
    k = Kernels()
    yield k
    k.set_grid_cus(0)


def across_cus(K, run):
    """run() -> tuple of numpy arrays, once per grid size; every run must match the first bit for bit."""
    outs = []
    for n in GRID_CUS:
        K.set_grid_cus(n)
        try:
            outs.append(run())
        finally:
            K.set_grid_cus(0)
    for n, o in zip(GRID_CUS[1:], outs[1:]):
        for k, (a, b) in enumerate(zip(o, outs[0])):
            assert_bits(a, b, f"output {k} with grids for {n} CUs")
    return outs[0]


# outer, R, inner: a full sum (chunk partials), few long rows, column scans split into chunk
# partials (inner > 1, grid-stride over a fixed partial set) and many short rows
REDUCE = [(1, 1 << 22, 1), (1, 1_000_003, 1), (3, 200_000, 1), (7, 3000, 130), (2, 40_000, 3), (4096, 1024, 1)]


@pytest.mark.parametrize("outer,R,inner", REDUCE)
@pytest.mark.parametrize("kind", ["sum", "mean", "max", "argmax"])
def test_reduce_independent_of_cus(K, outer, R, inner, kind):
    rng = np.random.default_rng(outer * 31 + R + inner)
    x = (rng.standard_normal((outer, R, inner)) * 2).astype(np.float32)
    if kind in ("max", "argmax"):
        x[:, R // 2, :] = x.max(axis=1)  # ties: the first index must win on every grid
    X = dev(x)
    n = outer * inner
    wsb = K.reduce_workspace(kind, outer, R, inner)
    ws = empty(max(wsb, 8))

    def run():
        Y, A = empty(4 * n), empty(4 * n)
        K.reduce_fwd(kind, outer, R, inner, X.ptr, Y.ptr if kind != "argmax" else None,
                     A.ptr if kind in ("max", "argmax") else None, ws.ptr, wsb)
        sync()
        return (Y.to_numpy(np.float32, n) if kind != "argmax" else np.zeros(1, np.float32),
                A.to_numpy(np.int32, n) if kind in ("max", "argmax") else np.zeros(1, np.int32))

    y, a = across_cus(K, run)
    if kind in ("max", "argmax"):
        want_y, want_a = O.reduce_fwd("max", x, 1)
        assert_bits(a.reshape(outer, inner), np.asarray(want_a, np.int32).reshape(outer, inner), "argmax")


# sum-to-shape of one operand (fixed (kept index, chunk) partials), the fused one-pass backward of
# both operands (plane ranges) and its single-operand forms
def test_sum_to_shape_independent_of_cus(K):
    rng = np.random.default_rng(5)
    A = rng.standard_normal((300, 1, 64)).astype(np.float32)
    B = (0.5 + rng.random((1, 512, 64))).astype(np.float32)
    shape = (300, 512, 64)
    G = rng.standard_normal(shape).astype(np.float32)
    sa, sb = bcast_strides(A.shape, strides_of(A), shape), bcast_strides(B.shape, strides_of(B), shape)
    so = strides_of(np.empty(shape, np.float32))
    Ad, Bd, Gd = dev(A), dev(B), dev(G)
    wsb = K.binary_bwd2_workspace(shape, sa, sb)
    ws = empty(max(wsb, 8))
    for op in ("add", "mul", "div"):
        def fused():
            GA, GB = dev(np.zeros(A.shape, np.float32)), dev(np.zeros(B.shape, np.float32))
            K.binary_bwd2(op, shape, Gd.ptr, so, Ad.ptr, sa, Bd.ptr, sb, GA.ptr, sa, GB.ptr, sb, ws.ptr, wsb,
                          accumulate=False)
            sync()
            return GA.to_numpy(np.float32, A.shape), GB.to_numpy(np.float32, B.shape)

        across_cus(K, fused)

    # a reduction the fused kernel does not take: g[40, 70, 33] to b[70, 1] and a[40, 1, 33]
    a2 = rng.standard_normal((40, 1, 33)).astype(np.float32)
    b2 = (0.5 + rng.random((70, 1))).astype(np.float32)
    shape2 = (40, 70, 33)
    g2 = rng.standard_normal(shape2).astype(np.float32)
    s2a, s2b = bcast_strides(a2.shape, strides_of(a2), shape2), bcast_strides(b2.shape, strides_of(b2), shape2)
    s2o = strides_of(np.empty(shape2, np.float32))
    A2, B2, G2 = dev(a2), dev(b2), dev(g2)
    for which, xs, sx in ((0, a2.shape, s2a), (1, b2.shape, s2b)):
        wsg = K.binary_bwd_workspace(shape2, sx)
        wsG = empty(max(wsg, 8))

        def single():
            GX = dev(np.zeros(xs, np.float32))
            K.binary_bwd("div", which, shape2, G2.ptr, s2o, A2.ptr, s2a, B2.ptr, s2b, GX.ptr, sx, wsG.ptr, wsg,
                         accumulate=False)
            sync()
            return (GX.to_numpy(np.float32, xs),)

        across_cus(K, single)


@pytest.mark.parametrize("rows,D", [(4099, 1024), (1031, 512), (300, 333), (9, 5000)])
def test_layer_norm_bwd_independent_of_cus(K, rows, D):
    """gw / gb: per-workgroup row partials (register paths) or (column, row chunk) partials (generic)."""
    rng = np.random.default_rng(rows + D)
    x = rng.standard_normal((rows, D)).astype(np.float32)
    g = rng.standard_normal((rows, D)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    Xd, Wd, Gd = dev(x), dev(w), dev(g)
    Sd, Yd = empty(8 * rows), empty(x.nbytes)
    K.layer_norm_fwd(rows, D, Xd.ptr, Wd.ptr, 0, 1e-5, Yd.ptr, Sd.ptr)
    wsb = K.layer_norm_bwd_workspace(rows, D)
    ws = empty(max(wsb, 8))

    def run():
        GX, GW, GB = empty(x.nbytes), dev(np.zeros(D, np.float32)), dev(np.zeros(D, np.float32))
        K.layer_norm_bwd(rows, D, Xd.ptr, Wd.ptr, Sd.ptr, Gd.ptr, GX.ptr, GW.ptr, GB.ptr, ws.ptr, wsb,
                         accumulate=False)
        sync()
        return GX.to_numpy(np.float32, (rows, D)), GW.to_numpy(np.float32, D), GB.to_numpy(np.float32, D)

    across_cus(K, run)


@pytest.mark.parametrize("n", [1_000_003, 1 << 24])
def test_sumsq_independent_of_cus(K, n):
    x = (np.random.default_rng(n).standard_normal(n) * 3).astype(np.float32)
    X = dev(x)
    wsb = K.sumsq_workspace(n)
    ws = empty(max(wsb, 8))

    def run():
        SS = dev(np.zeros(1, np.float64))
        K.sumsq(n, X.ptr, SS.ptr, False, ws.ptr, wsb)
        sync()
        return (SS.to_numpy(np.float64, 1),)

    across_cus(K, run)


@pytest.mark.parametrize("N,C", [(65536, 1024), (1000, 7), (300, 100)])
def test_losses_independent_of_cus(K, N, C):
    rng = np.random.default_rng(N + C)
    x = (rng.standard_normal((N, C)) * 3).astype(np.float32)
    lab = rng.integers(0, C, N).astype(np.int32)
    Xd, Ld = dev(x), dev(lab)
    wsb = K.loss_workspace(N, C)
    ws = empty(max(wsb, 8))

    def run():
        S, LS, NL, BAD = empty(8 * N), empty(4), empty(4), empty(8)
        K.cross_entropy_fwd(N, C, Xd.ptr, Ld.ptr, S.ptr, LS.ptr, BAD.ptr, ws.ptr, wsb)
        K.nll_loss_fwd(N, C, Xd.ptr, Ld.ptr, False, NL.ptr, BAD.ptr, ws.ptr, wsb)
        sync()
        return LS.to_numpy(np.float32, 1), NL.to_numpy(np.float32, 1), S.to_numpy(np.float32, (N, 2))

    across_cus(K, run)


# fp32 GEMM: the tile size follows the CU count (256 x 256 tiles when they give every CU one, else
# 128 x 128 or 64 x 64), and every tile size sums an output's K products in the same order, so the
# bits do not change; shapes straddle the tile-size thresholds for 32 .. 1024 CUs, with K below and
# above the direct-to-LDS threshold and a ragged one
GEMM = [(1024, 1024, 512, 0, 1), (2048, 1536, 256, 0, 0), (512, 768, 1040, 1, 1), (3000, 1000, 300, 1, 0),
        (4096, 2048, 64, 0, 1)]


# short-K batched products of whole 256 x 256 tiles (as attention scores: B a transposed view, A
# strided or broadcast over the batch, C = alpha A B), tiles from one to several per CU over the grids,
# against fp64 too.  batch, M, N, K, alpha, A batch stride (0: broadcast)
GEMM_PT = [(24, 1280, 1280, 128, 1.0, 1), (32, 1024, 1024, 64, 1.0, 1), (1, 8192, 4096, 512, 0.5, 1),
           (20, 1024, 512, 192, 1.0, 0)]


@pytest.mark.parametrize("bc,M,N,Kd,alpha,sa", GEMM_PT)
def test_gemm_f32_short_k_batch_independent_of_cus(K, bc, M, N, Kd, alpha, sa):
    rng = np.random.default_rng(bc * 7 + M + N + Kd)
    A = rng.standard_normal((max(bc * sa, 1), M, Kd)).astype(np.float32)
    B = rng.standard_normal((bc, N, Kd)).astype(np.float32)  # used transposed
    Ad, Bd = dev(A), dev(B)
    print(f"short-K GEMM batch {bc} {M}x{N}x{Kd}", flush=True)

    def run():
        C = empty(4 * bc * M * N)
        if bc == 1:
            K.gemm_f32(0, 1, M, N, Kd, alpha, Ad.ptr, Kd, Bd.ptr, Kd, 0.0, C.ptr, N)
        else:
            K.gemm_f32_bmm(0, 1, M, N, Kd, Ad.ptr, Kd, Bd.ptr, Kd, 0.0, C.ptr, N, (bc,), (sa * M * Kd,), (N * Kd,),
                           (M * N,))
        sync()
        return (C.to_numpy(np.float32, (bc, M, N)),)

    out = across_cus(K, run)[0]
    for b in (0, bc - 1):
        rows = np.arange(0, M, 97)
        a = A[b * sa][rows].astype(np.float64)
        want = alpha * (a @ B[b].T.astype(np.float64))
        terms = abs(alpha) * (np.abs(a) @ np.abs(B[b].T).astype(np.float64))
        assert O.gemm_excess(out[b][rows], want, terms, Kd) <= 1.0, f"batch {b}"


@pytest.mark.parametrize("M,N,Kd,ta,tb", GEMM)
def test_gemm_f32_independent_of_cus(K, M, N, Kd, ta, tb):
    rng = np.random.default_rng(M + N + Kd)
    A = rng.standard_normal((Kd, M) if ta else (M, Kd)).astype(np.float32)
    B = rng.standard_normal((N, Kd) if tb else (Kd, N)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    Ad, Bd = dev(A), dev(B)

    def run():
        Cd = dev(C0)
        K.gemm_f32(ta, tb, M, N, Kd, 0.5, Ad.ptr, A.shape[1], Bd.ptr, B.shape[1], 1.0, Cd.ptr, N)
        sync()
        return (Cd.to_numpy(np.float32, (M, N)),)

    across_cus(K, run)
