"""The run split of 2^32-element problems, driven at small sizes.

Broadcast gradients (nc_hip_binary_bwd / nc_hip_binary_bwd2, the reference's binary_bwd,
engine/src/ops/ops_elementwise.c:129-186), the sum / mean gradient (nc_hip_reduce_bwd, reduce_bwd,
engine/src/ops/ops_reduce.c:118-163) and the strided copy and scatter-add (nc_hip_copy_strided,
nc_hip_accumulate_strided) run problems of 2^32 elements or more as runs of at most 2^30
(kernels/common.hpp for_each_run): one launch per run, each operand advanced to the run's first
element, and an output that later runs add into taking the caller's accumulate flag in its first run
only.  The test hook NC_HIP_RUN_LIMIT=n lowers both the threshold and the run size to n, so the same
code runs here on problems of a few thousand elements, with limits that cut the outermost dim, an
inner dim and the innermost dim.  Checks: against the same call without the split, bit for bit,
wherever no run adds into another run's output (unreduced gradients, the broadcast-back, copies), and
against fp64 sums where runs add rounded partial sums of a reduced gradient in turn.
"""

import numpy as np
import pytest

from oracle import pyoracle as O
from tests.test_gpu_parity import (_random_bcast_case, assert_bits, assert_close64, bcast_strides, dev, empty,
                                   grad_terms64, strides_of, sum_to, sync)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    from newch_amd.hip import Kernels
    return Kernels()


def limits_for(shape):
    """Run limits that cut the outermost dim, a middle dim and the innermost dim of `shape`, kept to
    at most ~64 runs."""
    n = int(np.prod(shape))
    out = {max(1, n // 3 + 1)}
    inner = 1
    for d in reversed(shape[1:]):
        inner *= d
        if 1 < inner < n and n // max(inner // 2, 1) <= 64:
            out.add(max(1, inner // 2 + 1))
    out.add(max(1, n // 64 + 1))
    return sorted(v for v in out if 0 < v < n)


def _grads(K, op, out_shape, Gd, so, Ad, sa, Bd, sb, shapes, sgs, inits, accumulate):
    """per-operand and fused gradients of the binary op, from the given initial gradient buffers"""
    got1 = []
    for which in (0, 1):
        GX = dev(inits[which])
        wsb = K.binary_bwd_workspace(out_shape, sgs[which])
        ws = empty(max(wsb, 1))
        K.binary_bwd(op, which, out_shape, Gd.ptr, so, Ad.ptr, sa, Bd.ptr, sb, GX.ptr, sgs[which], ws.ptr, wsb,
                     accumulate=accumulate)
        sync()
        got1.append(GX.to_numpy(np.float32, shapes[which]))
    GA, GB = dev(inits[0]), dev(inits[1])
    wsb = K.binary_bwd2_workspace(out_shape, sgs[0], sgs[1])
    ws = empty(max(wsb, 1))
    K.binary_bwd2(op, out_shape, Gd.ptr, so, Ad.ptr, sa, Bd.ptr, sb, GA.ptr, sgs[0], GB.ptr, sgs[1], ws.ptr, wsb,
                  accumulate=accumulate)
    sync()
    return got1, [GA.to_numpy(np.float32, shapes[0]), GB.to_numpy(np.float32, shapes[1])]


@pytest.mark.parametrize("seed", range(24))
def test_binary_grads_in_runs(K, monkeypatch, seed):
    out_shape, ash, bsh, perm = _random_bcast_case(4000 + seed)
    if int(np.prod(out_shape)) < 4:
        pytest.skip("too small to split")
    rng = np.random.default_rng(7000 + seed)
    if perm is None:
        A = rng.standard_normal(ash).astype(np.float32)
        a = A
    else:
        inv = np.argsort(perm)
        A = np.ascontiguousarray(rng.standard_normal(ash).astype(np.float32).transpose(perm))
        a = A.transpose(inv)
    B = (0.5 + 1.5 * rng.random(bsh)).astype(np.float32)
    out_shape = tuple(O.broadcast_shape(a.shape, B.shape))
    sa = bcast_strides(a.shape, strides_of(a), out_shape)
    sb = bcast_strides(B.shape, strides_of(B), out_shape)
    so = [s // 4 for s in np.empty(out_shape, np.float32).strides]
    sgs = [bcast_strides(x.shape, [s // 4 for s in np.empty(x.shape, np.float32).strides], out_shape) for x in (a, B)]
    G = rng.standard_normal(out_shape).astype(np.float32)
    Ad, Bd, Gd = dev(A), dev(B), dev(G)
    shapes = (a.shape, B.shape)
    for op in ("add", "mul", "div"):
        ta, tb = grad_terms64(op, a, B, G)
        for accumulate in (True, False):
            inits = [rng.standard_normal(a.shape).astype(np.float32), rng.standard_normal(B.shape).astype(np.float32)]
            monkeypatch.delenv("NC_HIP_RUN_LIMIT", raising=False)
            whole1, whole2 = _grads(K, op, out_shape, Gd, so, Ad, sa, Bd, sb, shapes, sgs, inits, accumulate)
            for lim in limits_for(out_shape):
                monkeypatch.setenv("NC_HIP_RUN_LIMIT", str(lim))
                got1, got2 = _grads(K, op, out_shape, Gd, so, Ad, sa, Bd, sb, shapes, sgs, inits, accumulate)
                what = f"seed {seed} {op} acc {accumulate} out {out_shape} a {ash} perm {perm} b {bsh} runs of {lim}"
                for which, (x, t) in enumerate(((a, ta), (B, tb))):
                    init = inits[which].astype(np.float64) if accumulate else 0.0
                    if tuple(x.shape) == tuple(out_shape):
                        assert_bits(got1[which], whole1[which], f"{what} grad {which}")
                        assert_bits(got2[which], whole2[which], f"{what} fused grad {which}")
                    else:
                        red = sum_to(t, x.shape).reshape(x.shape)
                        terms = max(t.size // max(red.size, 1), 1)
                        scale = sum_to(np.abs(t), x.shape).reshape(x.shape) / np.sqrt(terms)
                        scale = scale + (np.abs(inits[which]) if accumulate else 0.0)
                        assert_close64(got1[which], init + red, scale, f"{what} grad {which}")
                        assert_close64(got2[which], init + red, scale, f"{what} fused grad {which}")
            monkeypatch.delenv("NC_HIP_RUN_LIMIT", raising=False)


@pytest.mark.parametrize("kind", ["sum", "mean"])
@pytest.mark.parametrize("outer,R,inner", [(7, 300, 33), (1, 5000, 3), (40, 1, 129), (3, 17, 1000)])
def test_reduce_bwd_in_runs(K, monkeypatch, kind, outer, R, inner):
    rng = np.random.default_rng(outer * 7 + R + inner)
    g = rng.standard_normal((outer, inner)).astype(np.float32)
    gi0 = rng.standard_normal((outer, R, inner)).astype(np.float32)
    Gd = dev(g)
    n = outer * R * inner
    for accumulate in (True, False):
        monkeypatch.delenv("NC_HIP_RUN_LIMIT", raising=False)
        GI = dev(gi0)
        K.reduce_bwd(kind, outer, R, inner, Gd.ptr, None, GI.ptr, accumulate=accumulate)
        sync()
        whole = GI.to_numpy(np.float32, (outer, R, inner))
        want = O.reduce_bwd(kind, (outer, R, inner), 1, g, None, gi0 if accumulate else None)
        assert_bits(whole, want, f"{kind} {outer},{R},{inner} acc {accumulate} whole")
        for lim in limits_for((outer, R, inner)) + [inner * R + 1, max(inner // 3, 1)]:
            if not 0 < lim < n or n // lim > 4096:
                continue
            monkeypatch.setenv("NC_HIP_RUN_LIMIT", str(lim))
            GI = dev(gi0)
            K.reduce_bwd(kind, outer, R, inner, Gd.ptr, None, GI.ptr, accumulate=accumulate)
            sync()
            assert_bits(GI.to_numpy(np.float32, (outer, R, inner)), whole,
                        f"{kind} {outer},{R},{inner} acc {accumulate} runs of {lim}")
        monkeypatch.delenv("NC_HIP_RUN_LIMIT", raising=False)


@pytest.mark.parametrize("shape,perm", [((6, 50, 40), (2, 0, 1)), ((300, 7), (1, 0)), ((4, 5, 6, 7), (3, 1, 0, 2)),
                                        ((2, 3000), None)])
def test_strided_copy_and_scatter_add_in_runs(K, monkeypatch, shape, perm):
    """copy_strided gathers a view stored in permuted order; accumulate_strided adds contiguous values
    into such a view: one call against the pieces the split makes, bit for bit."""
    from newch_amd.hip import _i64
    rng = np.random.default_rng(int(np.prod(shape)))
    perm = perm or tuple(range(len(shape)))
    inv = tuple(np.argsort(perm))
    pshape = tuple(shape[p] for p in perm)
    src_store = rng.standard_normal(pshape).astype(np.float32)   # storage, permuted order
    src = src_store.transpose(inv)                                # the logical view, shape `shape`
    dst_store0 = rng.standard_normal(pshape).astype(np.float32)
    vals = rng.standard_normal(shape).astype(np.float32)          # contiguous over `shape`
    S, V = dev(src_store), dev(vals)
    ss = strides_of(src)
    sd = strides_of(dst_store0.transpose(inv))
    n = int(np.prod(shape))
    for lim in [None] + limits_for(shape):
        if lim is None:
            monkeypatch.delenv("NC_HIP_RUN_LIMIT", raising=False)
        else:
            monkeypatch.setenv("NC_HIP_RUN_LIMIT", str(lim))
        what = f"{shape} perm {perm} runs of {lim}"
        D = empty(4 * n)
        K.copy_strided(4, shape, S.ptr, ss, D.ptr)
        sync()
        assert_bits(D.to_numpy(np.float32, shape), np.ascontiguousarray(src), what + " copy")
        Dst = dev(dst_store0)
        rc = K.lib.nc_hip_accumulate_strided(len(shape), _i64(shape), V.ptr, Dst.ptr, _i64(sd), None)
        assert rc == 0, what
        sync()
        got = Dst.to_numpy(np.float32, pshape).transpose(inv)
        want = (dst_store0.transpose(inv) + vals).astype(np.float32)
        assert_bits(np.ascontiguousarray(got), np.ascontiguousarray(want), what + " scatter-add")
    monkeypatch.delenv("NC_HIP_RUN_LIMIT", raising=False)
