"""Random chains of hot-path ops through both engines' nc.h API, compared with each other.

A seeded plan of 3-7 ops (activations, broadcast binary ops against parameters, a tensor combined with
itself (t op t) or with an activation of itself (t + f(t)), so that its gradient receives two terms,
sqrt / log / pow of t * t + 0.5, exp of tanh(t), strided slices,
sum / mean / max over an axis with or without keepdim, softmax / log_softmax, LayerNorm with weight and
bias, transposed and reshaped views, matmul and linear with parameters, and sometimes a cross-entropy,
nll or mse loss head) is built from a parameter x, the same plan runs in this
engine (tests/ncdrive.Engine over newch_amd/libnc.so, on the GPU) and in the reference engine compiled
from its sources (oracle/_ref/libnc_ref.so, on the CPU), then loss = sum(out * G) goes backward in
both.  The output and every parameter's gradient are compared: bit for bit when every op of the chain
is one whose result does not depend on a summation order (activations, same-shape binary ops and
their gradients, views, max), otherwise within 2e-4 of the tensor's largest magnitude or 2e-5 of the
chain's largest result, whichever is larger (these chains contain fp64-vs-fp32 reductions and fp32
GEMMs whose orders differ by design; the bar catches a wrong index, operand, axis or gradient path,
not last-bit differences, which the per-op parity tests pin).
This is the reference's Python-layer usage (newch/tensor.py over newch/_lib.py) replayed on both.
"""

import ctypes
from ctypes import c_float

import numpy as np
import pytest

from newch_amd import abi
from oracle import pyoracle as O
from tests.ncdrive import Engine
from tests.test_gpu_parity import SWEEP

pytestmark = pytest.mark.gpu

UNARY = ["relu", "relu6", "leaky_relu", "hardsigmoid", "hardswish", "silu", "gelu", "gelu_tanh", "sigmoid", "tanh",
         "neg", "scale", "add_scalar"]
BINARY = ["add", "sub", "mul", "div"]


@pytest.fixture(scope="module")
def engines():
    if not O.REF_LIB.exists():
        pytest.skip("oracle/_ref/libnc_ref.so is not built (make -C oracle ref)")
    gpu, cpu = Engine(), Engine(O.REF_LIB)
    yield gpu, cpu
    gpu.close()
    cpu.close()


def make_plan(seed, exact_only=False):
    """(x shape, [ops], exact, output shape): each op a tuple whose first element names it; shapes
    tracked here.  exact_only: only ops whose results do not depend on a summation order (binary ops
    against a parameter of the full shape, max as the only reduction)."""
    rng = np.random.default_rng(seed + (50_000 if exact_only else 0))
    while True:
        shape = [int(rng.choice([2, 3, 5, 8, 13, 32])) for _ in range(int(rng.integers(2, 5)))]
        if np.prod(shape) <= 6000:
            break
    x_shape = tuple(shape)
    ops, exact = [], True
    for _ in range(int(rng.integers(3, 8))):
        nd = len(shape)
        kinds = ["unary", "binary", "binary", "transpose", "self", "residual", "positive", "slice", "bounded_exp"]
        if nd >= 2:
            kinds += ["reduce", "reshape"]
        if shape[-1] >= 8 and not exact_only:
            kinds += ["softmax", "layer_norm"]
        if nd >= 2 and np.prod(shape) <= 4096 and not exact_only:
            kinds += ["matmul", "linear"]
        k = str(rng.choice(kinds))
        if k == "unary":
            ops.append(("unary", str(rng.choice(UNARY)), float(rng.choice([0.01, 0.2]))))
        elif k == "binary":
            lead = 0 if exact_only else int(rng.integers(0, nd))
            bshape = tuple(d if exact_only or rng.random() >= 0.4 else 1 for d in shape[lead:])
            ops.append(("binary", str(rng.choice(BINARY)), bshape))
            if tuple(bshape) != tuple(shape):
                exact = False  # the broadcast operand's gradient is a reduction
        elif k == "self":  # both operands the same tensor: its gradient receives both terms (not t - t,
            # whose exact zeros make a later LayerNorm's rows constant: rstd = eps^-1/2 then magnifies
            # the rounding noise of gradients the chain is invariant to past any fixed bar)
            ops.append(("self", str(rng.choice(["add", "mul"]))))
        elif k == "positive":  # f(t * t + 0.5) for the functions that need a positive argument
            f = str(rng.choice(["sqrt"] if exact_only else ["sqrt", "log", "pow"]))
            ops.append(("positive", f, 1.5))
            if f != "sqrt":
                exact = False  # log and pow: the host libm is off by an ulp on ~0.05% of inputs
        elif k == "slice":  # a strided view along one axis: its gradient scatters into the base
            axis = int(rng.integers(0, nd))
            dim = shape[axis]
            step = int(rng.choice([1, 2, 3])) if dim > 2 else 1
            start = int(rng.integers(0, dim))
            length = int(rng.integers(1, (dim - 1 - start) // step + 2))
            ops.append(("slice", axis, start, length, step))
            shape[axis] = length
        elif k == "bounded_exp":  # exp(tanh(t)): the reference's exp replica on a bounded argument
            ops.append(("bounded_exp",))
        elif k == "residual":  # t + f(t): the gradient reaches t along two paths
            ops.append(("residual", str(rng.choice(UNARY)), float(rng.choice([0.01, 0.2]))))
        elif k == "transpose":
            if nd < 2:
                continue
            a0, a1 = (int(v) for v in rng.choice(nd, 2, replace=False))
            ops.append(("transpose", a0, a1))
            shape[a0], shape[a1] = shape[a1], shape[a0]
        elif k == "reshape":
            ops.append(("reshape", tuple(shape[:-2]) + (shape[-2] * shape[-1],)))
            shape = shape[:-2] + [shape[-2] * shape[-1]]
        elif k == "reduce":
            kind = "max" if exact_only else str(rng.choice(["sum", "mean", "max"]))
            axis, keep = int(rng.integers(0, nd)), int(rng.integers(0, 2))
            if kind != "max" and axis == nd - 1 and ops and ops[-1] == ("softmax", False):
                kind = "max"  # a sum of softmax over its own axis is constant: every gradient ~0
            ops.append(("reduce", kind, axis, keep))
            shape = shape[:axis] + ([1] if keep else []) + shape[axis + 1:]
            if kind != "max":
                exact = False
        elif k == "softmax":
            ops.append(("softmax", bool(rng.integers(0, 2))))
            exact = False
        elif k == "layer_norm":
            ops.append(("layer_norm", shape[-1]))
            exact = False
        elif k in ("matmul", "linear"):
            n_out = int(rng.choice([3, 8, 17]))
            ops.append((k, shape[-1], n_out))
            shape = shape[:-1] + [n_out]
            exact = False
    if not exact_only and rng.random() < 0.3:
        # a loss head over rows of the last dim: cross entropy, or nll over log_softmax
        C = shape[-1]
        if C >= 2:
            ops.append(("loss", bool(rng.integers(0, 2)), int(np.prod(shape[:-1])), C))
            shape = []
            exact = False
    elif not exact_only and rng.random() < 0.15:
        ops.append(("mse", tuple(shape)))  # mse_loss against a fixed target of the same shape
        shape = []
        exact = False
    return x_shape, ops, exact, tuple(shape)


def run_plan(e, seed, x_shape, ops):
    """Builds the plan's parameters from the seed, runs it forward and backward in engine e:
    (output, [parameter gradients])."""
    L = e.lib
    rng = np.random.default_rng(10_000 + seed)
    logits_max = 0.0
    params = [e.param(rng.standard_normal(x_shape).astype(np.float32))]
    t = params[0]
    for op in ops:
        if op[0] == "unary":
            t = Engine.UNARY_CALLS[op[1]](L, t, op[2])
        elif op[0] == "binary":
            vals = rng.standard_normal(op[2]).astype(np.float32)
            if op[1] == "div":
                vals = (0.5 + 1.5 * rng.random(op[2])).astype(np.float32)
            p = e.param(vals)
            params.append(p)
            t = {"add": L.nc_add, "sub": L.nc_sub, "mul": L.nc_mul, "div": L.nc_div}[op[1]](t, p)
        elif op[0] == "self":
            t = {"add": L.nc_add, "sub": L.nc_sub, "mul": L.nc_mul}[op[1]](t, t)
        elif op[0] == "positive":
            t = Engine.UNARY_CALLS[op[1]](L, L.nc_add_scalar(L.nc_mul(t, t), c_float(0.5)), op[2])
        elif op[0] == "residual":
            t = L.nc_add(t, Engine.UNARY_CALLS[op[1]](L, t, op[2]))
        elif op[0] == "transpose":
            t = L.nc_transpose(t, op[1], op[2])
        elif op[0] == "slice":
            t = L.nc_slice(t, op[1], op[2], op[3], op[4])
        elif op[0] == "bounded_exp":
            t = L.nc_exp(L.nc_tanh(t))
        elif op[0] == "mse":
            t = L.nc_mse_loss(t, e.tensor(rng.standard_normal(op[1]).astype(np.float32)))
        elif op[0] == "reshape":
            nd, shp = abi.shape_arg(op[1])
            t = L.nc_reshape(t, nd, shp)
        elif op[0] == "reduce":
            t = {"sum": L.nc_sum, "mean": L.nc_mean, "max": L.nc_max}[op[1]](t, op[2], op[3])
        elif op[0] == "softmax":
            t = L.nc_log_softmax(t) if op[1] else L.nc_softmax(t)
        elif op[0] == "layer_norm":
            w = e.param((1 + 0.1 * rng.standard_normal(op[1])).astype(np.float32))
            b = e.param((0.1 * rng.standard_normal(op[1])).astype(np.float32))
            params += [w, b]
            t = L.nc_layer_norm(t, 1, w, b, c_float(1e-5))
        elif op[0] == "matmul":
            W = e.param((rng.standard_normal((op[1], op[2])) / np.sqrt(op[1])).astype(np.float32))
            params.append(W)
            t = L.nc_matmul(t, W)
        elif op[0] == "linear":
            W = e.param((rng.standard_normal((op[2], op[1])) / np.sqrt(op[1])).astype(np.float32))
            bias = e.param((0.1 * rng.standard_normal(op[2])).astype(np.float32))
            params += [W, bias]
            t = L.nc_linear_fn(t, W, bias)
        elif op[0] == "loss":
            rows, C = op[2], op[3]
            nd, shp = abi.shape_arg((rows, C))
            t2 = L.nc_reshape(t, nd, shp)
            logits_max = float(np.abs(e.read(t2)).max(initial=0.0))
            lab = e.tensor(rng.integers(0, C, rows).astype(np.int32))
            t = L.nc_cross_entropy(t2, lab) if op[1] else L.nc_nll_loss(L.nc_log_softmax(t2), lab, 0)
        e.check()
    out = e.read(t)
    G = rng.standard_normal(out.shape).astype(np.float32)
    e.backward_with(t, G)
    grads = [e.grad(p) for p in params]
    e.step_end()
    return out, grads, logits_max


def _same(got, want, exact, what, chain_scale, loss_floor=0.0):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    if exact:
        ok = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
        assert ok.all(), f"{what}: {int((~ok).sum())} of {ok.size} differ (exact chain)"
        return
    # 2e-4 of the tensor's own largest magnitude, and never less than 2e-5 of the chain's largest
    # result: a parameter the chain is invariant to (a shift or scale ahead of a normalisation over
    # the dims it is constant along) has a true gradient of ~0, and both engines return rounding
    # noise of the size of the terms that cancel
    # overflowed or invalid elements (a chain that squares and cubes its input can leave them) must
    # sit in the same places with the same values; the bar applies to the finite ones
    fin = np.isfinite(want)
    assert (np.isfinite(got) == fin).all() and (np.isnan(got) == np.isnan(want)).all(), \
        f"{what}: non-finite elements differ in place"
    assert (got[np.isinf(want)] == want[np.isinf(want)]).all(), f"{what}: infinities differ"
    got, want = got[fin], want[fin]
    tol = max(2e-4 * float(np.abs(want).max(initial=0.0)), 2e-5 * chain_scale, loss_floor, 1e-30)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert (err <= tol).all(), f"{what}: max error {float(err.max(initial=0.0)):.3g} over the bar {tol:.3g}"


@pytest.mark.parametrize("exact_only,seed",
                         [(False, s) for s in range(160 * SWEEP)] + [(True, s) for s in range(80 * SWEEP)])
def test_random_chain_matches_reference_engine(engines, exact_only, seed):
    x_shape, ops, exact, out_shape = make_plan(seed, exact_only)
    assert exact or not exact_only
    what = f"seed {seed} x {x_shape} ops {ops}"
    (gout, ggrads, _), (rout, rgrads, logits_max) = (run_plan(e, seed, x_shape, ops) for e in engines)
    assert len(ggrads) == len(rgrads)
    scale = max(float(np.abs(r[np.isfinite(r)]).max(initial=0.0)) for r in [rout] + rgrads)
    # a loss head's value carries the fp32 rounding of log-probabilities of logits this large (the
    # reference sums its exponentials in fp32, this engine in fp64)
    _same(gout, rout, exact, what + " output", scale, 1e-6 * logits_max)
    for i, (g, r) in enumerate(zip(ggrads, rgrads)):
        _same(g, r, exact, f"{what} grad of parameter {i}", scale)


def build_model(e, seed, x_shape, ops):
    """The plan's parameters (and loss labels, as persistent tensors) in engine e, and a function that
    runs the plan's forward over them: (params, forward)."""
    L = e.lib
    rng = np.random.default_rng(10_000 + seed)
    params = [e.param(rng.standard_normal(x_shape).astype(np.float32))]
    steps = []
    L.nc_persistent_begin(e.ctx)
    for op in ops:
        if op[0] == "binary":
            vals = rng.standard_normal(op[2]).astype(np.float32)
            if op[1] == "div":
                vals = (0.5 + 1.5 * rng.random(op[2])).astype(np.float32)
            params.append(e.param(vals))
            steps.append((op, [params[-1]]))
        elif op[0] == "layer_norm":
            params += [e.param((1 + 0.1 * rng.standard_normal(op[1])).astype(np.float32)),
                       e.param((0.1 * rng.standard_normal(op[1])).astype(np.float32))]
            steps.append((op, params[-2:]))
        elif op[0] == "matmul":
            params.append(e.param((rng.standard_normal((op[1], op[2])) / np.sqrt(op[1])).astype(np.float32)))
            steps.append((op, [params[-1]]))
        elif op[0] == "linear":
            params += [e.param((rng.standard_normal((op[2], op[1])) / np.sqrt(op[1])).astype(np.float32)),
                       e.param((0.1 * rng.standard_normal(op[2])).astype(np.float32))]
            steps.append((op, params[-2:]))
        elif op[0] == "loss":
            steps.append((op, [e.tensor(rng.integers(0, op[3], op[2]).astype(np.int32))]))
        elif op[0] == "mse":
            steps.append((op, [e.tensor(rng.standard_normal(op[1]).astype(np.float32))]))
        else:
            steps.append((op, []))
    L.nc_persistent_end(e.ctx)
    e.check()

    def forward():
        t = params[0]
        for op, ts in steps:
            if op[0] == "unary":
                t = Engine.UNARY_CALLS[op[1]](L, t, op[2])
            elif op[0] == "binary":
                t = {"add": L.nc_add, "sub": L.nc_sub, "mul": L.nc_mul, "div": L.nc_div}[op[1]](t, ts[0])
            elif op[0] == "self":
                t = {"add": L.nc_add, "mul": L.nc_mul}[op[1]](t, t)
            elif op[0] == "positive":
                t = Engine.UNARY_CALLS[op[1]](L, L.nc_add_scalar(L.nc_mul(t, t), c_float(0.5)), op[2])
            elif op[0] == "residual":
                t = L.nc_add(t, Engine.UNARY_CALLS[op[1]](L, t, op[2]))
            elif op[0] == "transpose":
                t = L.nc_transpose(t, op[1], op[2])
            elif op[0] == "slice":
                t = L.nc_slice(t, op[1], op[2], op[3], op[4])
            elif op[0] == "bounded_exp":
                t = L.nc_exp(L.nc_tanh(t))
            elif op[0] == "mse":
                t = L.nc_mse_loss(t, ts[0])
            elif op[0] == "reshape":
                nd, shp = abi.shape_arg(op[1])
                t = L.nc_reshape(t, nd, shp)
            elif op[0] == "reduce":
                t = {"sum": L.nc_sum, "mean": L.nc_mean, "max": L.nc_max}[op[1]](t, op[2], op[3])
            elif op[0] == "softmax":
                t = L.nc_log_softmax(t) if op[1] else L.nc_softmax(t)
            elif op[0] == "layer_norm":
                t = L.nc_layer_norm(t, 1, ts[0], ts[1], c_float(1e-5))
            elif op[0] == "matmul":
                t = L.nc_matmul(t, ts[0])
            elif op[0] == "linear":
                t = L.nc_linear_fn(t, ts[0], ts[1])
            elif op[0] == "loss":
                nd, shp = abi.shape_arg((op[2], op[3]))
                t2 = L.nc_reshape(t, nd, shp)
                t = L.nc_cross_entropy(t2, ts[0]) if op[1] else L.nc_nll_loss(L.nc_log_softmax(t2), ts[0], 0)
            e.check()
        return t

    return params, forward


OPTIMS = {"sgd": lambda L, c, p, n: L.nc_sgd(c, p, n, abi.OptimOpts(0.05, 0.9, 0.01, 0, 0, 0)),
          "sgd_small": lambda L, c, p, n: L.nc_sgd(c, p, n, abi.OptimOpts(0.01, 0.9, 0.01, 0, 0, 0)),
          "adam": lambda L, c, p, n: L.nc_adam(c, p, n, abi.OptimOpts(0.01, 0, 0, 0.9, 0.999, 1e-8)),
          "adamw": lambda L, c, p, n: L.nc_adamw(c, p, n, abi.OptimOpts(0.01, 0, 0.05, 0.9, 0.99, 1e-8)),
          "rmsprop": lambda L, c, p, n: L.nc_rmsprop(c, p, n, abi.OptimOpts(0.01, 0.5, 0, 0, 0.99, 1e-8), 0)}


def train(e, seed, x_shape, ops, optim, clip, iters=3):
    """iters steps of forward, backward of sum(out * G), clip_grad_norm (when clip), optimizer step and
    zero_grad; the parameters' final values and the norms clip_grad_norm returned."""
    L = e.lib
    params, forward = build_model(e, seed, x_shape, ops)
    plist = (ctypes.c_void_p * len(params))(*params)
    opt = OPTIMS[optim](L, e.ctx, plist, len(params))
    e.check()
    rng = np.random.default_rng(20_000 + seed)
    norms = []
    for _ in range(iters):
        out = forward()
        G = rng.standard_normal(e.read(out).shape).astype(np.float32)
        e.backward_with(out, G)
        if clip:
            norms.append(L.nc_clip_grad_norm(plist, len(params), c_float(clip)))
        L.nc_optim_step(opt)
        L.nc_optim_zero_grad(opt)
        e.check()
        e.step_end()
    final = [e.read(p) for p in params]
    L.nc_optim_free(opt)
    e.step_end()
    return final, norms


@pytest.mark.parametrize("exact_only,seed", [(False, s) for s in range(40 * SWEEP)] + [(True, s) for s in range(40 * SWEEP)])
def test_training_steps_match_reference_engine(engines, exact_only, seed):
    """Three training steps of a random chain in both engines: for chains of order-independent ops,
    SGD with momentum and weight decay, Adam, AdamW or RMSprop in turn by seed (clip_grad_norm before
    every other optimizer's steps), and the parameters after the last step bit for bit (the
    optimizers' updates are the reference's expressions); for the other chains SGD with a small step
    after clipping to norm 1, within the bar.  (Adam and RMSprop divide by the gradient's running
    magnitude, so a parameter whose true gradient is ~0 moves by about lr per step in whatever
    direction its rounding noise points, differently in each engine; and unclipped steps on chains
    that square and cube their input diverge, where any difference grows without bound.)"""
    x_shape, ops, exact, _ = make_plan(seed + 700, exact_only)
    names = ["sgd", "adam", "adamw", "rmsprop"]
    if exact_only:
        optim = names[seed % len(names)]
        clip = (0.5 if seed % 3 == 0 else 50.0) if (seed // len(names)) % 2 == 0 else 0.0
    else:
        optim, clip = "sgd_small", 1.0
    what = f"seed {seed} {optim} clip {clip} x {x_shape} ops {ops}"
    (gp, gn), (rp, rn) = (train(e, seed, x_shape, ops, optim, clip) for e in engines)
    if exact:
        _same(np.array(gn, np.float32), np.array(rn, np.float32), True, what + " clip norms", 0.0)
    else:
        # a norm over gradients that a saturated softmax leaves at rounding-noise size carries that
        # noise (this engine sums softmax's g . y in fp64, the reference in fp32): 1%, or 1e-6 for a
        # norm of pure rounding noise (a saturated loss), and the parameters below at the usual bar
        assert np.allclose(gn, rn, rtol=1e-2, atol=1e-6), f"{what} clip norms {gn} vs {rn}"
    scale = max(float(np.abs(r[np.isfinite(r)]).max(initial=0.0)) for r in rp)
    for i, (g, r) in enumerate(zip(gp, rp)):
        _same(g, r, exact, f"{what} parameter {i} after the steps", scale)


def run_twice(e, seed, x_shape, ops):
    """The plan once forward, then two backward passes over it (sum(out * G1), then sum(out * G2),
    the graph retained), the second adding into the gradients the first left."""
    params, forward = build_model(e, seed, x_shape, ops)
    out = forward()
    rng = np.random.default_rng(30_000 + seed)
    shape = e.read(out).shape
    for _ in range(2):
        e.backward_with(out, rng.standard_normal(shape).astype(np.float32))
    grads = [e.grad(p) for p in params]
    e.step_end()
    return grads


@pytest.mark.parametrize("exact_only,seed", [(False, s) for s in range(30 * SWEEP)] + [(True, s) for s in range(30 * SWEEP)])
def test_retained_graph_backward_twice(engines, exact_only, seed):
    """Two backward passes over one retained graph: every parameter's gradient holds both passes'
    sums, as the reference's (bit for bit for order-independent chains)."""
    x_shape, ops, exact, _ = make_plan(seed + 1400, exact_only)
    what = f"seed {seed} x {x_shape} ops {ops}"
    gg, rg = (run_twice(e, seed, x_shape, ops) for e in engines)
    scale = max(float(np.abs(r[np.isfinite(r)]).max(initial=0.0)) for r in rg)
    for i, (g, r) in enumerate(zip(gg, rg)):
        _same(g, r, exact, f"{what} grad of parameter {i} after two passes", scale)


@pytest.mark.parametrize("seed", range(12 * SWEEP))
def test_linear_int8_matches_reference(engines, seed):
    """quantize_rows of a weight, then linear_int8 of activations against it (with and without bias),
    on random shapes in both engines: quantized weights, scales and outputs bit for bit."""
    rng = np.random.default_rng(40_000 + seed)
    M, K, N = (int(v) for v in rng.integers(1, 300, 3))
    x = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    w = rng.standard_normal((N, K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) if seed % 2 else None
    outs = []
    for e in engines:
        L = e.lib
        sc = ctypes.c_void_p()
        wq = L.nc_quantize_rows(e.tensor(w), ctypes.byref(sc))
        e.check()
        y = L.nc_linear_int8(e.tensor(x), wq, sc, e.tensor(b) if b is not None else None)
        outs.append((e.read(wq), e.read(sc), e.read(y)))
        e.step_end()
    (gq, gs, gy), (rq, rs, ry) = outs
    what = f"seed {seed} M {M} K {K} N {N} bias {b is not None}"
    assert (gq == rq).all(), what + " quantized weight"
    _same(gs, rs, True, what + " scales", 0.0)
    _same(gy, ry, True, what + " linear_int8 output", 0.0)
