"""Writes the golden vectors in tests/golden/*.npz from the compiled reference engine.

Run in a container that has the reference tree (oracle/_ref/libnc_ref.so is built from it by
`make -C oracle ref`):

    python tests/golden/gen_golden.py

Every input is drawn here from numpy's seeded generator and stored next to the reference's outputs,
so the fixtures are self-contained data.  Outputs come from the reference's public C API (nc.h),
driven through ctypes exactly as its Python package drives it, and for the four vector
transcendentals from its kernel table (oracle/ref_probe.c).  Backward values are obtained the way
the reference computes them: loss = sum(out * G) and a retained backward pass, which seeds the
output grad with exactly G.
"""

from __future__ import annotations

import ctypes
import sys
from ctypes import c_float, c_int64, c_void_p
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from newch_amd import abi  # noqa: E402

OUT = Path(__file__).resolve().parent
REF_LIB = ROOT / "oracle" / "_ref" / "libnc_ref.so"

SPECIALS = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 1e-30, -1e-30, 1e-6, -1e-6,
                     -87.3365448, -87.34, -87.33, -87.5, -95.0, -120.0, 88.5, 88.7, 88.72, 88.8, 100.0,
                     0.25, 0.2499999, 0.2500001, -0.25, -0.2499999, 0.0625, -3.0, 3.0, -3.0000002, 3.0000002,
                     -2.9999998, 2.9999998, 6.0, 5.9999995, 6.0000005, -6.0, 0.5, -0.5, 1.0, -1.0, 2.0, -2.0,
                     -5.0, -7.5, -10.0, -13.0, -20.0, 5.0, 10.0, 20.0, 1e30, -1e30, 3.4e38, -3.4e38],
                    dtype=np.float32)


class Ref:
    """A reference engine context with helpers to move numpy arrays in and out."""

    def __init__(self, lib):
        self.lib = lib
        cfg = abi.Config(0, 1234, 0, 0)
        self.ctx = lib.nc_init(ctypes.byref(cfg))

    def check(self):
        if not self.lib.nc_ok(self.ctx):
            raise RuntimeError(self.lib.nc_error(self.ctx).decode())

    def tensor(self, arr, dtype=abi.F32):
        arr = np.array(arr, order="C", copy=True)  # keeps 0-d shapes (ascontiguousarray would not)
        nd, shp = abi.shape_arg(arr.shape)
        t = self.lib.nc_from_data(self.ctx, dtype, arr.ctypes.data_as(c_void_p), nd, shp)
        self.check()
        return t

    def param(self, arr):
        src = self.tensor(np.asarray(arr, np.float32))
        nd, shp = abi.shape_arg(arr.shape)
        p = self.lib.nc_parameter(self.ctx, src, nd, shp)
        self.check()
        return p

    def read(self, t, dtype=np.float32):
        self.check()
        n = self.lib.nc_numel(t)
        nd = self.lib.nc_ndim(t)
        shape = tuple(self.lib.nc_shape(t)[i] for i in range(nd))
        out = np.empty(n, dtype=dtype)
        ok = self.lib.nc_copy_to(t, out.ctypes.data_as(c_void_p), out.nbytes)
        if not ok:
            raise RuntimeError("copy_to failed")
        return out.reshape(shape)

    def backward_with(self, out, G):
        """loss = sum(out * G); retained backward, so the output grad is exactly G."""
        loss = self.lib.nc_sum(self.lib.nc_mul(out, self.tensor(G.astype(np.float32))), abi.ALL_AXES, 0)
        self.check()
        st = self.lib.nc_backward_ex(loss, abi.BACKWARD_RETAIN, None, 0)
        if st != 0:
            raise RuntimeError(self.lib.nc_error(self.ctx).decode())

    def grad(self, t):
        g = self.lib.nc_grad(t)
        if not g:
            raise RuntimeError("no grad")
        return self.read(g)

    def step_end(self):
        self.lib.nc_step_end(self.ctx)


def gen_transcendentals(lib, rng):
    grid = np.linspace(-100, 100, 2001, dtype=np.float32)
    dense = np.linspace(-6, 6, 1201, dtype=np.float32)
    rnd = (rng.standard_normal(2048) * 4).astype(np.float32)
    bits = np.frombuffer(rng.integers(0, 2 ** 32, 2048, dtype=np.uint32).tobytes(), np.float32)
    x = np.concatenate([SPECIALS, grid, dense, rnd, bits]).astype(np.float32)
    res = {"x": x}
    P = c_void_p
    for nm in ("exp", "sigmoid", "tanh", "erf"):
        y = np.empty_like(x)
        getattr(lib, f"ncref_{nm}_f32")(c_int64(x.size), x.ctypes.data_as(P), y.ctypes.data_as(P))
        res[nm] = y
    sums = []
    sx = rng.standard_normal(5000).astype(np.float32)
    lib.ncref_sum_f32.restype = c_float
    for n in (0, 1, 7, 15, 16, 17, 31, 32, 33, 100, 1000, 4999):
        sums.append(lib.ncref_sum_f32(c_int64(n), sx.ctypes.data_as(P)))
    res["sum_x"] = sx
    res["sum_n"] = np.array([0, 1, 7, 15, 16, 17, 31, 32, 33, 100, 1000, 4999], np.int64)
    res["sum_out"] = np.array(sums, np.float32)
    np.savez_compressed(OUT / "transcendentals.npz", **res)


UNARY = [  # name, kind (oracle numbering), nc.h call
    ("relu", 0, lambda L, t: L.nc_relu(t)),
    ("leaky_relu", 1, lambda L, t: L.nc_leaky_relu(t, 0.01)),
    ("leaky_relu_02", 1, lambda L, t: L.nc_leaky_relu(t, 0.2)),
    ("relu6", 2, lambda L, t: L.nc_relu6(t)),
    ("hardsigmoid", 3, lambda L, t: L.nc_hardsigmoid(t)),
    ("hardswish", 4, lambda L, t: L.nc_hardswish(t)),
    ("silu", 5, lambda L, t: L.nc_silu(t)),
    ("gelu", 6, lambda L, t: L.nc_gelu(t, 0)),
    ("gelu_tanh", 7, lambda L, t: L.nc_gelu(t, 1)),
    ("sigmoid", 8, lambda L, t: L.nc_sigmoid(t)),
    ("tanh", 9, lambda L, t: L.nc_tanh(t)),
    ("exp", 10, lambda L, t: L.nc_exp(t)),
]


def gen_unary(ref, rng):
    x = np.concatenate([SPECIALS, (rng.standard_normal(1037) * 3).astype(np.float32),
                        np.linspace(-8, 8, 513, dtype=np.float32)]).astype(np.float32)
    g = rng.standard_normal(x.size).astype(np.float32)
    res = {"x": x, "g": g}
    for name, _, fn in UNARY:
        p = ref.param(x)
        y = fn(ref.lib, p)
        res[f"{name}_y"] = ref.read(y)
        ref.backward_with(y, g)
        res[f"{name}_gx"] = ref.grad(p)
        ref.step_end()
    np.savez_compressed(OUT / "unary.npz", **res)


def make_view(ref, storage, view):
    """view: None | ('t', a0, a1) | ('t_reshape', a0, a1, shape)"""
    p = ref.param(storage)
    if view is None:
        return p, p
    v = ref.lib.nc_transpose(p, view[1], view[2])
    if view[0] == "t_reshape":
        nd, shp = abi.shape_arg(view[3])
        v = ref.lib.nc_reshape(v, nd, shp)
    ref.check()
    return p, v


BINARY_CASES = [
    # name, a storage shape, a view, b storage shape, b view
    ("bias4d", (4, 3, 5, 7), None, (1, 3, 1, 1), None),
    ("row", (2, 3), None, (3,), None),
    ("outer", (2, 1), None, (1, 3), None),
    ("scalar_lhs", (), None, (3,), None),
    ("scalar_rhs", (5, 4), None, (), None),
    ("cfg2_small", (5, 6, 1, 8), None, (1, 1, 7, 8), None),
    ("cfg2_batch_t", (6, 5, 1, 8), ("t", 0, 1), (1, 1, 7, 8), None),
    ("cfg2_inner_strided", (5, 8, 6), ("t_reshape", 1, 2, (5, 6, 1, 8)), (1, 1, 7, 8), None),
    ("same_flat", (17, 33), None, (17, 33), None),
    ("same_a_t", (33, 17), ("t", 0, 1), (17, 33), None),
    ("rank_mismatch", (3, 1, 5), None, (4, 1), None),
    ("ragged", (3, 1, 37), None, (1, 11, 37), None),
]


def gen_binary(ref, rng):
    res = {}
    ops = [("add", ref.lib.nc_add), ("sub", ref.lib.nc_sub), ("mul", ref.lib.nc_mul), ("div", ref.lib.nc_div)]
    for name, ash, aview, bsh, bview in BINARY_CASES:
        A = rng.standard_normal(ash).astype(np.float32)
        B = (0.5 + 1.5 * rng.random(bsh)).astype(np.float32)
        res[f"{name}/a_storage"] = A
        res[f"{name}/b_storage"] = B
        for opname, fn in ops:
            pa, va = make_view(ref, A, aview)
            pb, vb = make_view(ref, B, bview)
            out = fn(va, vb)
            y = ref.read(out)
            G = rng.standard_normal(y.shape).astype(np.float32)
            ref.backward_with(out, G)
            res[f"{name}/{opname}/out"] = y
            res[f"{name}/{opname}/G"] = G
            res[f"{name}/{opname}/ga"] = ref.grad(va)  # grad in the (view's) logical shape
            res[f"{name}/{opname}/gb"] = ref.grad(vb)
            ref.step_end()
    np.savez_compressed(OUT / "binary.npz", **res)


def gen_reduce(ref, rng):
    res = {}
    cases = {
        "r2x3": rng.standard_normal((2, 3)).astype(np.float32),
        "r4x5x6": rng.standard_normal((4, 5, 6)).astype(np.float32),
        "r3x1000": (rng.standard_normal((3, 1000)) * 2).astype(np.float32),
        "r5x13x9": rng.standard_normal((5, 13, 9)).astype(np.float32),
    }
    sp = rng.standard_normal((8, 9)).astype(np.float32)
    sp[0, 4] = sp[0, 7] = 5.0                        # tie: first index wins
    sp[1, 0] = np.nan                                # NaN first: sticky
    sp[2, 3] = np.nan                                # NaN later: ignored
    sp[3, :] = -np.inf                               # all -inf
    sp[4, :] = 0.0; sp[4, 0] = -0.0                  # signed zero ties
    sp[5, 2] = np.inf
    sp[6, :] = np.nan
    sp[7, 8] = 1e30
    cases["special"] = sp
    for cname, X in cases.items():
        res[f"{cname}/x"] = X
        axes = list(range(X.ndim)) + [abi.ALL_AXES]
        for axis in axes:
            for kname, fn in (("sum", ref.lib.nc_sum), ("mean", ref.lib.nc_mean), ("max", ref.lib.nc_max)):
                if cname == "special" and kname != "max":
                    continue
                p = ref.param(X)
                out = fn(p, axis, 0)
                y = ref.read(out)
                G = rng.standard_normal(y.shape).astype(np.float32)
                ref.backward_with(out, G)
                res[f"{cname}/{kname}/{axis}/y"] = y
                res[f"{cname}/{kname}/{axis}/G"] = G
                res[f"{cname}/{kname}/{axis}/gx"] = ref.grad(p)
                ref.step_end()
            t = ref.tensor(X)
            res[f"{cname}/argmax/{axis}/y"] = ref.read(ref.lib.nc_argmax(t, axis), np.int32)
            ref.step_end()
    empty = ref.tensor(np.zeros((0, 3), np.float32))
    res["empty/mean_all"] = ref.read(ref.lib.nc_mean(empty, abi.ALL_AXES, 0))
    res["empty/mean_0"] = ref.read(ref.lib.nc_mean(empty, 0, 0))
    res["empty/sum_0"] = ref.read(ref.lib.nc_sum(empty, 0, 0))
    ref.step_end()
    np.savez_compressed(OUT / "reduce.npz", **res)


def gen_softmax(ref, rng):
    res = {}
    for rows, C in ((3, 1), (4, 7), (5, 64), (3, 100), (2, 1030), (6, 17)):
        X = (rng.standard_normal((rows, C)) * 2).astype(np.float32)
        if C >= 7:
            X[0, 3] = -np.inf
            X[1, 2] = X[1, 5] = X[1].max() + 1.0
        key = f"{rows}x{C}"
        res[f"{key}/x"] = X
        for form, fn in (("softmax", ref.lib.nc_softmax), ("log_softmax", ref.lib.nc_log_softmax)):
            p = ref.param(X)
            out = fn(p)
            y = ref.read(out)
            G = rng.standard_normal(y.shape).astype(np.float32)
            ref.backward_with(out, G)
            res[f"{key}/{form}/y"] = y
            res[f"{key}/{form}/G"] = G
            res[f"{key}/{form}/gx"] = ref.grad(p)
            ref.step_end()
    np.savez_compressed(OUT / "softmax.npz", **res)


def gen_layer_norm(ref, rng):
    res = {}
    for key, shape, k in (("6x10", (6, 10), 1), ("3x4x5", (3, 4, 5), 2), ("4x1024", (4, 1024), 1),
                          ("2x3", (2, 3), 1)):
        X = (rng.standard_normal(shape) * 2 + 0.5).astype(np.float32)
        D = int(np.prod(shape[len(shape) - k:]))
        W = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
        Bv = (0.1 * rng.standard_normal(D)).astype(np.float32)
        res[f"{key}/x"] = X
        res[f"{key}/w"] = W
        res[f"{key}/b"] = Bv
        res[f"{key}/k"] = np.array(k)
        for variant in ("wb", "w", "none"):
            px = ref.param(X)
            pw = ref.param(W) if variant in ("wb", "w") else None
            pb = ref.param(Bv) if variant == "wb" else None
            out = ref.lib.nc_layer_norm(px, k, pw, pb, c_float(1e-5))
            y = ref.read(out)
            G = rng.standard_normal(y.shape).astype(np.float32)
            ref.backward_with(out, G)
            res[f"{key}/{variant}/y"] = y
            res[f"{key}/{variant}/G"] = G
            res[f"{key}/{variant}/gx"] = ref.grad(px)
            if pw:
                res[f"{key}/{variant}/gw"] = ref.grad(pw)
            if pb:
                res[f"{key}/{variant}/gb"] = ref.grad(pb)
            ref.step_end()
    np.savez_compressed(OUT / "layernorm.npz", **res)


def gen_quant(ref, rng):
    W = (rng.standard_normal((12, 70)) * 0.2).astype(np.float32)
    idx = rng.choice(W.size, 8, replace=False)
    W.flat[idx] *= 50
    W[3, :] = 0.0                                             # zero row: scale 1
    W[4, :9] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]  # exact ties, scale 1
    W[4, 9:] = 0.25
    W[5, 0] = np.nan                                          # NaN ignored by the absmax, quantizes to 0
    W[6, 5] = np.inf                                          # inf absmax: scale inf, all zeros
    W[7, :] = -3e-39                                          # denormal row
    W[8, :] = np.linspace(-1, 1, 70, dtype=np.float32)
    W[9, 0] = -5.0
    res = {"w": W}
    pw = ref.tensor(W)
    sc = c_void_p()
    q = ref.lib.nc_quantize_rows(pw, ctypes.byref(sc))
    res["q"] = ref.read(q, np.int8)
    res["scale"] = ref.read(sc.value)
    qf = ref.lib.nc_to_dtype(q, abi.F32)
    nd, shp = abi.shape_arg((W.shape[0], 1))
    deq = ref.lib.nc_mul(qf, ref.lib.nc_reshape(sc.value, nd, shp))
    res["deq"] = ref.read(deq)
    ref.step_end()
    np.savez_compressed(OUT / "quant.npz", **res)


def gen_chain(ref, rng):
    """The MNIST-CNN-shaped chain at a small batch: relu(x + bias).sum((2, 3)), with the reference
    Python package's multi-dim reduction composition (one keepdim sum per dim, last dim first,
    then a reshape: newch/tensor.py:701-717)."""
    X = rng.uniform(-1, 1, (4, 16, 28, 28)).astype(np.float32)
    Bv = rng.uniform(-0.1, 0.1, (1, 16, 1, 1)).astype(np.float32)
    G = rng.standard_normal((4, 16)).astype(np.float32)
    px, pb = ref.param(X), ref.param(Bv)
    h = ref.lib.nc_relu(ref.lib.nc_add(px, pb))
    s = ref.lib.nc_sum(ref.lib.nc_sum(h, 3, 1), 2, 1)
    nd, shp = abi.shape_arg((4, 16))
    y = ref.lib.nc_reshape(s, nd, shp)
    out = ref.read(y)
    ref.backward_with(y, G)
    np.savez_compressed(OUT / "chain.npz", x=X, bias=Bv, G=G, y=out, gx=ref.grad(px), gbias=ref.grad(pb))
    ref.step_end()


def gen_loss(ref, rng):
    """cross_entropy and nll_loss (mean and sum): loss, and the input gradient for an upstream grad
    G (a scalar), from a retained backward; plus the reference's messages for out-of-range labels."""
    res = {}
    cases = [("3x5", 3, 5), ("8x10", 8, 10), ("4x1", 4, 1), ("6x64", 6, 64), ("5x1030", 5, 1030), ("0x7", 0, 7)]
    for key, N, C in cases:
        X = (rng.standard_normal((N, C)) * 3).astype(np.float32)
        lab = rng.integers(0, C, N).astype(np.int32)
        if N >= 4:
            lab[0], lab[1] = 0, C - 1
        if N >= 4 and C >= 7:
            X[2, 3] = -np.inf
            X[3, :] = 0.0  # a uniform row
        res[f"{key}/x"] = X
        res[f"{key}/lab"] = lab
        G = np.float32(rng.standard_normal())
        res[f"{key}/G"] = G
        for form in ("ce", "nll_mean", "nll_sum"):
            p = ref.param(X)
            t = ref.tensor(lab, dtype=abi.I32)
            if form == "ce":
                out = ref.lib.nc_cross_entropy(p, t)
            else:
                out = ref.lib.nc_nll_loss(p, t, int(form == "nll_sum"))
            res[f"{key}/{form}/loss"] = ref.read(out)
            if N > 0:
                ref.backward_with(out, np.asarray(G))
                res[f"{key}/{form}/gx"] = ref.grad(p)
            ref.step_end()
    # out-of-range labels: the reference's error text
    X = rng.standard_normal((4, 6)).astype(np.float32)
    for name, lab in (("high", [0, 1, 6, 2]), ("negative", [0, -1, 2, 9])):
        lab = np.array(lab, np.int32)
        for form, fn in (("ce", lambda p, t: ref.lib.nc_cross_entropy(p, t)),
                         ("nll", lambda p, t: ref.lib.nc_nll_loss(p, t, 0))):
            out = fn(ref.tensor(X), ref.tensor(lab, dtype=abi.I32))
            assert not out and not ref.lib.nc_ok(ref.ctx)
            res[f"bad_{name}/{form}/message"] = np.array(ref.lib.nc_error(ref.ctx).decode())
            res[f"bad_{name}/{form}/status"] = np.int32(ref.lib.nc_status_code(ref.ctx))
            ref.lib.nc_clear_error(ref.ctx)
        res[f"bad_{name}/x"] = X
        res[f"bad_{name}/lab"] = lab
    ref.step_end()
    np.savez_compressed(OUT / "loss.npz", **res)


OPTIM_CONFIGS = [
    # name, constructor, opts (lr, momentum, weight_decay, beta1, beta2, eps), rmsprop eps_inside_sqrt,
    # accumulation steps, micro-steps
    ("sgd", "nc_sgd", (0.1, 0, 0, 0, 0, 0), None, 1, 3),
    ("sgd_mom_wd", "nc_sgd", (0.05, 0.9, 0.01, 0, 0, 0), None, 1, 3),
    ("adam", "nc_adam", (0.01, 0, 0.01, 0, 0, 0), None, 1, 3),
    ("adamw", "nc_adamw", (0.01, 0, 0.1, 0.8, 0.99, 1e-6), None, 1, 3),
    ("rmsprop", "nc_rmsprop", (0.01, 0, 0, 0, 0, 0), 0, 1, 3),
    ("rmsprop_keras_mom", "nc_rmsprop", (0.01, 0.5, 0.001, 0, 0.9, 1e-7), 1, 1, 3),
    ("adam_accum2", "nc_adam", (0.01, 0, 0, 0, 0, 0), None, 2, 4),
]
OPTIM_SHAPES = [(7,), (3, 5)]


def optim_scenario(e, lib, cfg, W, Gs):
    """Runs one optimizer configuration on params initialised to W with upstream grads Gs[step][param]
    (loss = sum_i sum(p_i * G_i), so each step's grads are exactly G); returns per-step weights and
    state.  `e` is any context wrapper with tensor / param / read (the reference's or this engine's)."""
    name, ctor, opts, inside, accum, steps = cfg
    params = [e.param(w) for w in W]
    arr = (ctypes.c_void_p * len(params))(*params)
    o_opts = abi.OptimOpts(*[float(v) for v in opts])
    o = getattr(lib, ctor)(e.ctx, arr, len(params), o_opts) if inside is None else \
        lib.nc_rmsprop(e.ctx, arr, len(params), o_opts, inside)
    assert o, lib.nc_error(e.ctx)
    if accum > 1:
        lib.nc_optim_set_accumulation(o, accum)
    out = {}
    for k in range(steps):
        lib.nc_optim_zero_grad(o)
        loss = None
        for p, G in zip(params, Gs[k]):
            term = lib.nc_sum(lib.nc_mul(p, e.tensor(G)), abi.ALL_AXES, 0)
            loss = term if loss is None else lib.nc_add(loss, term)
        assert lib.nc_backward_ex(loss, 0, None, 0) == 0, lib.nc_error(e.ctx)
        lib.nc_optim_step(o)
        for i, p in enumerate(params):
            out[f"{name}/step{k}/w{i}"] = e.read(p)
            for slot in (0, 1):
                ptr = lib.nc_optim_state(o, i, slot)
                if ptr:
                    n = W[i].size
                    out[f"{name}/step{k}/s{slot}_{i}"] = np.ctypeslib.as_array(
                        (ctypes.c_float * n).from_address(ptr)).reshape(W[i].shape).copy()
        e.step_end()
    out[f"{name}/t"] = np.int64(lib.nc_optim_get_step(o))
    lib.nc_optim_free(o)
    return out


def gen_optim(ref, rng):
    """Every optimizer kind through the reference's nc.h, a few steps each, plus clip_grad_norm."""
    res = {}
    lib = ref.lib
    for cfg in OPTIM_CONFIGS:
        name, steps = cfg[0], cfg[5]
        W = [rng.standard_normal(sh).astype(np.float32) for sh in OPTIM_SHAPES]
        Gs = [[rng.standard_normal(sh).astype(np.float32) for sh in OPTIM_SHAPES] for _ in range(steps)]
        for i, w in enumerate(W):
            res[f"{name}/w_init{i}"] = w
        for k in range(steps):
            for i, G in enumerate(Gs[k]):
                res[f"{name}/G{k}_{i}"] = G
        res.update(optim_scenario(ref, lib, cfg, W, Gs))
    # clip_grad_norm: one case that clips, one that does not
    for case, factor in (("clip", 0.5), ("noclip", 10.0)):
        W = [rng.standard_normal(sh).astype(np.float32) for sh in OPTIM_SHAPES]
        G = [rng.standard_normal(sh).astype(np.float32) * 3 for sh in OPTIM_SHAPES]
        params = [ref.param(w) for w in W]
        loss = None
        for p, g in zip(params, G):
            term = lib.nc_sum(lib.nc_mul(p, ref.tensor(g)), abi.ALL_AXES, 0)
            loss = term if loss is None else lib.nc_add(loss, term)
        assert lib.nc_backward_ex(loss, 0, None, 0) == 0
        norm = float(np.sqrt(sum((g.astype(np.float64) ** 2).sum() for g in G)))
        max_norm = np.float32(norm * factor)
        arr = (ctypes.c_void_p * len(params))(*params)
        total = lib.nc_clip_grad_norm(arr, len(params), max_norm)
        res[f"{case}/max_norm"] = max_norm
        res[f"{case}/total"] = np.float32(total)
        for i in range(len(params)):
            res[f"{case}/G{i}"] = G[i]
            res[f"{case}/g{i}"] = ref.grad(params[i])
        ref.step_end()
    np.savez_compressed(OUT / "optim.npz", **res)


MATMUL_CASES = [
    # name, a storage shape, a view, b storage shape, b view  (nc_matmul: b 2-D -> matmul, else bmm)
    ("mm_2d", (33, 70), None, (70, 45), None),
    ("mm_fold3d", (3, 17, 40), None, (40, 29), None),
    ("mm_a_t", (70, 33), ("t", 0, 1), (70, 45), None),
    ("mm_b_t", (33, 70), None, (45, 70), ("t", 0, 1)),
    ("mm_both_t", (70, 33), ("t", 0, 1), (45, 70), ("t", 0, 1)),
    ("mm_outer", (8, 1), None, (1, 9), None),
    ("mm_fold_t", (3, 40, 17), ("t", 1, 2), (40, 29), None),
    ("bmm_same", (4, 9, 20), None, (4, 20, 11), None),
    ("bmm_bcast_a2d", (9, 20), None, (4, 20, 11), None),
    ("bmm_bcast_4d", (2, 1, 9, 20), None, (1, 3, 20, 11), None),
    ("bmm_b_t", (2, 3, 9, 20), None, (2, 3, 11, 20), ("t", 2, 3)),
    ("bmm_rank", (5, 9, 20), None, (2, 1, 20, 11), None),
    ("bmm_batch_t", (9, 4, 20), ("t", 0, 1), (4, 20, 11), None),
]

LINEAR_CASES = [  # name, x storage shape, x view, W shape, bias
    ("lin_bias", (6, 70), None, (13, 70), True),
    ("lin_nobias_3d", (2, 5, 33), None, (17, 33), False),
    ("lin_x_t", (70, 6), ("t", 0, 1), (13, 70), True),
    ("lin_wide", (20, 160), None, (130, 160), True),
]

QLINEAR_CASES = [  # name, x shape, W shape, bias
    ("q_ref_test", (7, 70), (13, 70), True),          # the reference's own int8 test sizes (test_main.c:1046)
    ("q_aligned", (37, 128), (70, 128), False),
    ("q_3d", (2, 3, 64), (5, 64), True),
    ("q_tiles", (131, 80), (130, 80), True),          # four 128 x 128 tiles, K % 64 = 16
    ("q_odd_k", (9, 37), (11, 37), True),
]


def gen_linalg(ref, rng):
    """matmul / bmm / linear forward and grads, linear_int8 outputs, and the int8 GEMM kernel
    (ops_linalg.c, ops_quant.c:41-113, kernels_avx2.c:314-340)."""
    res = {}
    for name, ash, aview, bsh, bview in MATMUL_CASES:
        A = rng.standard_normal(ash).astype(np.float32)
        B = rng.standard_normal(bsh).astype(np.float32)
        pa, va = make_view(ref, A, aview)
        pb, vb = make_view(ref, B, bview)
        out = ref.lib.nc_matmul(va, vb)
        y = ref.read(out)
        G = rng.standard_normal(y.shape).astype(np.float32)
        ref.backward_with(out, G)
        res.update({f"{name}/a_storage": A, f"{name}/b_storage": B, f"{name}/out": y, f"{name}/G": G,
                    f"{name}/ga": ref.grad(va), f"{name}/gb": ref.grad(vb)})
        ref.step_end()
    for name, xsh, xview, wsh, has_b in LINEAR_CASES:
        X = rng.standard_normal(xsh).astype(np.float32)
        W = (rng.standard_normal(wsh) * 0.2).astype(np.float32)
        Bv = rng.standard_normal(wsh[0]).astype(np.float32)
        px, vx = make_view(ref, X, xview)
        pw = ref.param(W)
        pbias = ref.param(Bv) if has_b else None
        out = ref.lib.nc_linear_fn(vx, pw, pbias)
        y = ref.read(out)
        G = rng.standard_normal(y.shape).astype(np.float32)
        ref.backward_with(out, G)
        res.update({f"{name}/x_storage": X, f"{name}/w": W, f"{name}/out": y, f"{name}/G": G,
                    f"{name}/gx": ref.grad(vx), f"{name}/gw": ref.grad(pw)})
        if has_b:
            res[f"{name}/bias"] = Bv
            res[f"{name}/gbias"] = ref.grad(pbias)
        ref.step_end()
    for name, xsh, wsh, has_b in QLINEAR_CASES:
        X = rng.standard_normal(xsh).astype(np.float32)
        if name == "q_tiles":
            X[3] = 0.0                      # zero row: scale 1
            X[5, 7] = 40.0                  # one large value dominates its row's scale
        W = (rng.standard_normal(wsh) * 0.2).astype(np.float32)
        Bv = rng.standard_normal(wsh[0]).astype(np.float32)
        pw = ref.tensor(W)
        sc = c_void_p()
        q = ref.lib.nc_quantize_rows(pw, ctypes.byref(sc))
        out = ref.lib.nc_linear_int8(ref.tensor(X), q, sc.value, ref.tensor(Bv) if has_b else None)
        res.update({f"{name}/x": X, f"{name}/w": W, f"{name}/q": ref.read(q, np.int8),
                    f"{name}/scale": ref.read(sc.value), f"{name}/out": ref.read(out),
                    f"{name}/fp32_out": ref.read(ref.lib.nc_linear_fn(ref.tensor(X), pw,
                                                                      ref.tensor(Bv) if has_b else None))})
        if has_b:
            res[f"{name}/bias"] = Bv
        ref.step_end()
    # the int8 GEMM of the kernel table on the reference's own known-answer inputs (test_main.c:1062-1073)
    # and on random ones; kernel-table entries are reached through oracle/ref_probe.c
    P = c_void_p
    kat_a = np.array([(i * 37) % 255 - 127 for i in range(5 * 37)], np.int8).reshape(5, 37)
    kat_b = np.array([(i * 91) % 255 - 127 for i in range(6 * 37)], np.int8).reshape(6, 37)
    for name, A, B in (("s8_kat", kat_a, kat_b),
                       ("s8_rand", rng.integers(-127, 128, (19, 131)).astype(np.int8),
                        rng.integers(-127, 128, (23, 131)).astype(np.int8)),
                       ("s8_extreme", np.full((4, 300), -127, np.int8), np.full((3, 300), -127, np.int8))):
        C = np.empty((A.shape[0], B.shape[0]), np.int32)
        ref.lib.ncref_gemm_s8_nt(c_int64(A.shape[0]), c_int64(B.shape[0]), c_int64(A.shape[1]), A.ctypes.data_as(P),
                                 c_int64(A.shape[1]), B.ctypes.data_as(P), c_int64(B.shape[1]), C.ctypes.data_as(P),
                                 c_int64(B.shape[0]))
        res.update({f"{name}/a": A, f"{name}/b": B, f"{name}/c": C})
    np.savez_compressed(OUT / "linalg.npz", **res)


GENERATORS = ["transcendentals", "unary", "binary", "reduce", "softmax", "layer_norm", "quant", "chain", "loss",
              "optim", "linalg"]


def main():
    lib = abi.load(REF_LIB)
    lib.ncref_backend.restype = ctypes.c_char_p
    backend = lib.ncref_backend().decode()
    if backend != "avx2":
        raise SystemExit(f"reference kernel tier is {backend!r}; fixtures must come from the avx2 tier")
    # every generator draws from its own seeded stream, so one fixture can be rewritten alone:
    #   python tests/golden/gen_golden.py loss
    only = sys.argv[1:] or GENERATORS
    ref = Ref(lib)
    rng = np.random.default_rng(20261201)  # the first eight share one stream, in this order
    if any(g in only for g in GENERATORS[:8]):
        gen_transcendentals(lib, rng)
        gen_unary(ref, rng)
        gen_binary(ref, rng)
        gen_reduce(ref, rng)
        gen_softmax(ref, rng)
        gen_layer_norm(ref, rng)
        gen_quant(ref, rng)
        gen_chain(ref, rng)
    if "loss" in only:
        gen_loss(ref, np.random.default_rng(20261202))
    if "optim" in only:
        gen_optim(ref, np.random.default_rng(20261203))
    if "linalg" in only:
        gen_linalg(ref, np.random.default_rng(20261204))
    (OUT / "PROVENANCE.txt").write_text(
        "Written by tests/golden/gen_golden.py from oracle/_ref/libnc_ref.so, which oracle/Makefile builds\n"
        "from the reference engine sources (engine/src/**/*.c) with gcc 11.4, -O2 -std=gnu11, x86-64\n"
        f"baseline + AVX2/FMA target functions; kernel tier: {backend}; numpy seeds 20261201 (one stream\n"
        "for transcendentals .. chain, in that order), 20261202 (loss), 20261203 (optim) and\n"
        "20261204 (linalg).\n")
    for f in sorted(OUT.glob("*.npz")):
        print(f"{f.name}: {f.stat().st_size / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
