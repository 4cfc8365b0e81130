"""numpy wrappers over the C oracle (oracle/_build/liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, to check results
against and as the CPU baseline.  The product library never uses it.  Function semantics: see oracle.h.
"""

from __future__ import annotations

import ctypes
import subprocess
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"
REF_LIB = HERE / "_ref" / "libnc_ref.so"

UN = {"relu": 0, "leaky_relu": 1, "relu6": 2, "hardsigmoid": 3, "hardswish": 4, "silu": 5, "gelu": 6,
      "gelu_tanh": 7, "sigmoid": 8, "tanh": 9, "exp": 10, "neg": 11, "scale": 12, "add_scalar": 13, "log": 14,
      "sqrt": 15, "pow": 16}
BIN = {"add": 0, "sub": 1, "mul": 2, "div": 3}
RED = {"sum": 0, "mean": 1, "max": 2, "argmax": 3}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE), "port"], check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        for nm in ("or_exp", "or_sigmoid", "or_tanh", "or_erf"):
            getattr(L, nm).restype = c_float
            getattr(L, nm).argtypes = [c_float]
        L.or_sum_f32.restype = c_float
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i64(v):
    v = list(v)
    return (c_int64 * max(len(v), 1))(*v)


def vmap(fn: str, x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().or_map(c_int({"exp": 0, "sigmoid": 1, "tanh": 2, "erf": 3}[fn]), c_int64(x.size), _p(x), _p(y))
    return y


def sum_f32(x):
    x = _f32(x)
    return np.float32(lib().or_sum_f32(c_int64(x.size), _p(x)))


def unary_fwd(kind: str, x, s: float = 0.0):
    x = _f32(x)
    y = np.empty_like(x)
    lib().or_unary_fwd(c_int(UN[kind]), c_float(s), _p(x), _p(y), c_int64(x.size))
    return y


def unary_bwd(kind: str, x, y, g, gi=None, s: float = 0.0):
    x, g = _f32(x), _f32(g)
    y = None if y is None else _f32(y)
    gi = np.zeros_like(g) if gi is None else _f32(gi).copy()
    lib().or_unary_bwd(c_int(UN[kind]), c_float(s), _p(x), _p(y), _p(g), _p(gi), c_int64(g.size))
    return gi


def broadcast_shape(*shapes):
    nd = max(len(s) for s in shapes)
    out = []
    for i in range(nd):
        dims = [s[i - (nd - len(s))] if i - (nd - len(s)) >= 0 else 1 for s in shapes]
        d = max(dims)
        out.append(d if all(x in (1, d) for x in dims) else None)
    if None in out:
        raise ValueError(f"shapes {shapes} are not broadcastable")
    return tuple(out)


def _elem_strides(a: np.ndarray):
    return tuple(s // a.itemsize for s in a.strides)


def _bcast_strides(shape, strides, out_shape):
    nd = len(out_shape)
    res = []
    for i in range(nd):
        j = i - (nd - len(shape))
        res.append(0 if j < 0 or (shape[j] == 1 and out_shape[i] != 1) else strides[j])
    return res


def _base_and_offset(a: np.ndarray):
    """(flat float32 base array, element offset of a[0,...]) for a view into a contiguous base."""
    base = a
    while base.base is not None and isinstance(base.base, np.ndarray):
        base = base.base
    off = (a.__array_interface__["data"][0] - base.__array_interface__["data"][0]) // a.itemsize
    return base, off


def binary_fwd(op: str, a, b):
    """a, b: float32 numpy arrays, possibly strided views (a view's strides are honoured)."""
    out_shape = broadcast_shape(a.shape, b.shape)
    o = np.empty(out_shape, np.float32)
    sa = _bcast_strides(a.shape, _elem_strides(a), out_shape)
    sb = _bcast_strides(b.shape, _elem_strides(b), out_shape)
    so = _elem_strides(o) if o.ndim else ()
    nd = len(out_shape)
    # pass a pointer to element 0 of each (possibly strided) view
    lib().or_binary_fwd(c_int(BIN[op]), c_int(nd), _i64(out_shape), c_void_p(a.__array_interface__["data"][0]),
                        _i64(sa), c_void_p(b.__array_interface__["data"][0]), _i64(sb), _p(o), _i64(so))
    return o


def binary_bwd(op: str, a, b, g, need_a=True, need_b=True, ga0=None, gb0=None):
    """Grads (in a's and b's logical shapes, contiguous) of sum(op(a, b) * g), accumulated onto
    ga0 / gb0 (zeros when not given)."""
    g = _f32(g)
    ga = (np.zeros(a.shape, np.float32) if ga0 is None else _f32(ga0).copy()) if need_a else None
    gb = (np.zeros(b.shape, np.float32) if gb0 is None else _f32(gb0).copy()) if need_b else None
    lib().or_binary_bwd(c_int(BIN[op]), c_int(a.ndim), _i64(a.shape), _i64(_elem_strides(a)),
                        c_void_p(a.__array_interface__["data"][0]), c_int(b.ndim), _i64(b.shape),
                        _i64(_elem_strides(b)), c_void_p(b.__array_interface__["data"][0]), _p(g), _p(ga), _p(gb))
    return ga, gb


def reduce_dims(shape, axis):
    if axis is None or axis == -128:
        return 1, int(np.prod(shape)), 1
    axis = axis % len(shape)
    outer = int(np.prod(shape[:axis]))
    inner = int(np.prod(shape[axis + 1:]))
    return outer, int(shape[axis]), inner


def reduce_fwd(kind: str, x, axis):
    x = _f32(x)
    outer, R, inner = reduce_dims(x.shape, axis)
    y = np.empty(outer * inner, np.float32)
    arg = np.empty(outer * inner, np.int32)
    lib().or_reduce_fwd(c_int(RED[kind]), c_int64(outer), c_int64(R), c_int64(inner), _p(x), _p(y), _p(arg))
    return (arg if kind == "argmax" else y), arg


def reduce_bwd(kind: str, x_shape, axis, g, arg=None, gi=None):
    outer, R, inner = reduce_dims(x_shape, axis)
    g = _f32(g)
    gi = np.zeros(int(np.prod(x_shape)), np.float32) if gi is None else _f32(gi).copy().ravel()
    lib().or_reduce_bwd(c_int(RED[kind]), c_int64(outer), c_int64(R), c_int64(inner), _p(g),
                        _p(None if arg is None else np.ascontiguousarray(arg, np.int32)), _p(gi))
    return gi.reshape(x_shape)


def softmax_fwd(x, log_form=False):
    x = _f32(x)
    C = x.shape[-1]
    y = np.empty_like(x)
    lib().or_softmax_fwd(c_int(int(log_form)), c_int64(x.size // max(C, 1)), c_int64(C), _p(x), _p(y))
    return y


def softmax_bwd(y, g, log_form=False, gi=None):
    y, g = _f32(y), _f32(g)
    C = y.shape[-1]
    gi = np.zeros_like(y) if gi is None else _f32(gi).copy()
    lib().or_softmax_bwd(c_int(int(log_form)), c_int64(y.size // max(C, 1)), c_int64(C), _p(y), _p(g), _p(gi))
    return gi


def layer_norm_fwd(x, D, w=None, b=None, eps=1e-5):
    x = _f32(x)
    rows = x.size // D
    y = np.empty_like(x)
    stats = np.empty(2 * rows, np.float32)
    lib().or_layer_norm_fwd(c_int64(rows), c_int64(D), _p(x), _p(None if w is None else _f32(w)),
                            _p(None if b is None else _f32(b)), c_float(eps), _p(y), _p(stats))
    return y, stats


def layer_norm_bwd(x, D, stats, g, w=None, need_w=False, need_b=False):
    x, g = _f32(x), _f32(g)
    rows = x.size // D
    gx = np.zeros_like(x)
    gw = np.zeros(D, np.float32) if need_w else None
    gb = np.zeros(D, np.float32) if need_b else None
    lib().or_layer_norm_bwd(c_int64(rows), c_int64(D), _p(x), _p(None if w is None else _f32(w)), _p(_f32(stats)),
                            _p(g), _p(gx), _p(gw), _p(gb))
    return gx, gw, gb


def quantize_rows(w):
    w = _f32(w)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    lib().or_quantize_rows(c_int64(rows), c_int64(cols), _p(w), _p(q), _p(s))
    return q, s


def dequantize_rows(q, scale):
    q = np.ascontiguousarray(q, np.int8)
    rows, cols = q.shape
    w = np.empty((rows, cols), np.float32)
    lib().or_dequantize_rows(c_int64(rows), c_int64(cols), _p(q), _p(_f32(scale)), _p(w))
    return w


def cross_entropy_fwd(x, lab):
    """(loss, prob) of cross_entropy(x [N, C], lab [N]); raises ValueError naming the first bad row."""
    x = _f32(x)
    lab = np.ascontiguousarray(lab, np.int32)
    N, C = x.shape
    prob = np.empty_like(x)
    loss = c_float(0.0)
    L = lib()
    L.or_cross_entropy_fwd.restype = c_int64
    bad = L.or_cross_entropy_fwd(c_int64(N), c_int64(C), _p(x), _p(lab), _p(prob), ctypes.byref(loss))
    if bad >= 0:
        raise ValueError(f"label {int(lab[bad])} at row {bad} outside [0, {C})")
    return np.float32(loss.value), prob


def cross_entropy_bwd(prob, lab, gout, gi=None):
    prob = _f32(prob)
    lab = np.ascontiguousarray(lab, np.int32)
    N, C = prob.shape
    gi = np.zeros_like(prob) if gi is None else _f32(gi).copy()
    lib().or_cross_entropy_bwd(c_int64(N), c_int64(C), _p(prob), _p(lab), c_float(gout), _p(gi))
    return gi


def nll_loss_fwd(x, lab, sum=False):
    x = _f32(x)
    lab = np.ascontiguousarray(lab, np.int32)
    N, C = x.shape
    loss = c_float(0.0)
    L = lib()
    L.or_nll_loss_fwd.restype = c_int64
    bad = L.or_nll_loss_fwd(c_int64(N), c_int64(C), _p(x), _p(lab), c_int(int(sum)), ctypes.byref(loss))
    if bad >= 0:
        raise ValueError(f"label {int(lab[bad])} at row {bad} outside [0, {C})")
    return np.float32(loss.value)


def nll_loss_bwd(shape, lab, gout, sum=False, gi=None):
    N, C = shape
    lab = np.ascontiguousarray(lab, np.int32)
    gi = np.zeros((N, C), np.float32) if gi is None else _f32(gi).copy()
    lib().or_nll_loss_bwd(c_int64(N), c_int64(C), _p(lab), c_float(gout), c_int(int(sum)), _p(gi))
    return gi


OPT = {"sgd": 0, "adam": 1, "adamw": 2, "rmsprop": 3}


def optim_step(kind, w, g, s1, s2, lr, momentum=0.0, weight_decay=0.0, beta1=0.0, beta2=0.0, eps=0.0, gs=1.0,
               bc1=1.0, bc2=1.0, eps_inside_sqrt=False):
    """One update in place on float32 arrays w, s1, s2 (s1 / s2 may be None); returns (w, s1, s2)."""
    from ctypes import c_double  # noqa: F401
    for a in (w, s1, s2):
        assert a is None or (a.dtype == np.float32 and a.flags.c_contiguous)
    g = _f32(g)
    lib().or_optim_step(c_int(OPT[kind]), c_int64(w.size), _p(w), _p(g), _p(s1), _p(s2), c_float(lr),
                        c_float(momentum), c_float(weight_decay), c_float(beta1), c_float(beta2), c_float(eps),
                        c_float(gs), c_float(bc1), c_float(bc2), c_int(int(eps_inside_sqrt)))
    return w, s1, s2


def sumsq(x):
    from ctypes import c_double
    L = lib()
    L.or_sumsq.restype = c_double
    x = _f32(x)
    return L.or_sumsq(c_int64(x.size), _p(x))


_libm = None


def powf(x, y):
    """glibc powf, as the reference computes Adam's bias corrections (optim.c:167-168)."""
    global _libm
    if _libm is None:
        _libm = ctypes.CDLL("libm.so.6")
        _libm.powf.restype = c_float
        _libm.powf.argtypes = [c_float, c_float]
    return np.float32(_libm.powf(float(x), float(y)))


def optim_defaults(ctor, opts, inside=None):
    """The constructors' defaults for zero hyperparameters (optim.c:101-124)."""
    lr, mom, wd, b1, b2, eps = (np.float32(v) for v in opts)
    if ctor in ("nc_adam", "nc_adamw"):
        b1 = b1 or np.float32(0.9)
        b2 = b2 or np.float32(0.999)
        eps = eps or np.float32(1e-8)
    elif ctor == "nc_rmsprop":
        b2 = b2 or np.float32(0.99)
        eps = eps or np.float32(1e-8)
    return lr, mom, wd, b1, b2, eps


def optim_replay(cfg, W, Gs):
    """The optimizer scenario of tests/golden/gen_golden.py on the oracle: per step, grads accumulate
    (zero_grad is skipped mid-accumulation), every accum-th call updates.  Returns the same keys."""
    name, ctor, opts, inside, accum, steps = cfg
    kind = {"nc_sgd": "sgd", "nc_adam": "adam", "nc_adamw": "adamw", "nc_rmsprop": "rmsprop"}[ctor]
    lr, mom, wd, b1, b2, eps = optim_defaults(ctor, opts, inside)
    w = [np.array(x, np.float32, copy=True) for x in W]
    adam = kind in ("adam", "adamw")
    s1 = [np.zeros_like(x) for x in w] if (adam or mom != 0) else [None] * len(w)
    s2 = [np.zeros_like(x) for x in w] if (adam or kind == "rmsprop") else [None] * len(w)
    grads = [np.zeros_like(x) for x in w]
    t, count, out = 0, 0, {}
    for k in range(steps):
        if count == 0:
            grads = [np.zeros_like(x) for x in w]
        grads = [g + np.asarray(G, np.float32) for g, G in zip(grads, Gs[k])]  # fp32 accumulation
        count += 1
        if not (accum > 1 and count < accum):
            count = 0
            t += 1
            gs = np.float32(1.0) / np.float32(accum)
            bc1 = np.float32(1.0) - powf(b1, np.float32(t)) if adam else np.float32(1.0)
            bc2 = np.float32(1.0) - powf(b2, np.float32(t)) if adam else np.float32(1.0)
            for i in range(len(w)):
                optim_step(kind, w[i], grads[i], s1[i], s2[i], lr, mom, wd, b1, b2, eps, gs, bc1, bc2,
                           bool(inside))
        for i in range(len(w)):
            out[f"{name}/step{k}/w{i}"] = w[i].copy()
            for slot, s in ((0, s1[i]), (1, s2[i])):
                if s is not None:
                    out[f"{name}/step{k}/s{slot}_{i}"] = s.copy()
    out[f"{name}/t"] = np.int64(t)
    return out


def clip_grad_norm(grads, max_norm):
    """(total, scaled grads) as nc_clip_grad_norm (optim.c:216-233): fp64 sum of squares in order."""
    ss = 0.0
    for g in grads:
        ss += sumsq(g)
    total = np.float32(np.sqrt(ss))
    coef = np.float32(max_norm) / (total + np.float32(1e-6))
    if coef < np.float32(1.0):
        grads = [(np.asarray(g, np.float32) * coef).astype(np.float32) for g in grads]
    return total, grads


# ---- int8 GEMM and linear_int8 (exact; C restatement) ------------------------------------------
def gemm_s8_nt(A, B):
    """C = A @ B^T in int32 for A [M, K], B [N, K] int8 (kernels_ref.c:117-128)."""
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    (M, K), N = A.shape, B.shape[0]
    C = np.empty((M, N), np.int32)
    lib().or_gemm_s8_nt(c_int64(M), c_int64(N), c_int64(K), _p(A), c_int64(K), _p(B), c_int64(K), _p(C),
                        c_int64(N))
    return C


def linear_int8(x, wq, ws, bias=None):
    """linear_int8 forward (ops_quant.c:72-113) for x [..., K]; returns y [..., N]."""
    x = _f32(x)
    wq = np.ascontiguousarray(wq, np.int8)
    N, K = wq.shape
    M = int(np.prod(x.shape[:-1]))
    y = np.empty(x.shape[:-1] + (N,), np.float32)
    lib().or_linear_int8(c_int64(M), c_int64(K), c_int64(N), _p(x), _p(wq), _p(_f32(ws)),
                         _p(None if bias is None else _f32(bias)), _p(y))
    return y


# ---- fp32 GEMM ops: fp64 truth ------------------------------------------------------------------
# The reference's fp32 GEMMs (kernels_avx2.c:182-303, split over threads by nc__gemm,
# threadpool.c:243-265) sum in an order that is theirs alone; the truth here is the exact product in
# fp64, and results (the reference's and the HIP path's) are held to
#     |y - y64| <= rtol * max(|y64|, T / sqrt(K)),   T = sum_k |a_k b_k|  (|A| @ |B| in fp64),
# the reductions' tolerance applied to a K-term dot product.
def sum_to_shape(x, shape):
    """Sums a broadcast result back to `shape` (numpy broadcasting rules)."""
    x = np.asarray(x)
    lead = x.ndim - len(shape)
    if lead:
        x = x.sum(axis=tuple(range(lead)))
    axes = tuple(i for i, s in enumerate(shape) if s == 1 and x.shape[i] != 1)
    if axes:
        x = x.sum(axis=axes, keepdims=True)
    return x.reshape(shape)


def matmul64(a, b):
    """Forward truth and term bound of matmul / bmm (ops_linalg.c:58-66, :220-234): numpy's
    broadcasting matmul has the reference's semantics ([..., M, K] @ [K, N] folds a's leading dims;
    3-D+ operands broadcast their batch dims)."""
    a64, b64 = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.matmul(a64, b64), np.matmul(np.abs(a64), np.abs(b64))


def matmul_grads64(a, b, G):
    """(ga, gb, ta, tb): gradients of sum(matmul(a, b) * G) (ops_linalg.c:68-85, :236-262) summed to
    the operands' shapes, and their term bounds."""
    a64, b64, G64 = (np.asarray(v, np.float64) for v in (a, b, G))
    bt, at = np.swapaxes(b64, -1, -2), np.swapaxes(a64, -1, -2)
    if b64.ndim == 2 and a64.ndim > 2:  # folded: a [..., M, K]
        M = a64.size // a64.shape[-1]
        a2, G2 = a64.reshape(M, -1), G64.reshape(M, -1)
        ga = (G2 @ b64.T).reshape(a64.shape)
        ta = (np.abs(G2) @ np.abs(b64.T)).reshape(a64.shape)
        gb, tb = a2.T @ G2, np.abs(a2.T) @ np.abs(G2)
        return ga, gb, ta, tb
    ga = sum_to_shape(np.matmul(G64, bt), a64.shape)
    ta = sum_to_shape(np.matmul(np.abs(G64), np.abs(bt)), a64.shape)
    gb = sum_to_shape(np.matmul(at, G64), b64.shape)
    tb = sum_to_shape(np.matmul(np.abs(at), np.abs(G64)), b64.shape)
    return ga, gb, ta, tb


def linear64(x, W, bias=None):
    """(y, t): y = x @ W^T + b (ops_linalg.c:296-306) in fp64 and its term bound."""
    x64, W64 = np.asarray(x, np.float64), np.asarray(W, np.float64)
    y, t = x64 @ W64.T, np.abs(x64) @ np.abs(W64.T)
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
        t = t + np.abs(np.asarray(bias, np.float64))
    return y, t


def linear_grads64(x, W, G):
    """(gx, gW, gb, tx, tW, tb): gradients of sum(linear(x, W, b) * G) (ops_linalg.c:308-330)."""
    x64, W64, G64 = (np.asarray(v, np.float64) for v in (x, W, G))
    N, K = W64.shape
    x2, G2 = x64.reshape(-1, K), G64.reshape(-1, N)
    gx = (G2 @ W64).reshape(x64.shape)
    tx = (np.abs(G2) @ np.abs(W64)).reshape(x64.shape)
    return gx, G2.T @ x2, G2.sum(0), tx, np.abs(G2.T) @ np.abs(x2), np.abs(G2).sum(0)


def gemm_excess(got, truth, terms, K, rtol=1e-5):
    """max over elements of |got - truth| / (rtol * max(|truth|, terms / sqrt(K))); <= 1 passes.

    terms / sqrt(K) is the scale of a K-term sum whose rounding errors cancel like a random walk.  A
    blocked fp32 sum (panels of 256 products summed from zero, each added into the running total, as
    the reference's KC = 256 panels at kernels_avx2.c:234-247) stays well inside it; an fp32 sum that
    adds one product at a time to the running total rounds K sums of size ~sqrt(K) terms, so its error
    grows like terms itself and leaves the bound past a few thousand terms."""
    got = np.asarray(got, np.float64)
    bound = rtol * np.maximum(np.abs(truth), np.asarray(terms) / np.sqrt(max(K, 1)))
    err = np.abs(got - truth)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(err == 0, 0.0, err / bound)  # a nonzero error on a zero bound is inf; NaN stays NaN
    r = np.where(np.isnan(r), np.inf, r)
    return float(r.max()) if r.size else 0.0
