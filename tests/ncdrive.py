"""Drives any library with the nc.h C ABI through ctypes, the way the reference's Python package
drives its engine (newch/tensor.py over newch/_lib.py).  The same driver runs the compiled reference
(oracle/_ref/libnc_ref.so) and the MI355X engine (newch_amd/libnc.so), so a test reads the same
for both."""

from __future__ import annotations

import ctypes
from ctypes import c_char_p, c_float, c_void_p

import numpy as np

from newch_amd import abi

NP_DTYPE = {abi.F32: np.float32, abi.I32: np.int32, abi.I8: np.int8, abi.U8: np.uint8}


class NcError(RuntimeError):
    pass


class Engine:
    def __init__(self, lib_path=None, seed: int = 1234, lib=None):
        self.lib = lib if lib is not None else abi.load(lib_path)
        cfg = abi.Config(0, seed, 0, 0)
        self.ctx = self.lib.nc_init(ctypes.byref(cfg))
        if not self.ctx:
            raise NcError("nc_init failed")

    # context management ------------------------------------------------------------------------
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def close(self):
        if self.ctx:
            self.lib.nc_free_ctx(self.ctx)
            self.ctx = None

    def check(self):
        if not self.lib.nc_ok(self.ctx):
            msg = self.lib.nc_error(self.ctx).decode()
            self.lib.nc_clear_error(self.ctx)
            raise NcError(msg)

    def step_end(self):
        self.lib.nc_step_end(self.ctx)

    # tensors ---------------------------------------------------------------------------------------
    def tensor(self, arr, dtype=None):
        arr = np.array(arr, order="C", copy=True)  # keeps 0-d shapes (ascontiguousarray would not)
        if dtype is None:
            dtype = {np.dtype(np.float32): abi.F32, np.dtype(np.int32): abi.I32, np.dtype(np.int8): abi.I8,
                     np.dtype(np.uint8): abi.U8}[arr.dtype]
        nd, shp = abi.shape_arg(arr.shape)
        t = self.lib.nc_from_data(self.ctx, dtype, arr.ctypes.data_as(c_void_p), nd, shp)
        self.check()
        return t

    def param(self, arr):
        arr = np.asarray(arr, np.float32)
        src = self.tensor(arr)
        nd, shp = abi.shape_arg(arr.shape)
        p = self.lib.nc_parameter(self.ctx, src, nd, shp)
        self.check()
        return p

    def shape(self, t):
        nd = self.lib.nc_ndim(t)
        sp = self.lib.nc_shape(t)
        return tuple(sp[i] for i in range(nd))

    def read(self, t):
        self.check()
        if not t:
            raise NcError("NULL tensor")
        dt = NP_DTYPE[self.lib.nc_get_dtype(t)]
        out = np.empty(self.lib.nc_numel(t), dtype=dt)
        if not self.lib.nc_copy_to(t, out.ctypes.data_as(c_void_p), out.nbytes):
            self.check()
            raise NcError("nc_copy_to failed")
        return out.reshape(self.shape(t))

    def view(self, storage_t, view):
        """view: None | ('t', a0, a1) | ('t_reshape', a0, a1, shape)"""
        if view is None:
            return storage_t
        v = self.lib.nc_transpose(storage_t, view[1], view[2])
        if view[0] == "t_reshape":
            nd, shp = abi.shape_arg(view[3])
            v = self.lib.nc_reshape(v, nd, shp)
        self.check()
        return v

    # autograd --------------------------------------------------------------------------------------
    def backward_with(self, out, G, flags=abi.BACKWARD_RETAIN):
        """loss = sum(out * G), then backward: the output grad is exactly G."""
        loss = self.lib.nc_sum(self.lib.nc_mul(out, self.tensor(np.asarray(G, np.float32))), abi.ALL_AXES, 0)
        self.check()
        if self.lib.nc_backward_ex(loss, flags, None, 0) != 0:
            self.check()

    def grad(self, t):
        g = self.lib.nc_grad(t)
        if not g:
            self.check()
            raise NcError("tensor has no grad")
        return self.read(g)

    # op helpers used by several tests ---------------------------------------------------------------
    UNARY_CALLS = {
        "relu": lambda L, t, s: L.nc_relu(t),
        "leaky_relu": lambda L, t, s: L.nc_leaky_relu(t, c_float(s)),
        "leaky_relu_02": lambda L, t, s: L.nc_leaky_relu(t, c_float(s)),
        "relu6": lambda L, t, s: L.nc_relu6(t),
        "hardsigmoid": lambda L, t, s: L.nc_hardsigmoid(t),
        "hardswish": lambda L, t, s: L.nc_hardswish(t),
        "silu": lambda L, t, s: L.nc_silu(t),
        "gelu": lambda L, t, s: L.nc_gelu(t, 0),
        "gelu_tanh": lambda L, t, s: L.nc_gelu(t, 1),
        "sigmoid": lambda L, t, s: L.nc_sigmoid(t),
        "tanh": lambda L, t, s: L.nc_tanh(t),
        "exp": lambda L, t, s: L.nc_exp(t),
        "neg": lambda L, t, s: L.nc_neg(t),
        "scale": lambda L, t, s: L.nc_scale(t, c_float(s)),
        "add_scalar": lambda L, t, s: L.nc_add_scalar(t, c_float(s)),
        "log": lambda L, t, s: L.nc_log(t),
        "sqrt": lambda L, t, s: L.nc_sqrt(t),
        "pow": lambda L, t, s: L.nc_pow_scalar(t, c_float(s)),
    }

    def unary(self, name, x, g, s=0.0):
        """(y, dL/dx) for y = f(x), dL/dy = g."""
        p = self.param(x)
        y = self.UNARY_CALLS[name](self.lib, p, s)
        yv = self.read(y)
        self.backward_with(y, g)
        gx = self.grad(p)
        self.step_end()
        return yv, gx


# ---- NCW1 files --------------------------------------------------------------------------------------
def io_tensors(e: "Engine", rng_seed: int = 0, big: int = 0):
    """A fixed set of named tensors built in engine `e`: f32 / i32 / i8 / u8, a 0-d scalar, an empty
    tensor, a transposed (strided) view, a parameter, and optionally one f32 tensor of `big` floats.
    Returns (names, tensors, numpy values in file order)."""
    rng = np.random.default_rng(rng_seed)
    L = e.lib
    vals = {
        "w": rng.standard_normal((3, 4)).astype(np.float32),
        "idx": np.arange(-2, 3, dtype=np.int32),
        "q": rng.integers(-127, 128, (2, 3)).astype(np.int8),
        "mask": rng.integers(0, 256, 7).astype(np.uint8),
        "scalar": np.array(2.5, np.float32),
        "empty": np.zeros((0, 3), np.float32),
    }
    names, tensors, arrays = [], [], []
    for k, v in vals.items():
        names.append(k)
        tensors.append(e.tensor(v))
        arrays.append(v)
    base = rng.standard_normal((4, 5)).astype(np.float32)
    names.append("w_t")
    tensors.append(L.nc_transpose(e.tensor(base), 0, 1))
    arrays.append(np.ascontiguousarray(base.T))
    p = rng.standard_normal(6).astype(np.float32)
    names.append("0.weight")
    tensors.append(e.param(p))
    arrays.append(p)
    if big:
        b = rng.standard_normal(big).astype(np.float32)
        names.append("big")
        tensors.append(e.tensor(b))
        arrays.append(b)
    e.check()
    return names, tensors, arrays


def io_save(e: "Engine", path, names, tensors):
    arr_n = (c_char_p * len(names))(*[n.encode() for n in names])
    arr_t = (c_void_p * len(tensors))(*tensors)
    return e.lib.nc_save(e.ctx, str(path).encode(), len(names), arr_n, arr_t)


def io_load(e: "Engine", path, names, tensors):
    arr_n = (c_char_p * len(names))(*[n.encode() for n in names])
    arr_t = (c_void_p * len(tensors))(*tensors)
    return e.lib.nc_load(e.ctx, str(path).encode(), len(names), arr_n, arr_t)
