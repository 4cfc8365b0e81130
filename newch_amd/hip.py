"""ctypes binding of the nc_hip.h kernel layer (exported by newch_amd/libnc.so).

The functions take raw device addresses, element counts/strides and a hipStream_t.  `Kernels`
wraps them for callers that hold device buffers (``newch_amd.hipmem.DeviceBuffer`` in the tests and
the benchmark; any device address on the same HIP runtime works): pointers are plain integers and
``stream=None`` is the null stream.  Every wrapper raises ``HipLayerError`` with the library's
message when a call returns an error code; nothing here falls back to the host.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_size_t, c_uint32, c_uint64, c_void_p

from . import abi

UN = {"relu": 0, "leaky_relu": 1, "relu6": 2, "hardsigmoid": 3, "hardswish": 4, "silu": 5, "gelu": 6,
      "gelu_tanh": 7, "sigmoid": 8, "tanh": 9, "exp": 10, "neg": 11, "scale": 12, "add_scalar": 13, "log": 14,
      "sqrt": 15, "pow": 16}
BIN = {"add": 0, "sub": 1, "mul": 2, "div": 3}
RED = {"sum": 0, "mean": 1, "max": 2, "argmax": 3}
OPT = {"sgd": 0, "adam": 1, "adamw": 2, "rmsprop": 3}
# which tensor an activation's backward reads besides g
BWD_READS_Y = {"sigmoid", "tanh", "exp", "sqrt"}
BWD_READS_NONE = {"neg", "scale", "add_scalar"}

P = c_void_p
I64P = POINTER(c_int64)


class OptParam(ctypes.Structure):
    """nc_hip_opt_param: one parameter of nc_hip_optim_step_multi."""
    _fields_ = [("w", c_void_p), ("g", c_void_p), ("s1", c_void_p), ("s2", c_void_p), ("n", c_int64)]

SIGNATURES = {
    "nc_hip_last_error": (c_char_p, []),
    "nc_hip_device_count": (c_int, []),
    "nc_hip_check_intdiv": (c_uint64, [POINTER(c_uint32), c_int, POINTER(c_uint32), c_int]),
    "nc_hip_set_grid_cus": (None, [c_int]),
    "nc_hip_unary_fwd": (c_int, [c_int, c_float, P, P, c_int64, P]),
    "nc_hip_unary_bwd": (c_int, [c_int, c_float, P, P, P, P, c_int64, c_int, P]),
    "nc_hip_binary_fwd": (c_int, [c_int, c_int, I64P, P, I64P, P, I64P, P, I64P, P]),
    "nc_hip_binary_bwd_workspace": (c_size_t, [c_int, I64P, I64P]),
    "nc_hip_binary_bwd": (c_int, [c_int, c_int, c_int, I64P, P, I64P, P, I64P, P, I64P, P, I64P, c_int, P, c_size_t, P]),
    "nc_hip_binary_bwd2_workspace": (c_size_t, [c_int, I64P, I64P, I64P]),
    "nc_hip_binary_bwd2": (c_int, [c_int, c_int, I64P, P, I64P, P, I64P, P, I64P, P, I64P, P, I64P, c_int, P,
                                   c_size_t, P]),
    "nc_hip_copy_strided": (c_int, [c_int, c_int, I64P, P, I64P, P, P]),
    "nc_hip_accumulate_strided": (c_int, [c_int, I64P, P, P, I64P, P]),
    "nc_hip_axpy": (c_int, [c_int64, c_float, P, P, P]),
    "nc_hip_fill": (c_int, [P, c_int, c_uint64, c_int64, P]),
    "nc_hip_convert": (c_int, [c_int, c_int, c_int64, P, P, P]),
    "nc_hip_add_scalar_at": (c_int, [P, c_float, P]),
    "nc_hip_reduce_workspace": (c_size_t, [c_int, c_int64, c_int64, c_int64]),
    "nc_hip_reduce_fwd": (c_int, [c_int, c_int64, c_int64, c_int64, P, P, P, P, c_size_t, P]),
    "nc_hip_reduce_bwd": (c_int, [c_int, c_int64, c_int64, c_int64, P, P, P, c_int, P]),
    "nc_hip_reduce_sum_i32": (c_int, [c_int64, c_int64, c_int64, P, P, P]),
    "nc_hip_softmax_fwd": (c_int, [c_int, c_int64, c_int64, P, P, P]),
    "nc_hip_softmax_bwd": (c_int, [c_int, c_int64, c_int64, P, P, P, c_int, P]),
    "nc_hip_layer_norm_fwd": (c_int, [c_int64, c_int64, P, P, P, c_float, P, P, P]),
    "nc_hip_layer_norm_bwd_workspace": (c_size_t, [c_int64, c_int64]),
    "nc_hip_layer_norm_bwd": (c_int, [c_int64, c_int64, P, P, P, P, P, P, P, c_int, P, c_size_t, P]),
    "nc_hip_quantize_rows": (c_int, [c_int64, c_int64, P, P, P, P]),
    "nc_hip_dequantize_rows": (c_int, [c_int64, c_int64, P, P, P, P]),
    "nc_hip_optim_step": (c_int, [c_int, c_int64, P, P, P, P, c_float, c_float, c_float, c_float, c_float, c_float,
                                  c_float, c_float, c_float, c_int, P]),
    "nc_hip_optim_step_multi": (c_int, [c_int, c_int, P, c_float, c_float, c_float, c_float, c_float, c_float,
                                        c_float, c_float, c_float, c_int, P]),
    "nc_hip_sumsq_workspace": (c_size_t, [c_int64]),
    "nc_hip_sumsq": (c_int, [c_int64, P, P, c_int, P, c_size_t, P]),
    "nc_hip_sumsq_multi_workspace": (c_size_t, [c_int, P]),
    "nc_hip_sumsq_multi": (c_int, [c_int, P, P, P, c_int, P, c_size_t, P]),
    "nc_hip_scale_multi": (c_int, [c_int, P, P, c_float, P]),
    "nc_hip_loss_workspace": (c_size_t, [c_int64, c_int64]),
    "nc_hip_cross_entropy_fwd": (c_int, [c_int64, c_int64, P, P, P, P, P, P, c_size_t, P]),
    "nc_hip_cross_entropy_bwd": (c_int, [c_int64, c_int64, P, P, P, P, P, c_int, P]),
    "nc_hip_nll_loss_fwd": (c_int, [c_int64, c_int64, P, P, c_int, P, P, P, c_size_t, P]),
    "nc_hip_nll_loss_bwd": (c_int, [c_int64, c_int64, P, P, c_int, P, P]),
    "nc_hip_gemm_f32": (c_int, [c_int, c_int, c_int64, c_int64, c_int64, c_float, P, c_int64, P, c_int64, c_float, P,
                                c_int64, P]),
    "nc_hip_gemm_f32_bias": (c_int, [c_int, c_int, c_int64, c_int64, c_int64, c_float, P, c_int64, P, c_int64, P, P,
                                     c_int64, P]),
    "nc_hip_gemm_f32_batched": (c_int, [c_int, c_int, c_int64, c_int64, c_int64, c_float, P, c_int64, P, c_int64,
                                        c_float, P, c_int64, c_int64, P]),
    "nc_hip_gemm_f32_bmm_workspace": (c_size_t, [c_int64]),
    "nc_hip_gemm_f32_bmm": (c_int, [c_int, c_int, c_int64, c_int64, c_int64, P, c_int64, P, c_int64, c_float, P,
                                    c_int64, c_int, I64P, I64P, I64P, I64P, P, c_size_t, P]),
    "nc_hip_gemm_s8_nt": (c_int, [c_int64, c_int64, c_int64, P, c_int64, P, c_int64, P, c_int64, P]),
    "nc_hip_linear_int8_workspace": (c_size_t, [c_int64, c_int64]),
    "nc_hip_linear_int8": (c_int, [c_int64, c_int64, c_int64, P, P, P, P, P, P, c_size_t, P]),
}


class HipLayerError(RuntimeError):
    pass


def bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


def _i64(v):
    v = [int(x) for x in v]
    return (c_int64 * max(len(v), 1))(*v)


class Kernels:
    """Thin checked wrappers; every pointer argument is an int device address (or None)."""

    def __init__(self, lib: ctypes.CDLL | None = None):
        self.lib = bind(lib if lib is not None else ctypes.CDLL(str(abi.LIB_PATH)))

    def _ok(self, rc: int, what: str):
        if rc != 0:
            raise HipLayerError(f"{what}: {self.lib.nc_hip_last_error().decode()} (code {rc})")

    def set_grid_cus(self, n):
        """Grids of grid-stride kernels sized for n CUs (0: the device's own count); results must not
        change."""
        self.lib.nc_hip_set_grid_cus(int(n))

    def unary_fwd(self, kind, x, y, n, s=0.0, stream=None):
        self._ok(self.lib.nc_hip_unary_fwd(UN[kind], s, x, y, n, stream), "unary_fwd")

    def unary_bwd(self, kind, x, y, g, gi, n, s=0.0, accumulate=True, stream=None):
        self._ok(self.lib.nc_hip_unary_bwd(UN[kind], s, x, y, g, gi, n, int(accumulate), stream), "unary_bwd")

    def binary_fwd(self, op, shape, a, sa, b, sb, o, so, stream=None):
        self._ok(self.lib.nc_hip_binary_fwd(BIN[op], len(shape), _i64(shape), a, _i64(sa), b, _i64(sb), o, _i64(so),
                                            stream), "binary_fwd")

    def binary_bwd_workspace(self, shape, sgx):
        return self.lib.nc_hip_binary_bwd_workspace(len(shape), _i64(shape), _i64(sgx))

    def binary_bwd(self, op, which, shape, g, sg, a, sa, b, sb, gx, sgx, ws=None, ws_bytes=0, accumulate=True,
                   stream=None):
        self._ok(self.lib.nc_hip_binary_bwd(BIN[op], which, len(shape), _i64(shape), g, _i64(sg), a, _i64(sa), b,
                                            _i64(sb), gx, _i64(sgx), int(accumulate), ws, ws_bytes, stream),
                 "binary_bwd")

    def binary_bwd2_workspace(self, shape, sga, sgb):
        return self.lib.nc_hip_binary_bwd2_workspace(len(shape), _i64(shape), _i64(sga), _i64(sgb))

    def binary_bwd2(self, op, shape, g, sg, a, sa, b, sb, ga, sga, gb, sgb, ws=None, ws_bytes=0, accumulate=True,
                    stream=None):
        self._ok(self.lib.nc_hip_binary_bwd2(BIN[op], len(shape), _i64(shape), g, _i64(sg), a, _i64(sa), b, _i64(sb),
                                             ga, _i64(sga), gb, _i64(sgb), int(accumulate), ws, ws_bytes, stream),
                 "binary_bwd2")

    def fill(self, dst, elem_bytes, pattern, n, stream=None):
        self._ok(self.lib.nc_hip_fill(dst, elem_bytes, pattern, n, stream), "fill")

    def copy_strided(self, elem_bytes, shape, src, ss, dst, stream=None):
        self._ok(self.lib.nc_hip_copy_strided(elem_bytes, len(shape), _i64(shape), src, _i64(ss), dst, stream),
                 "copy_strided")

    def reduce_workspace(self, kind, outer, R, inner):
        return self.lib.nc_hip_reduce_workspace(RED[kind], outer, R, inner)

    def reduce_fwd(self, kind, outer, R, inner, x, y, arg, ws=None, ws_bytes=0, stream=None):
        self._ok(self.lib.nc_hip_reduce_fwd(RED[kind], outer, R, inner, x, y, arg, ws, ws_bytes, stream), "reduce_fwd")

    def reduce_bwd(self, kind, outer, R, inner, g, arg, gi, accumulate=True, stream=None):
        self._ok(self.lib.nc_hip_reduce_bwd(RED[kind], outer, R, inner, g, arg, gi, int(accumulate), stream),
                 "reduce_bwd")

    def softmax_fwd(self, log_form, rows, C, x, y, stream=None):
        self._ok(self.lib.nc_hip_softmax_fwd(int(log_form), rows, C, x, y, stream), "softmax_fwd")

    def softmax_bwd(self, log_form, rows, C, y, g, gi, accumulate=True, stream=None):
        self._ok(self.lib.nc_hip_softmax_bwd(int(log_form), rows, C, y, g, gi, int(accumulate), stream), "softmax_bwd")

    def layer_norm_fwd(self, rows, D, x, w, b, eps, y, stats, stream=None):
        self._ok(self.lib.nc_hip_layer_norm_fwd(rows, D, x, w, b, eps, y, stats, stream), "layer_norm_fwd")

    def layer_norm_bwd_workspace(self, rows, D):
        return self.lib.nc_hip_layer_norm_bwd_workspace(rows, D)

    def layer_norm_bwd(self, rows, D, x, w, stats, g, gx, gw, gb, ws=None, ws_bytes=0, accumulate=True,
                       stream=None):
        self._ok(self.lib.nc_hip_layer_norm_bwd(rows, D, x, w, stats, g, gx, gw, gb, int(accumulate), ws, ws_bytes,
                                                stream), "layer_norm_bwd")

    def quantize_rows(self, rows, cols, w, q, scale, stream=None):
        self._ok(self.lib.nc_hip_quantize_rows(rows, cols, w, q, scale, stream), "quantize_rows")

    def optim_step(self, kind, n, w, g, s1, s2, lr, momentum=0.0, weight_decay=0.0, beta1=0.0, beta2=0.0, eps=0.0,
                   gs=1.0, bc1=1.0, bc2=1.0, eps_inside_sqrt=False, stream=None):
        self._ok(self.lib.nc_hip_optim_step(OPT[kind], n, w, g, s1, s2, lr, momentum, weight_decay, beta1, beta2, eps,
                                            gs, bc1, bc2, int(eps_inside_sqrt), stream), "optim_step")

    def optim_step_multi(self, kind, params, lr, momentum=0.0, weight_decay=0.0, beta1=0.0, beta2=0.0, eps=0.0,
                         gs=1.0, bc1=1.0, bc2=1.0, eps_inside_sqrt=False, stream=None):
        """params: (w, g, s1, s2, n) per parameter (device addresses; s1 / s2 None when absent)."""
        arr = (OptParam * max(len(params), 1))()
        for i, (w, g, s1, s2, n) in enumerate(params):
            arr[i] = OptParam(w, g, s1, s2, n)
        self._ok(self.lib.nc_hip_optim_step_multi(OPT[kind], len(params), ctypes.addressof(arr), lr, momentum,
                                                  weight_decay, beta1, beta2, eps, gs, bc1, bc2,
                                                  int(eps_inside_sqrt), stream), "optim_step_multi")

    def sumsq_workspace(self, n):
        return self.lib.nc_hip_sumsq_workspace(n)

    def sumsq(self, n, x, ss, accumulate, ws, ws_bytes, stream=None):
        self._ok(self.lib.nc_hip_sumsq(n, x, ss, int(accumulate), ws, ws_bytes, stream), "sumsq")

    @staticmethod
    def _tables(tensors):
        k = max(len(tensors), 1)
        ptrs, ns = (ctypes.c_void_p * k)(), (ctypes.c_int64 * k)()
        for i, (x, n) in enumerate(tensors):
            ptrs[i], ns[i] = x, n
        return ptrs, ns

    def sumsq_multi_workspace(self, sizes):
        ns = (ctypes.c_int64 * max(len(sizes), 1))(*sizes)
        return self.lib.nc_hip_sumsq_multi_workspace(len(sizes), ctypes.addressof(ns))

    def sumsq_multi(self, tensors, ss, accumulate, ws, ws_bytes, stream=None):
        """tensors: (device address, n) per tensor."""
        ptrs, ns = self._tables(tensors)
        self._ok(self.lib.nc_hip_sumsq_multi(len(tensors), ctypes.addressof(ptrs), ctypes.addressof(ns), ss,
                                             int(accumulate), ws, ws_bytes, stream), "sumsq_multi")

    def scale_multi(self, tensors, coef, stream=None):
        ptrs, ns = self._tables(tensors)
        self._ok(self.lib.nc_hip_scale_multi(len(tensors), ctypes.addressof(ptrs), ctypes.addressof(ns), coef,
                                             stream), "scale_multi")

    def loss_workspace(self, N, C):
        return self.lib.nc_hip_loss_workspace(N, C)

    def cross_entropy_fwd(self, N, C, x, lab, stats, loss, bad, ws, ws_bytes, stream=None):
        """stats: [N][2] floats {row max, log-sum-exp} for the backward."""
        self._ok(self.lib.nc_hip_cross_entropy_fwd(N, C, x, lab, stats, loss, bad, ws, ws_bytes, stream),
                 "cross_entropy_fwd")

    def cross_entropy_bwd(self, N, C, x, stats, lab, gout, gi, accumulate=True, stream=None):
        self._ok(self.lib.nc_hip_cross_entropy_bwd(N, C, x, stats, lab, gout, gi, int(accumulate), stream),
                 "cross_entropy_bwd")

    def nll_loss_fwd(self, N, C, x, lab, sum, loss, bad, ws, ws_bytes, stream=None):
        self._ok(self.lib.nc_hip_nll_loss_fwd(N, C, x, lab, int(sum), loss, bad, ws, ws_bytes, stream),
                 "nll_loss_fwd")

    def nll_loss_bwd(self, N, C, lab, gout, sum, gi, stream=None):
        self._ok(self.lib.nc_hip_nll_loss_bwd(N, C, lab, gout, int(sum), gi, stream), "nll_loss_bwd")

    def dequantize_rows(self, rows, cols, q, scale, w, stream=None):
        self._ok(self.lib.nc_hip_dequantize_rows(rows, cols, q, scale, w, stream), "dequantize_rows")

    def gemm_f32(self, ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stream=None):
        self._ok(self.lib.nc_hip_gemm_f32(int(ta), int(tb), M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stream),
                 "gemm_f32")

    def gemm_f32_bias(self, ta, tb, M, N, K, alpha, A, lda, B, ldb, bias, C, ldc, stream=None):
        self._ok(self.lib.nc_hip_gemm_f32_bias(int(ta), int(tb), M, N, K, alpha, A, lda, B, ldb, bias, C, ldc, stream),
                 "gemm_f32_bias")

    def gemm_f32_batched(self, ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, count, stream=None):
        self._ok(self.lib.nc_hip_gemm_f32_batched(int(ta), int(tb), M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, count,
                                                  stream), "gemm_f32_batched")

    def gemm_f32_bmm_workspace(self, count):
        return self.lib.nc_hip_gemm_f32_bmm_workspace(count)

    def gemm_f32_bmm(self, ta, tb, M, N, K, A, lda, B, ldb, beta, C, ldc, bshape, sa, sb, sc, ws=None, ws_bytes=0,
                     stream=None):
        self._ok(self.lib.nc_hip_gemm_f32_bmm(int(ta), int(tb), M, N, K, A, lda, B, ldb, beta, C, ldc, len(bshape),
                                              _i64(bshape), _i64(sa), _i64(sb), _i64(sc), ws, ws_bytes, stream),
                 "gemm_f32_bmm")

    def gemm_s8_nt(self, M, N, K, A, lda, B, ldb, C, ldc, stream=None):
        self._ok(self.lib.nc_hip_gemm_s8_nt(M, N, K, A, lda, B, ldb, C, ldc, stream), "gemm_s8_nt")

    def linear_int8_workspace(self, M, K):
        return self.lib.nc_hip_linear_int8_workspace(M, K)

    def linear_int8(self, M, K, N, x, wq, wscale, bias, y, ws, ws_bytes, stream=None):
        self._ok(self.lib.nc_hip_linear_int8(M, K, N, x, wq, wscale, bias, y, ws, ws_bytes, stream), "linear_int8")
