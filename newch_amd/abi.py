"""ctypes view of the nc.h C ABI.

The engine library this package builds (``newch_amd/libnc.so``) exports the same C ABI as the
reference engine's ``libnc.so`` (``engine/include/nc.h``), so one signature table binds either of
them.  The table below covers every ``NC_API`` function of that header, which is a superset of the
111 names the reference's Python bindings resolve at import (``newch/_lib.py:78-177``), plus the
additive device functions this engine exports (``nc_device_*``, ``nc_set_stream``...), which are
bound only when present.

Struct layouts (``Config``, ``MemStats``, ``CpuInfo``, ``OptimOpts``) are frozen by that ABI:
``nc.h:78-83``, ``:109-114``, ``:123-133``, ``:372-376``.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, Structure, c_char_p, c_float, c_int, c_int64, c_size_t, c_uint64, c_void_p
from pathlib import Path

F32, I32, F16, I8, U8 = 0, 1, 2, 3, 4
ALL_AXES = -128
MAX_DIMS = 6
OK, ERR_SHAPE, ERR_DTYPE, ERR_OOM, ERR_ARG, ERR_STATE = range(6)
BACKWARD_FREE_GRAPH, BACKWARD_RETAIN = 1, 2


class Config(Structure):
    _fields_ = [("arena_chunk_bytes", c_size_t), ("seed", c_uint64), ("force_reference", c_int),
                ("threads", c_int)]


class MemStats(Structure):
    _fields_ = [("persistent_bytes", c_size_t), ("arena_bytes_in_use", c_size_t),
                ("arena_bytes_reserved", c_size_t), ("arena_peak_bytes", c_size_t)]


class CpuInfo(Structure):
    _fields_ = [("arch", c_char_p), ("has_neon", c_int), ("has_dotprod", c_int), ("has_fp16", c_int),
                ("has_avx2", c_int), ("has_fma", c_int), ("has_rvv", c_int), ("n_cores", c_int),
                ("n_big_cores", c_int)]


class OptimOpts(Structure):
    _fields_ = [(n, c_float) for n in ("lr", "momentum", "weight_decay", "beta1", "beta2", "eps")]


P = c_void_p
I64P = POINTER(c_int64)
PP = POINTER(c_void_p)

# name -> (restype, argtypes); every NC_API function of nc.h
NC_SIGNATURES: dict[str, tuple] = {
    # context
    "nc_init": (P, [POINTER(Config)]),
    "nc_free_ctx": (None, [P]),
    "nc_manual_seed": (None, [P, c_uint64]),
    "nc_step_end": (None, [P]),
    "nc_arena_trim": (None, [P]),
    "nc_num_threads": (c_int, [P]),
    "nc_persistent_begin": (None, [P]),
    "nc_persistent_end": (None, [P]),
    "nc_set_grad_enabled": (c_int, [P, c_int]),
    "nc_ok": (c_int, [P]),
    "nc_status_code": (c_int, [P]),
    "nc_error": (c_char_p, [P]),
    "nc_clear_error": (None, [P]),
    "nc_get_mem_stats": (MemStats, [P]),
    "nc_reset_peak": (None, [P]),
    "nc_cpu": (POINTER(CpuInfo), [P]),
    "nc_kernel_backend": (c_char_p, [P]),
    # tensors
    "nc_empty": (P, [P, c_int, c_int, I64P]),
    "nc_zeros": (P, [P, c_int, c_int, I64P]),
    "nc_full": (P, [P, c_float, c_int, I64P]),
    "nc_randn": (P, [P, c_float, c_int, I64P]),
    "nc_rand_uniform": (P, [P, c_float, c_float, c_int, I64P]),
    "nc_from_data": (P, [P, c_int, c_void_p, c_int, I64P]),
    "nc_scalar": (P, [P, c_float]),
    "nc_parameter": (P, [P, P, c_int, I64P]),
    "nc_ndim": (c_int, [P]),
    "nc_dim": (c_int64, [P, c_int]),
    "nc_shape": (I64P, [P]),
    "nc_numel": (c_int64, [P]),
    "nc_get_dtype": (c_int, [P]),
    "nc_is_contiguous": (c_int, [P]),
    "nc_requires_grad": (c_int, [P]),
    "nc_is_persistent": (c_int, [P]),
    "nc_release": (None, [P]),
    "nc_set_requires_grad": (None, [P, c_int]),
    "nc_grad": (P, [P]),
    "nc_set_name": (None, [P, c_char_p]),
    "nc_name": (c_char_p, [P]),
    "nc_data_f32": (c_void_p, [P]),
    "nc_data_i32": (c_void_p, [P]),
    "nc_item": (c_float, [P]),
    "nc_get": (c_float, [P, I64P]),
    "nc_copy_to": (c_int, [P, c_void_p, c_size_t]),
    "nc_copy_from": (c_int, [P, c_void_p, c_size_t]),
    "nc_print": (None, [P]),
    # ops
    **{f"nc_{n}": (P, [P, P]) for n in ("add", "sub", "mul", "div", "matmul", "cross_entropy", "mse_loss",
                                         "index_select")},
    **{f"nc_{n}": (P, [P]) for n in ("neg", "exp", "log", "sqrt", "relu", "sigmoid", "tanh", "contiguous",
                                      "log_softmax", "softmax", "detach", "relu6", "hardsigmoid", "hardswish",
                                      "silu")},
    **{f"nc_{n}": (P, [P, c_float]) for n in ("scale", "add_scalar", "pow_scalar", "leaky_relu", "dropout")},
    **{f"nc_{n}": (P, [P, c_int, c_int]) for n in ("sum", "mean", "max", "transpose")},
    "nc_gelu": (P, [P, c_int]),
    "nc_linear_fn": (P, [P, P, P]),
    "nc_reshape": (P, [P, c_int, I64P]),
    "nc_slice": (P, [P, c_int, c_int64, c_int64, c_int64]),
    "nc_conv2d": (P, [P, P, P, c_int, c_int, c_int, c_int]),
    "nc_conv2d_ex": (P, [P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "nc_max_pool2d": (P, [P, c_int, c_int, c_int, c_int, c_int, c_int]),
    "nc_avg_pool2d": (P, [P, c_int, c_int, c_int, c_int, c_int, c_int]),
    "nc_batch_norm": (P, [P, P, P, P, P, c_int, c_float, c_float]),
    "nc_layer_norm": (P, [P, c_int, P, P, c_float]),
    "nc_masked_fill": (P, [P, P, c_float]),
    "nc_nll_loss": (P, [P, P, c_int]),
    "nc_argmax": (P, [P, c_int]),
    "nc_compare": (P, [P, P, c_int]),
    "nc_cat": (P, [c_int, PP, c_int]),
    "nc_to_dtype": (P, [P, c_int]),
    "nc_quantize_rows": (P, [P, PP]),
    "nc_linear_int8": (P, [P, P, P, P]),
    # serialization
    "nc_save": (c_int, [P, c_char_p, c_int, POINTER(c_char_p), PP]),
    "nc_load": (c_int, [P, c_char_p, c_int, POINTER(c_char_p), PP]),
    # autograd
    "nc_backward": (c_int, [P]),
    "nc_backward_ex": (c_int, [P, c_int, PP, c_int]),
    "nc_release_temp": (None, [P]),
    "nc_zero_grad": (None, [P]),
    "nc_clear_grad": (None, [P]),
    "nc_gradcheck": (c_float, [P, c_void_p, PP, c_int, c_void_p, c_float]),
    # modules
    "nc_linear": (P, [P, c_int64, c_int64, c_int]),
    "nc_act": (P, [P, c_int]),
    "nc_sequential": (P, [P, c_int, PP]),
    "nc_forward": (P, [P, P]),
    "nc_parameters": (c_int, [P, PP, c_int]),
    "nc_module_name": (c_char_p, [P]),
    "nc_set_training": (None, [P, c_int]),
    # optimizers
    "nc_sgd": (P, [P, PP, c_int, OptimOpts]),
    "nc_adam": (P, [P, PP, c_int, OptimOpts]),
    "nc_adamw": (P, [P, PP, c_int, OptimOpts]),
    "nc_rmsprop": (P, [P, PP, c_int, OptimOpts, c_int]),
    "nc_optim_zero_grad": (None, [P]),
    "nc_optim_clear_grad": (None, [P]),
    "nc_optim_step": (None, [P]),
    "nc_optim_free": (None, [P]),
    "nc_optim_set_lr": (None, [P, c_float]),
    "nc_optim_state": (c_void_p, [P, c_int, c_int]),
    "nc_optim_get_step": (c_int64, [P]),
    "nc_optim_set_step": (None, [P, c_int64]),
    "nc_optim_set_opts": (None, [P, OptimOpts]),
    "nc_optim_set_accumulation": (None, [P, c_int]),
    "nc_clip_grad_norm": (c_float, [PP, c_int, c_float]),
}

# Additive functions of this engine (not in the reference ABI): device selection, stream hand-over,
# synchronisation, device pointers of tensors.  Declared in include/nc.h under "device extensions".
NC_DEVICE_SIGNATURES: dict[str, tuple] = {
    "nc_device_count": (c_int, []),
    "nc_set_device": (c_int, [P, c_int]),
    "nc_get_device": (c_int, [P]),
    "nc_set_stream": (None, [P, c_void_p]),
    "nc_get_stream": (c_void_p, [P]),
    "nc_synchronize": (c_int, [P]),
    "nc_device_ptr": (c_void_p, [P]),
    "nc_from_device": (P, [P, c_int, c_void_p, c_int, I64P]),
    "nc_device_alloc_count": (c_uint64, [P]),
}


def bind(lib: ctypes.CDLL, strict: bool = True) -> ctypes.CDLL:
    """Sets restype/argtypes for every nc.h function (raises AttributeError on a missing one when
    strict) and for the device extensions the library has."""
    for name, (res, args) in NC_SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError:
            if strict:
                raise
            continue
        fn.restype, fn.argtypes = res, args
    for name, (res, args) in NC_DEVICE_SIGNATURES.items():
        if hasattr(lib, name):
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
    return lib


def shape_arg(shape) -> tuple[int, ctypes.Array]:
    shape = tuple(int(s) for s in shape)
    return len(shape), (c_int64 * max(len(shape), 1))(*shape)


def ptr_array(ptrs) -> ctypes.Array:
    ptrs = list(ptrs)
    return (c_void_p * max(len(ptrs), 1))(*ptrs)


PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libnc.so"


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Loads and binds an nc.h library: `path`, else $NEWCH_LIB, else this package's libnc.so."""
    path = path or os.environ.get("NEWCH_LIB") or LIB_PATH
    if not Path(path).exists():
        raise OSError(f"nc library not found at {path}: build it with `python -m newch_amd.build`")
    return bind(ctypes.CDLL(str(path)))
