"""Engine state on the device: lazily zeroed gradients, residency of views, device selection, the
device step arena's steady state and its debug poison.  Everything goes through the nc.h C ABI.

The reference's contracts pinned here:
  * nc_zero_grad zero-fills the gradient (engine/src/autograd/autograd.c:187-190), so a copy into it,
    a view of it and an optimizer step after it all see plain memory;
  * nc_load writes the named tensors' bytes and nothing else (engine/src/io/io.c:120-167);
  * NC_DEBUG_POISON=1 fills released memory with 0xCD (engine/src/core/ctx.c:41-56), and the
    reference's CI runs every test that way;
  * a steady-state step allocates nothing new: the arena keeps its chunks and its large blocks within
    the peak budget (ctx.c:113-149, 320-339).
The device selection (NC_DEVICE, nc_set_device) is this engine's additive contract (include/nc.h).
"""

import ctypes
import math
import os
from ctypes import c_float, c_void_p

import numpy as np
import pytest

from newch_amd import abi
from tests.ncdrive import Engine, io_load, io_save
from tests.test_gpu_parity import assert_bits, assert_close64, bcast_strides, dev, empty, strides_of, sync

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    L = abi.load(abi.LIB_PATH)
    assert L.nc_device_count() > 0, "no HIP device visible: the GPU tests need an MI355X"
    return L


@pytest.fixture()
def eng(lib):
    e = Engine(lib=lib)
    yield e
    e.close()


def fresh_grad(eng, shape, seed):
    """A parameter whose gradient buffer exists, then lazily zeroed by nc_zero_grad."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal(shape).astype(np.float32)
    g = rng.standard_normal(shape).astype(np.float32)
    p = eng.param(w)
    L = eng.lib
    assert L.nc_backward(L.nc_sum(L.nc_mul(p, eng.tensor(g)), abi.ALL_AXES, 0)) == 0
    assert_bits(eng.grad(p), g, "grad before zero_grad")
    L.nc_zero_grad(p)
    return p, w


def test_copy_into_zeroed_grad_is_kept(eng):
    """zero_grad, then the caller's values copied into p.grad: reads, the clip norm and an SGD step
    all use the copied values (a lazily zeroed buffer must not wipe them afterwards)."""
    L = eng.lib
    p, w = fresh_grad(eng, (37, 11), 1)
    v = np.random.default_rng(2).standard_normal((37, 11)).astype(np.float32)
    G = L.nc_grad(p)
    assert L.nc_copy_from(G, v.ctypes.data_as(c_void_p), v.nbytes) == 1
    assert_bits(eng.read(G), v, "grad after copy_from")
    params = (c_void_p * 1)(p)
    norm = L.nc_clip_grad_norm(params, 1, c_float(1e30))
    exact = math.sqrt(float(np.sum(v.astype(np.float64) ** 2)))
    assert abs(norm - exact) <= 1e-6 * exact, (norm, exact)
    o = L.nc_sgd(eng.ctx, params, 1, abi.OptimOpts(0.5, 0, 0, 0, 0, 0))
    L.nc_optim_step(o)
    eng.check()
    assert_bits(eng.read(p), (w - np.float32(0.5) * v).astype(np.float32), "sgd step on copied grad")
    L.nc_optim_free(o)
    eng.step_end()


def test_views_of_zeroed_grad_read_zeros(eng):
    """A transpose, reshape or slice of a lazily zeroed gradient reads zeros, not the previous step's
    values; a partial copy into a slice keeps zeros around it."""
    L = eng.lib
    p, _ = fresh_grad(eng, (6, 8), 3)
    G = L.nc_grad(p)
    assert_bits(eng.read(L.nc_transpose(G, 0, 1)), np.zeros((8, 6), np.float32), "transpose of zeroed grad")
    nd, shp = abi.shape_arg((48,))
    assert_bits(eng.read(L.nc_reshape(G, nd, shp)), np.zeros(48, np.float32), "reshape of zeroed grad")
    p2, _ = fresh_grad(eng, (6, 8), 4)
    G2 = L.nc_grad(p2)
    rows = L.nc_slice(G2, 0, 2, 2, 1)  # rows 2..3: a contiguous view of part of the storage
    v = np.full((2, 8), 5.0, np.float32)
    assert L.nc_copy_from(rows, v.ctypes.data_as(c_void_p), v.nbytes) == 1
    want = np.zeros((6, 8), np.float32)
    want[2:4] = 5.0
    assert_bits(eng.read(G2), want, "partial copy into a zeroed grad")
    eng.step_end()


def test_load_into_view_keeps_host_writes(eng, tmp_path):
    """nc_load into a contiguous row slice of a tensor whose host copy is authoritative (written
    through nc_data_f32): the loaded rows change, the other rows keep the host writes."""
    L = eng.lib
    src = eng.tensor(np.full((2, 16), 9.0, np.float32))
    assert io_save(eng, tmp_path / "rows.ncw", ["rows"], [src]) == 0, L.nc_error(eng.ctx)
    L.nc_persistent_begin(eng.ctx)
    t = L.nc_zeros(eng.ctx, abi.F32, *abi.shape_arg((8, 16)))
    L.nc_persistent_end(eng.ctx)
    host = ctypes.cast(L.nc_data_f32(t), ctypes.POINTER(ctypes.c_float))
    base = np.arange(128, dtype=np.float32).reshape(8, 16)
    for i in range(128):
        host[i] = float(base.flat[i])
    view = L.nc_slice(t, 0, 2, 2, 1)
    assert io_load(eng, tmp_path / "rows.ncw", ["rows"], [view]) == 0, L.nc_error(eng.ctx)
    want = base.copy()
    want[2:4] = 9.0
    assert_bits(eng.read(t), want, "tensor after loading a row slice")
    L.nc_release(t)
    eng.step_end()


def test_fused_div_grad_with_subnormal_divisor():
    """Fused broadcast backward of a / b with nonzero subnormal entries in b: 1/b overflows there, so
    grad_a must come from g / b (finite, as the reference's row_acc_div, ops_elementwise.c:43-46)."""
    from newch_amd.hip import Kernels
    K = Kernels()
    rng = np.random.default_rng(11)
    P, H, W = 40, 512, 64
    A = rng.standard_normal((P, 1, W)).astype(np.float32)
    B = (0.5 + rng.random((1, H, W))).astype(np.float32)
    G = rng.standard_normal((P, H, W)).astype(np.float32)
    tiny = rng.random((H, W)) < 0.01
    B[0][tiny] = (rng.uniform(1.5e-39, 3e-39, int(tiny.sum()))).astype(np.float32)
    G[:, tiny] *= np.float32(1e-3)  # keeps g / b finite in fp32
    shape = (P, H, W)
    sa, sb = bcast_strides(A.shape, strides_of(A), shape), bcast_strides(B.shape, strides_of(B), shape)
    so = strides_of(np.empty(shape, np.float32))
    Ad, Bd, Gd = dev(A), dev(B), dev(G)
    wsb = K.binary_bwd2_workspace(shape, sa, sb)
    ws = empty(max(wsb, 8))
    GA, GB = dev(np.zeros(A.shape, np.float32)), dev(np.zeros(B.shape, np.float32))
    K.binary_bwd2("div", shape, Gd.ptr, so, Ad.ptr, sa, Bd.ptr, sb, GA.ptr, sa, GB.ptr, sb, ws.ptr, wsb,
                  accumulate=False)
    sync()
    got = GA.to_numpy(np.float32, A.shape)
    terms = (G / B).astype(np.float32).astype(np.float64)  # the reference's fp32 g / b
    assert np.isfinite(terms).all()
    ref = terms.sum(axis=1, keepdims=True)
    assert_close64(got, ref, np.abs(terms).sum(axis=1, keepdims=True) / math.sqrt(H), "grad_a with subnormal b")


def test_device_selection(lib):
    """NC_DEVICE ("hip:N" or "N") picks the context's device at nc_init; a device out of range is
    NC_ERR_ARG; nc_set_device works on an empty context and is refused once it holds a tensor."""
    n = lib.nc_device_count()
    old = os.environ.get("NC_DEVICE")
    try:
        for val in ("hip:0", "0", None):
            if val is None:
                os.environ.pop("NC_DEVICE", None)
            else:
                os.environ["NC_DEVICE"] = val
            with Engine(lib=lib) as e:
                assert lib.nc_ok(e.ctx), lib.nc_error(e.ctx)
                assert lib.nc_get_device(e.ctx) == 0
                assert lib.nc_kernel_backend(e.ctx).startswith(b"hip:gfx9")
                assert_bits(e.read(lib.nc_relu(e.tensor(np.array([-1.0, 2.0], np.float32)))),
                            np.array([0.0, 2.0], np.float32), f"relu on NC_DEVICE={val}")
        os.environ["NC_DEVICE"] = f"hip:{n}"
        with Engine(lib=lib) as e:
            assert lib.nc_status_code(e.ctx) == abi.ERR_ARG
            assert b"out of range" in lib.nc_error(e.ctx)
    finally:
        if old is None:
            os.environ.pop("NC_DEVICE", None)
        else:
            os.environ["NC_DEVICE"] = old
    with Engine(lib=lib) as e:
        assert lib.nc_set_device(e.ctx, 0) == 1 and lib.nc_get_device(e.ctx) == 0
        assert lib.nc_set_device(e.ctx, n) == 0 and lib.nc_status_code(e.ctx) == abi.ERR_ARG
        lib.nc_clear_error(e.ctx)
        e.tensor(np.zeros(4, np.float32))
        assert lib.nc_set_device(e.ctx, 0) == 0
        assert lib.nc_status_code(e.ctx) == abi.ERR_STATE
        assert b"already holds tensors" in lib.nc_error(e.ctx)


def chain_step(e, px, pb, G):
    """The MNIST-CNN-shaped chain of the configuration: bias add, ReLU, sum over dims 3 then 2,
    backward against a fixed output gradient, zero_grad, step_end."""
    L = e.lib
    h = L.nc_relu(L.nc_add(px, pb))
    s = L.nc_sum(L.nc_sum(h, 3, 0), 2, 0)
    loss = L.nc_sum(L.nc_mul(s, e.tensor(G)), abi.ALL_AXES, 0)
    assert L.nc_backward(loss) == 0, L.nc_error(e.ctx)
    L.nc_zero_grad(px)
    L.nc_zero_grad(pb)
    e.step_end()
    e.check()


def test_arena_steady_state(lib):
    """After two warm steps the chain allocates nothing: reserved arena bytes and the context's
    hipMalloc count stay constant over ten more steps, and nothing is in use between steps."""
    rng = np.random.default_rng(0)
    with Engine(lib=lib) as e:
        px = e.param(rng.uniform(-1, 1, (64, 16, 28, 28)).astype(np.float32))
        pb = e.param(rng.uniform(-0.1, 0.1, (1, 16, 1, 1)).astype(np.float32))
        G = rng.standard_normal((64, 16)).astype(np.float32)
        for _ in range(2):
            chain_step(e, px, pb, G)
        st0 = lib.nc_get_mem_stats(e.ctx)
        n0 = lib.nc_device_alloc_count(e.ctx)
        assert n0 > 0
        for _ in range(10):
            chain_step(e, px, pb, G)
            st = lib.nc_get_mem_stats(e.ctx)
            assert st.arena_bytes_in_use == 0
            assert st.arena_bytes_reserved == st0.arena_bytes_reserved
            assert lib.nc_device_alloc_count(e.ctx) == n0


@pytest.fixture()
def poisoned(lib):
    old = os.environ.get("NC_DEBUG_POISON")
    os.environ["NC_DEBUG_POISON"] = "1"
    try:
        e = Engine(lib=lib)
    finally:
        if old is None:
            os.environ.pop("NC_DEBUG_POISON", None)
        else:
            os.environ["NC_DEBUG_POISON"] = old
    yield e
    e.close()


def test_poison_fills_released_blocks(poisoned):
    """A released temporary's device block reads back as 0xCD bytes."""
    e = poisoned
    L = e.lib
    t = L.nc_relu(e.tensor(np.arange(1000, dtype=np.float32)))
    e.check()
    ptr = L.nc_device_ptr(t)
    assert ptr
    L.nc_release_temp(t)
    L.nc_synchronize(e.ctx)
    from newch_amd.hipmem import D2H, check, runtime
    out = np.empty(4000, np.uint8)
    check(runtime().hipMemcpy(out.ctypes.data_as(c_void_p), c_void_p(ptr), out.nbytes, D2H), "download")
    assert (out == 0xCD).all()
    e.step_end()


def test_engine_golden_with_poison(poisoned):
    """The engine's golden replays with every released device block poisoned: no op reads memory the
    arena already took back."""
    from tests import test_gpu_parity as T
    e = poisoned
    for name, s in T.UNARY:
        T.test_engine_unary_golden(e, name, s)
    for case, aview in T.BINARY_CASES:
        for op in ("add", "sub", "mul", "div"):
            T.test_engine_binary_golden(e, case, aview, op)
    for case in ("r2x3", "r4x5x6", "r3x1000", "r5x13x9", "special"):
        T.test_engine_reduce_golden(e, case)
    for key in ("3x1", "4x7", "5x64", "3x100", "2x1030", "6x17"):
        T.test_engine_softmax_golden(e, key)
    for key in ("6x10", "3x4x5", "4x1024", "2x3"):
        T.test_engine_layer_norm_golden(e, key)
    T.test_engine_quantize_golden(e)
    T.test_engine_chain_golden(e)
    for key in T.LOSS_KEYS:
        T.test_engine_loss_golden(e, key)
    for cfg in T._optim_configs():
        T.test_engine_optim_golden(e, cfg)
    for case, aview, bview in T.MATMUL_CASES:
        T.test_engine_matmul_golden(e, case, aview, bview)
    for case, xview, has_b in T.LINEAR_CASES:
        T.test_engine_linear_golden(e, case, xview, has_b)
    e.check()


def test_forced_device_out_of_memory_is_sticky_and_recovers(monkeypatch):
    """NC_FAIL_ALLOC_AT=4: the context's fourth device allocation fails.  A parameter of 32 MiB (its
    staging tensor and its persistent storage: allocations 1 and 2) and relu's output (3) succeed; the
    add's output (4) fails: NULL and a sticky NC_ERR_OOM, another op returns NULL with the first
    message kept; after nc_clear_error and nc_step_end the same op computes (the reference's sticky
    errors, engine/src/core/ctx.c:375-390)."""
    print("engine: NC_FAIL_ALLOC_AT=4, 32 MiB tensors", flush=True)
    monkeypatch.setenv("NC_FAIL_ALLOC_AT", "4")
    x = np.random.default_rng(12).standard_normal(1 << 23).astype(np.float32)
    with Engine(lib=abi.load(abi.LIB_PATH)) as eng:
        L = eng.lib
        p = eng.param(x)
        y = L.nc_relu(p)
        eng.check()
        assert L.nc_device_alloc_count(eng.ctx) == 3
        assert not L.nc_add(p, y)
        assert L.nc_status_code(eng.ctx) == abi.ERR_OOM
        first = L.nc_error(eng.ctx).decode()
        assert "out of memory" in first
        assert not L.nc_mul(p, p)
        assert L.nc_status_code(eng.ctx) == abi.ERR_OOM and L.nc_error(eng.ctx).decode() == first
        L.nc_clear_error(eng.ctx)
        L.nc_step_end(eng.ctx)
        z = L.nc_add(p, p)
        eng.check()
        assert (eng.read(z).view(np.uint32) == (x + x).view(np.uint32)).all()
        eng.step_end()
