"""CPU tests of the engine library (no GPU): the C ABI loads and exports everything the headers
declare, the reference's bindings resolve, host-side logic (shape inference, error messages, views,
the RNG, the index divider) matches the compiled reference, and compute ops fail loudly without a
HIP device instead of falling back to the host."""

import ctypes
import random
import re
from ctypes import c_char_p, c_float, c_uint32, c_void_p
from pathlib import Path

import numpy as np
import pytest

from newch_amd import abi
from oracle import pyoracle as O
from tests.ncdrive import Engine, NcError

ROOT = Path(__file__).resolve().parents[1]
GOLD = Path(__file__).resolve().parent / "golden"


def declared(header: Path) -> set[str]:
    text = header.read_text()
    return set(re.findall(r"^(?:NC_API|NC_HIP_API)\s+[^;]*?\b(nc_[a-z0-9_]+)\s*\(", text, flags=re.M))


@pytest.fixture(scope="module")
def lib():
    return abi.load(abi.LIB_PATH)


def has_device(lib) -> bool:
    return lib.nc_device_count() > 0


def test_exports_every_declared_symbol(lib):
    names = declared(ROOT / "include" / "nc.h") | declared(ROOT / "include" / "nc_hip.h")
    assert len(names) >= 150
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing


def test_nc_h_declares_the_full_reference_api():
    ours = declared(ROOT / "include" / "nc.h")
    assert set(abi.NC_SIGNATURES) <= ours


def test_reference_python_bindings_resolve(lib):
    names = (GOLD / "lib_py_names.txt").read_text().split()
    assert len(names) == 111
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_kernel_layer_binds(lib):
    from newch_amd import hip
    hip.bind(ctypes.CDLL(str(abi.LIB_PATH)))


def test_multi_tensor_workspace_queries(lib):
    """Host-only queries of the multi-tensor entry points: the sum-of-squares workspace of a table is
    the sum of its tensors' one-tensor workspaces (no device needed)."""
    from newch_amd import hip
    K = hip.Kernels(ctypes.CDLL(str(abi.LIB_PATH)))
    sizes = [0, 1, 7, 65536, 1_000_003, 1 << 26]
    assert K.sumsq_multi_workspace(sizes) == sum(K.sumsq_workspace(n) for n in sizes)
    assert K.sumsq_multi_workspace([]) == 0
    assert K.sumsq_workspace(0) == 0 and K.sumsq_workspace(1) >= 8


def test_index_divider_matches_integer_division(lib):
    from newch_amd import hip
    L = hip.bind(ctypes.CDLL(str(abi.LIB_PATH)))
    rng = random.Random(5)
    divs = list(range(1, 1025)) + [rng.randrange(1, 2 ** 32) for _ in range(2000)]
    for k in range(1, 32):
        divs += [2 ** k - 1, 2 ** k, 2 ** k + 1]
    nums = list(range(0, 4097)) + [2 ** 32 - 1 - i for i in range(4096)] + [rng.randrange(0, 2 ** 32) for _ in range(20000)]
    for k in range(1, 32):
        nums += [2 ** k - 1, 2 ** k, 2 ** k + 1]
    dv = (c_uint32 * len(divs))(*divs)
    nv = (c_uint32 * len(nums))(*nums)
    assert L.nc_hip_check_intdiv(dv, len(divs), nv, len(nums)) == 0
    # edge numerators for each divisor: multiples and their neighbours
    edge = []
    for d in divs[:3000:7]:
        for m in (1, 2, 3, (2 ** 32 - 1) // d):
            for t in (d * m - 1, d * m, d * m + 1):
                if 0 <= t < 2 ** 32:
                    edge.append(t)
    ev = (c_uint32 * len(edge))(*edge)
    assert L.nc_hip_check_intdiv(dv, len(divs), ev, len(edge)) == 0


# ------------------------------------------------------------------------------------------------
# behaviour without a device (this container): host logic works, compute refuses
# ------------------------------------------------------------------------------------------------
@pytest.fixture
def eng(lib):
    if has_device(lib):
        pytest.skip("a HIP device is visible: the no-device behaviour is not observable here")
    e = Engine(lib=lib)
    yield e
    e.close()


def test_no_device_compute_fails_loudly(eng):
    L = eng.lib
    assert L.nc_kernel_backend(eng.ctx) == b"hip:none"
    a = eng.tensor(np.arange(6, dtype=np.float32).reshape(2, 3))
    for fn in (lambda: L.nc_relu(a), lambda: L.nc_add(a, a), lambda: L.nc_sum(a, 0, 0),
               lambda: L.nc_softmax(a), lambda: L.nc_gelu(a, 0)):
        assert not fn()
        assert L.nc_status_code(eng.ctx) == abi.ERR_STATE
        assert b"no HIP device" in L.nc_error(eng.ctx)
        L.nc_clear_error(eng.ctx)


def test_off_path_ops_report_not_in_this_engine(eng):
    L = eng.lib
    a = eng.tensor(np.ones((1, 1, 2, 2), np.float32))
    assert not L.nc_conv2d(a, a, None, 1, 1, 0, 0)
    assert L.nc_status_code(eng.ctx) == abi.ERR_STATE and b"not in this engine" in L.nc_error(eng.ctx)
    L.nc_clear_error(eng.ctx)
    assert not L.nc_dropout(a, c_float(0.5))
    assert b"not in this engine" in L.nc_error(eng.ctx)


def test_optimizer_argument_errors_match_reference(eng):
    """Parameter validation happens before any device work: same status and message as the reference."""
    def calls(e):
        L = e.lib
        t = e.tensor(np.ones(3, np.float32))            # not a parameter
        p = e.param(np.ones((2, 2), np.float32))
        pt = L.nc_transpose(p, 0, 1)                    # not contiguous (and not persistent)
        out = []
        for params in ([t], [p, t], [pt]):
            arr = (ctypes.c_void_p * len(params))(*params)
            o = L.nc_adam(e.ctx, arr, len(params), abi.OptimOpts(0.1, 0, 0, 0, 0, 0))
            out.append((bool(o), L.nc_status_code(e.ctx), L.nc_error(e.ctx).decode()))
            L.nc_clear_error(e.ctx)
        e.step_end()
        return out
    if not O.REF_LIB.exists():
        pytest.skip("oracle/_ref/libnc_ref.so not built")
    with Engine(O.REF_LIB) as ref:
        want = calls(ref)
    assert calls(eng) == want


ref_only = pytest.mark.skipif(not O.REF_LIB.exists(), reason="oracle/_ref/libnc_ref.so not built")


def _errors(e: Engine, calls):
    """Runs each call on fresh inputs; returns [(status, message)] with the context cleared between."""
    out = []
    for make in calls:
        r = make(e)
        out.append((bool(r), e.lib.nc_status_code(e.ctx), e.lib.nc_error(e.ctx).decode()))
        e.lib.nc_clear_error(e.ctx)
        e.step_end()
    return out


SHAPE_ERRORS = [
    lambda e: e.lib.nc_add(e.tensor(np.ones((2, 3), np.float32)), e.tensor(np.ones((4,), np.float32))),
    lambda e: e.lib.nc_mul(e.tensor(np.ones((2, 3, 5), np.float32)), e.tensor(np.ones((3, 4), np.float32))),
    lambda e: e.lib.nc_add(e.tensor(np.ones((2,), np.int32)), e.tensor(np.ones((2,), np.float32))),
    lambda e: e.lib.nc_sum(e.tensor(np.ones((2, 3), np.float32)), 2, 0),
    lambda e: e.lib.nc_max(e.tensor(np.ones((0, 3), np.float32)), 0, 0),
    lambda e: e.lib.nc_argmax(e.tensor(np.ones((0,), np.float32)), abi.ALL_AXES),
    lambda e: e.lib.nc_relu(e.tensor(np.ones((2,), np.int32))),
    lambda e: e.lib.nc_softmax(e.tensor(np.ones((), np.float32))),
    lambda e: e.lib.nc_layer_norm(e.tensor(np.ones((1, 4), np.float32)), 1, e.tensor(np.ones(3, np.float32)), None,
                                  c_float(1e-5)),
    lambda e: e.lib.nc_layer_norm(e.tensor(np.ones((1, 4), np.float32)), 3, None, None, c_float(1e-5)),
    lambda e: e.lib.nc_reshape(e.tensor(np.ones((2, 3), np.float32)), *abi.shape_arg((4, 2))),
    lambda e: e.lib.nc_reshape(e.tensor(np.ones((2, 3), np.float32)), *abi.shape_arg((-2, 3))),
    lambda e: e.lib.nc_transpose(e.tensor(np.ones((2, 3), np.float32)), 0, 2),
    lambda e: e.lib.nc_slice(e.tensor(np.ones((5, 3), np.float32)), 0, 2, 3, 2),
    lambda e: e.lib.nc_slice(e.tensor(np.ones((5, 3), np.float32)), 1, 0, 1, 0),
    lambda e: e.lib.nc_quantize_rows(e.tensor(np.ones((2, 3, 4), np.float32)), None),
    lambda e: e.lib.nc_to_dtype(e.tensor(np.ones((2,), np.float32)), abi.F16),
    lambda e: e.lib.nc_empty(e.ctx, abi.F32, 7, abi.shape_arg((1,) * 7)[1]),
    lambda e: e.lib.nc_empty(e.ctx, abi.F32, 2, abi.shape_arg((2, -1))[1]),
    # losses: label dtype, logits / labels shapes, empty classes
    lambda e: e.lib.nc_cross_entropy(e.tensor(np.ones((2, 3), np.float32)), e.tensor(np.zeros(2, np.float32))),
    lambda e: e.lib.nc_cross_entropy(e.tensor(np.ones((2, 3, 1), np.float32)), e.tensor(np.zeros(2, np.int32))),
    lambda e: e.lib.nc_cross_entropy(e.tensor(np.ones((2, 3), np.float32)), e.tensor(np.zeros(3, np.int32))),
    lambda e: e.lib.nc_cross_entropy(e.tensor(np.ones((2, 0), np.float32)), e.tensor(np.zeros(2, np.int32))),
    lambda e: e.lib.nc_cross_entropy(e.tensor(np.ones((2, 3), np.int32)), e.tensor(np.zeros(2, np.int32))),
    lambda e: e.lib.nc_nll_loss(e.tensor(np.ones((4,), np.float32)), e.tensor(np.zeros(4, np.int32)), 0),
    lambda e: e.lib.nc_nll_loss(e.tensor(np.ones((2, 3), np.float32)), e.tensor(np.zeros((2, 1), np.int32)), 1),
    lambda e: e.lib.nc_nll_loss(e.tensor(np.ones((2, 3), np.float32)), e.tensor(np.zeros(2, np.int8)), 0),
    lambda e: e.lib.nc_mse_loss(e.tensor(np.ones((2, 3), np.float32)), e.tensor(np.ones((4,), np.float32))),
    # matmul / bmm / linear / linear_int8: ranks, inner dims, batch broadcast, dtypes
    lambda e: e.lib.nc_matmul(e.tensor(np.ones((3,), np.float32)), e.tensor(np.ones((3, 4), np.float32))),
    lambda e: e.lib.nc_matmul(e.tensor(np.ones((2, 3), np.float32)), e.tensor(np.ones((4, 5), np.float32))),
    lambda e: e.lib.nc_matmul(e.tensor(np.ones((2, 3, 4), np.float32)), e.tensor(np.ones((3, 4, 6), np.float32))),
    lambda e: e.lib.nc_matmul(e.tensor(np.ones((2, 3), np.float32)), e.tensor(np.ones((2, 4, 5), np.float32))),
    lambda e: e.lib.nc_matmul(e.tensor(np.ones((2, 3), np.int32)), e.tensor(np.ones((3, 5), np.float32))),
    lambda e: e.lib.nc_linear_fn(e.tensor(np.ones((2, 3), np.float32)), e.tensor(np.ones((4, 5), np.float32)), None),
    lambda e: e.lib.nc_linear_fn(e.tensor(np.ones((2, 5), np.float32)), e.tensor(np.ones((4, 5), np.float32)),
                                 e.tensor(np.ones((3,), np.float32))),
    lambda e: e.lib.nc_linear_fn(e.tensor(np.ones((2, 5), np.float32)), e.tensor(np.ones((5,), np.float32)), None),
    lambda e: e.lib.nc_linear_fn(e.tensor(np.ones((2, 5), np.float32)), e.tensor(np.ones((4, 5), np.int32)), None),
    lambda e: e.lib.nc_linear_int8(e.tensor(np.ones((2, 5), np.float32)), e.tensor(np.ones((4, 5), np.float32)),
                                   e.tensor(np.ones((4,), np.float32)), None),
    lambda e: e.lib.nc_linear_int8(e.tensor(np.ones((2, 5), np.float32)), e.tensor(np.ones((4, 5), np.int8), abi.I8),
                                   e.tensor(np.ones((3,), np.float32)), None),
    lambda e: e.lib.nc_linear_int8(e.tensor(np.ones((2, 6), np.float32)), e.tensor(np.ones((4, 5), np.int8), abi.I8),
                                   e.tensor(np.ones((4,), np.float32)), e.tensor(np.ones((4,), np.float32))),
]


@ref_only
def test_shape_errors_match_reference(eng):
    with Engine(O.REF_LIB) as ref:
        want = _errors(ref, SHAPE_ERRORS)
    got = _errors(eng, SHAPE_ERRORS)
    for i, (w, g) in enumerate(zip(want, got)):
        assert w == g, f"case {i}: reference {w}, this engine {g}"


def _views(e: Engine):
    """View results observable without device compute: shapes, contiguity, aliasing, element reads."""
    L = e.lib
    t = e.tensor(np.arange(1, 25, dtype=np.float32).reshape(2, 3, 4))
    out = []
    r = L.nc_reshape(t, *abi.shape_arg((6, -1)))
    out.append(("reshape", e.shape(r), L.nc_is_contiguous(r), L.nc_data_f32(r) == L.nc_data_f32(t)))
    tt = L.nc_transpose(t, 0, 2)
    out.append(("transpose", e.shape(tt), L.nc_is_contiguous(tt),
                [L.nc_get(tt, abi.shape_arg(ix)[1]) for ix in ((3, 2, 1), (0, 1, 1), (2, 0, 0))]))
    s = L.nc_slice(t, 2, 1, 2, 2)
    out.append(("slice", e.shape(s), L.nc_is_contiguous(s),
                [L.nc_get(s, abi.shape_arg(ix)[1]) for ix in ((1, 2, 1), (0, 0, 0))]))
    v = L.nc_reshape(L.nc_transpose(t, 1, 2), *abi.shape_arg((2, 4, 3, 1)))  # viewable
    out.append(("reshape_of_view", e.shape(v), bool(v) and L.nc_is_contiguous(v)))
    d = L.nc_detach(t)
    out.append(("detach", e.shape(d), L.nc_requires_grad(d)))
    e.step_end()
    return out


@ref_only
def test_views_match_reference(eng):
    with Engine(O.REF_LIB) as ref:
        want = _views(ref)
    assert _views(eng) == want


@ref_only
def test_rng_matches_reference(eng):
    """nc_randn / nc_rand_uniform draw the reference's xoshiro256** stream bit for bit."""
    with Engine(O.REF_LIB, seed=77) as ref:
        a = ref.read(ref.lib.nc_randn(ref.ctx, c_float(0.5), *abi.shape_arg((1000,))))
        b = ref.read(ref.lib.nc_rand_uniform(ref.ctx, c_float(-1), c_float(2), *abi.shape_arg((333,))))
    e = Engine(lib=eng.lib, seed=77)
    try:
        a2 = e.read(e.lib.nc_randn(e.ctx, c_float(0.5), *abi.shape_arg((1000,))))
        b2 = e.read(e.lib.nc_rand_uniform(e.ctx, c_float(-1), c_float(2), *abi.shape_arg((333,))))
    finally:
        e.close()
    assert a.tobytes() == a2.tobytes() and b.tobytes() == b2.tobytes()


def test_mem_stats_layout(eng):
    s = eng.lib.nc_get_mem_stats(eng.ctx)
    assert ctypes.sizeof(s) == 4 * ctypes.sizeof(ctypes.c_size_t)
    assert s.arena_bytes_in_use == 0


def test_sticky_error_and_null_propagation(eng):
    L = eng.lib
    two = eng.tensor(np.ones(2, np.float32))
    assert not L.nc_reshape(eng.tensor(np.ones(3, np.float32)), *abi.shape_arg((2,)))
    msg = L.nc_error(eng.ctx)
    assert b"reshape: cannot view [3] as [2]" == msg
    assert not L.nc_relu(None)
    assert not L.nc_add(two, None)
    assert not L.nc_transpose(two, 0, 0)  # ops refuse to run while an error is pending
    assert L.nc_error(eng.ctx) == msg  # first error sticks
    L.nc_clear_error(eng.ctx)
    assert L.nc_ok(eng.ctx)


# ------------------------------------------------------------------------------------------------
# NCW1 files: the reference's bytes and messages (host storage: no device needed)
# ------------------------------------------------------------------------------------------------
@ref_only
def test_ncw1_bytes_match_reference(eng, tmp_path):
    from tests.ncdrive import io_save, io_tensors
    with Engine(O.REF_LIB) as ref:
        names, ts, _ = io_tensors(ref)
        assert io_save(ref, tmp_path / "ref.ncw", names, ts) == 0
    names, ts, _ = io_tensors(eng)
    assert io_save(eng, tmp_path / "ours.ncw", names, ts) == 0
    assert (tmp_path / "ours.ncw").read_bytes() == (tmp_path / "ref.ncw").read_bytes()
    eng.step_end()


@ref_only
def test_ncw1_load_reference_file(eng, tmp_path):
    from tests.ncdrive import io_load, io_save, io_tensors
    with Engine(O.REF_LIB) as ref:
        names, ts, arrays = io_tensors(ref, rng_seed=5)
        assert io_save(ref, tmp_path / "ref.ncw", names, ts) == 0
    # fresh contiguous targets of the same dtypes / shapes; ask for a subset in another order
    L = eng.lib
    want = {n: a for n, a in zip(names, arrays)}
    pick = ["0.weight", "q", "w_t", "scalar", "empty", "mask"]
    targets = [eng.tensor(np.zeros_like(want[n])) for n in pick]
    assert io_load(eng, tmp_path / "ref.ncw", pick, targets) == 0, L.nc_error(eng.ctx)
    for n, t in zip(pick, targets):
        got = eng.read(t)
        assert got.dtype == want[n].dtype and got.shape == want[n].shape and (got == want[n]).all(), n
    eng.step_end()


def _io_errors(e, tmp_path):
    from tests.ncdrive import io_load, io_save
    L = e.lib
    good = tmp_path / "good.ncw"
    t = e.tensor(np.ones((2, 3), np.float32))
    assert io_save(e, good, ["a"], [t]) == 0
    raw = good.read_bytes()
    (tmp_path / "magic.ncw").write_bytes(b"XXXX" + raw[4:])
    (tmp_path / "version.ncw").write_bytes(raw[:4] + (2).to_bytes(4, "little") + raw[8:])
    (tmp_path / "trunc.ncw").write_bytes(raw[:-5])
    (tmp_path / "header.ncw").write_bytes(raw[:20])
    nb = raw.index((24).to_bytes(8, "little"))
    (tmp_path / "bytes.ncw").write_bytes(raw[:nb] + (28).to_bytes(8, "little") + raw[nb + 8:] + b"\0" * 4)
    out = []

    def record(rc):
        out.append((rc, L.nc_status_code(e.ctx), L.nc_error(e.ctx).decode().replace(str(tmp_path), "<dir>")))
        L.nc_clear_error(e.ctx)

    record(io_load(e, tmp_path / "missing.ncw", ["a"], [t]))
    for f in ("magic", "version", "trunc", "header", "bytes"):
        record(io_load(e, tmp_path / f"{f}.ncw", ["a"], [e.tensor(np.zeros((2, 3), np.float32))]))
    record(io_load(e, good, ["b"], [e.tensor(np.zeros((2, 3), np.float32))]))               # not found
    record(io_load(e, good, ["a"], [e.tensor(np.zeros((3, 2), np.float32))]))               # shape
    record(io_load(e, good, ["a"], [e.tensor(np.zeros((2, 3), np.int32))]))                 # dtype
    record(io_load(e, good, ["a"], [L.nc_transpose(e.tensor(np.zeros((3, 2), np.float32)), 0, 1)]))  # view
    record(io_save(e, tmp_path / "nope" / "x.ncw", ["a"], [t]))                              # unopenable
    arr_n = (c_char_p * 2)(b"a", None)
    arr_t = (c_void_p * 2)(t, t)
    record(L.nc_save(e.ctx, str(tmp_path / "n.ncw").encode(), 2, arr_n, arr_t))              # NULL name
    e.step_end()
    return out


@ref_only
def test_ncw1_errors_match_reference(eng, tmp_path):
    (tmp_path / "r").mkdir()
    (tmp_path / "o").mkdir()
    with Engine(O.REF_LIB) as ref:
        want = _io_errors(ref, tmp_path / "r")
    got = _io_errors(eng, tmp_path / "o")
    for i, (w, g) in enumerate(zip(want, got)):
        assert w == g, f"case {i}: reference {w}, this engine {g}"


def test_reduce_plans_fit_the_no_alloc_scratch(lib):
    """nc_hip_reduce_fwd_noalloc keeps its partials in an 8 MiB static array: every reduction plan
    needs at most that.  The plan (host arithmetic, no device) is evaluated at the boundaries of each
    mode -- column scans whose column count sits just past target / k for k = 1..2048 (the chunk count
    P = ceil(target / cols) steps there, cols * P is largest), few long rows just past and below the
    wave-per-row cutoffs -- and over a seeded random sweep."""
    from newch_amd.hip import RED
    fn = lib.nc_hip_reduce_workspace
    fn.restype = ctypes.c_size_t
    fn.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]
    limit = 8 << 20
    target = 256 * 2048  # columns the column-scan plan aims its partials at
    shapes = []
    for k in range(1, 2049):
        for cols in (target // k - 1, target // k, target // k + 1):
            if cols >= 2:
                shapes += [(1, 1 << 20, cols), (2, 1 << 20, max(cols // 2, 2))]
    for outer in (1, 2, 3, 255, 256, 257, 4095, 4096):
        for R in (4097, 65536, 1 << 20, 1 << 24, 1 << 30, 1 << 32):
            shapes.append((outer, R, 1))
    rng = np.random.default_rng(8)
    for _ in range(4000):
        outer, R, inner = (int(v) for v in np.exp(rng.uniform(0, [9, 24, 16])).astype(np.int64) + 1)
        shapes.append((outer, R, inner))
    worst = 0
    for outer, R, inner in shapes:
        for kind in ("sum", "max"):
            need = fn(RED[kind], outer, R, inner)
            worst = max(worst, need)
            assert need <= limit, (kind, outer, R, inner, need)
    assert worst > limit // 2  # the boundary shapes come close to the bound


def test_forced_out_of_memory_is_sticky_and_recovers(lib, monkeypatch):
    """NC_FAIL_ALLOC_AT=2 makes the context's second storage allocation fail: the call returns NULL
    with NC_ERR_OOM, later calls keep the first error (the reference's sticky errors,
    engine/src/core/ctx.c:375-390; ops return NULL while it stands, autograd.c:16), and
    nc_clear_error plus nc_step_end recover."""
    monkeypatch.setenv("NC_FAIL_ALLOC_AT", "2")
    with Engine(lib=lib) as eng:
        L = eng.lib
        if has_device(L):
            pytest.skip("host storage path: the device's allocations are tested on the GPU")
        a = eng.tensor(np.arange(6, dtype=np.float32))
        b = np.ones(6, np.float32)
        nd, shp = abi.shape_arg((6,))
        assert not L.nc_from_data(eng.ctx, abi.F32, b.ctypes.data_as(c_void_p), nd, shp)
        assert L.nc_status_code(eng.ctx) == abi.ERR_OOM
        first = L.nc_error(eng.ctx).decode()
        assert "out of host memory" in first
        nd2, shp2 = abi.shape_arg((2, 3))
        assert not L.nc_reshape(a, nd2, shp2)  # an op while the error stands
        assert L.nc_status_code(eng.ctx) == abi.ERR_OOM and L.nc_error(eng.ctx).decode() == first
        L.nc_clear_error(eng.ctx)
        L.nc_step_end(eng.ctx)
        t = L.nc_from_data(eng.ctx, abi.F32, b.ctypes.data_as(c_void_p), nd, shp)
        assert t and L.nc_ok(eng.ctx)
        r = L.nc_reshape(t, nd2, shp2)
        assert r and eng.shape(r) == (2, 3)
        assert (eng.read(r) == 1).all()
