"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Three independent pins per function:
  * the golden vectors in tests/golden/ (written by the compiled reference engine), bit for bit;
  * the live reference library oracle/_ref/libnc_ref.so on fresh random inputs, when it is built;
  * closed forms / invariants / the reference's own known answers (engine/tests/test_main.c,
    tests/test_extras.py), chosen so a dropped term, wrong sign or wrong index fails.
"""

import math
import zlib
from pathlib import Path

import numpy as np
import pytest

from oracle import pyoracle as O

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(GOLD / f"{name}.npz")


def bits_equal(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    if a.dtype.kind == "f":
        nan = np.isnan(a) & np.isnan(b)
        ok = (a.view(np.uint32) == b.view(np.uint32)) | nan
        return bool(ok.all()), int((~ok).sum())
    ok = a == b
    return bool(ok.all()), int((~ok).sum())


def assert_bits(a, b, what=""):
    ok, nbad = bits_equal(a, b)
    assert ok, f"{what}: {nbad} elements differ"


# ------------------------------------------------------------------------------------------------
# golden vectors
# ------------------------------------------------------------------------------------------------
def test_transcendentals_golden():
    d = load("transcendentals")
    for fn in ("exp", "sigmoid", "tanh", "erf"):
        assert_bits(O.vmap(fn, d["x"]), d[fn], fn)
    for n, want in zip(d["sum_n"], d["sum_out"]):
        assert_bits(O.sum_f32(d["sum_x"][:n]), want, f"sum_f32 n={n}")


UNARY = [("relu", "relu", 0.0), ("leaky_relu", "leaky_relu", 0.01), ("leaky_relu_02", "leaky_relu", 0.2),
         ("relu6", "relu6", 0.0), ("hardsigmoid", "hardsigmoid", 0.0), ("hardswish", "hardswish", 0.0),
         ("silu", "silu", 0.0), ("gelu", "gelu", 0.0), ("gelu_tanh", "gelu_tanh", 0.0),
         ("sigmoid", "sigmoid", 0.0), ("tanh", "tanh", 0.0), ("exp", "exp", 0.0)]


@pytest.mark.parametrize("name,kind,s", UNARY)
def test_unary_golden(name, kind, s):
    d = load("unary")
    x, g = d["x"], d["g"]
    y = O.unary_fwd(kind, x, s)
    assert_bits(y, d[f"{name}_y"], f"{name} fwd")
    gx = O.unary_bwd(kind, x, y, g, s=s)
    assert_bits(gx, d[f"{name}_gx"], f"{name} bwd")


def make_view(storage, view):
    if view is None:
        return storage
    v = np.swapaxes(storage, view[1], view[2])
    if view[0] == "t_reshape":
        v = v.reshape(view[3])
        assert not v.flags.c_contiguous and np.shares_memory(v, storage)
    return v


BINARY_CASES = [
    ("bias4d", None, None), ("row", None, None), ("outer", None, None), ("scalar_lhs", None, None),
    ("scalar_rhs", None, None), ("cfg2_small", None, None), ("cfg2_batch_t", ("t", 0, 1), None),
    ("cfg2_inner_strided", ("t_reshape", 1, 2, (5, 6, 1, 8)), None), ("same_flat", None, None),
    ("same_a_t", ("t", 0, 1), None), ("rank_mismatch", None, None), ("ragged", None, None)]


@pytest.mark.parametrize("case,aview,bview", BINARY_CASES)
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_binary_golden(case, aview, bview, op):
    d = load("binary")
    a = make_view(d[f"{case}/a_storage"], aview)
    b = make_view(d[f"{case}/b_storage"], bview)
    out = O.binary_fwd(op, a, b)
    assert_bits(out, d[f"{case}/{op}/out"], f"{case} {op} fwd")
    ga, gb = O.binary_bwd(op, a, b, d[f"{case}/{op}/G"])
    assert_bits(ga, d[f"{case}/{op}/ga"], f"{case} {op} grad a")
    assert_bits(gb, d[f"{case}/{op}/gb"], f"{case} {op} grad b")


def _axes(x):
    return list(range(x.ndim)) + [-128]


@pytest.mark.parametrize("case", ["r2x3", "r4x5x6", "r3x1000", "r5x13x9", "special"])
def test_reduce_golden(case):
    d = load("reduce")
    x = d[f"{case}/x"]
    for axis in _axes(x):
        for kind in ("sum", "mean", "max"):
            key = f"{case}/{kind}/{axis}"
            if f"{key}/y" not in d:
                continue
            y, arg = O.reduce_fwd(kind, x, axis)
            want = d[f"{key}/y"]
            assert_bits(y.reshape(want.shape), want, f"{key} fwd")
            gx = O.reduce_bwd(kind, x.shape, axis, d[f"{key}/G"], arg)
            assert_bits(gx, d[f"{key}/gx"], f"{key} bwd")
        want = d[f"{case}/argmax/{axis}/y"]
        got, _ = O.reduce_fwd("argmax", x, axis)
        assert_bits(got.reshape(want.shape), want, f"{case} argmax {axis}")


def test_reduce_empty_golden():
    d = load("reduce")
    y, _ = O.reduce_fwd("mean", np.zeros((0, 3), np.float32), -128)
    assert np.isnan(y[0]) and np.isnan(d["empty/mean_all"])
    y, _ = O.reduce_fwd("mean", np.zeros((0, 3), np.float32), 0)
    assert_bits(y, d["empty/mean_0"])
    y, _ = O.reduce_fwd("sum", np.zeros((0, 3), np.float32), 0)
    assert_bits(y, d["empty/sum_0"])


@pytest.mark.parametrize("key", ["3x1", "4x7", "5x64", "3x100", "2x1030", "6x17"])
def test_softmax_golden(key):
    d = load("softmax")
    x = d[f"{key}/x"]
    for form in ("softmax", "log_softmax"):
        lf = form == "log_softmax"
        y = O.softmax_fwd(x, lf)
        assert_bits(y, d[f"{key}/{form}/y"], f"{key} {form}")
        gx = O.softmax_bwd(y, d[f"{key}/{form}/G"], lf)
        assert_bits(gx, d[f"{key}/{form}/gx"], f"{key} {form} bwd")


@pytest.mark.parametrize("key", ["6x10", "3x4x5", "4x1024", "2x3"])
def test_layer_norm_golden(key):
    d = load("layernorm")
    x, w, b, k = d[f"{key}/x"], d[f"{key}/w"], d[f"{key}/b"], int(d[f"{key}/k"])
    D = int(np.prod(x.shape[x.ndim - k:]))
    for variant in ("wb", "w", "none"):
        ww = w if variant in ("wb", "w") else None
        bb = b if variant == "wb" else None
        y, stats = O.layer_norm_fwd(x, D, ww, bb, 1e-5)
        assert_bits(y, d[f"{key}/{variant}/y"], f"{key} {variant} fwd")
        gx, gw, gb = O.layer_norm_bwd(x, D, stats, d[f"{key}/{variant}/G"], ww, ww is not None, bb is not None)
        assert_bits(gx, d[f"{key}/{variant}/gx"], f"{key} {variant} gx")
        if ww is not None:
            assert_bits(gw, d[f"{key}/{variant}/gw"], f"{key} {variant} gw")
        if bb is not None:
            assert_bits(gb, d[f"{key}/{variant}/gb"], f"{key} {variant} gb")


def test_quant_golden():
    d = load("quant")
    q, s = O.quantize_rows(d["w"])
    assert_bits(q, d["q"], "q")
    assert_bits(s, d["scale"], "scale")
    assert_bits(O.dequantize_rows(q, s), d["deq"], "dequant")


def test_chain_golden():
    """relu(x + bias).sum((2, 3)): the oracle composes add -> relu -> two keepdim sums."""
    d = load("chain")
    x, bias, G = d["x"], d["bias"], d["G"]
    h0 = O.binary_fwd("add", x, bias)
    h = O.unary_fwd("relu", h0)
    s3, _ = O.reduce_fwd("sum", h, 3)
    s3 = s3.reshape(4, 16, 28, 1)
    s2, _ = O.reduce_fwd("sum", s3, 2)
    assert_bits(s2.reshape(4, 16), d["y"], "chain fwd")
    g3 = O.reduce_bwd("sum", s3.shape, 2, G.reshape(4, 16, 1, 1))
    gh = O.reduce_bwd("sum", h.shape, 3, g3)
    gh0 = O.unary_bwd("relu", h0, h, gh)
    gx, gb = O.binary_bwd("add", x, bias, gh0)
    assert_bits(gx, d["gx"], "chain grad x")
    assert_bits(gb, d["gbias"], "chain grad bias")


LOSS_CASES = ["3x5", "8x10", "4x1", "6x64", "5x1030", "0x7"]


@pytest.mark.parametrize("key", LOSS_CASES)
def test_loss_golden(key):
    d = load("loss")
    x, lab, G = d[f"{key}/x"], d[f"{key}/lab"], float(d[f"{key}/G"])
    N = x.shape[0]
    loss, prob = O.cross_entropy_fwd(x, lab)
    assert_bits(loss, d[f"{key}/ce/loss"], f"{key} cross_entropy")
    if N:
        assert_bits(O.cross_entropy_bwd(prob, lab, G), d[f"{key}/ce/gx"], f"{key} cross_entropy bwd")
    for form, sm in (("nll_mean", False), ("nll_sum", True)):
        assert_bits(O.nll_loss_fwd(x, lab, sm), d[f"{key}/{form}/loss"], f"{key} {form}")
        if N:
            assert_bits(O.nll_loss_bwd(x.shape, lab, G, sm), d[f"{key}/{form}/gx"], f"{key} {form} bwd")


@pytest.mark.parametrize("which", ["high", "negative"])
def test_loss_bad_label_golden(which):
    d = load("loss")
    x, lab = d[f"bad_{which}/x"], d[f"bad_{which}/lab"]
    for form, fn in (("ce", lambda: O.cross_entropy_fwd(x, lab)), ("nll", lambda: O.nll_loss_fwd(x, lab))):
        with pytest.raises(ValueError) as e:
            fn()
        msg = str(d[f"bad_{which}/{form}/message"])
        assert msg.endswith(str(e.value)), (msg, str(e.value))


def optim_configs():
    from tests.golden.gen_golden import OPTIM_CONFIGS
    return OPTIM_CONFIGS


@pytest.mark.parametrize("cfg", optim_configs(), ids=[c[0] for c in optim_configs()])
def test_optim_golden(cfg):
    d = load("optim")
    name, steps = cfg[0], cfg[5]
    W = [d[f"{name}/w_init{i}"] for i in range(2)]
    Gs = [[d[f"{name}/G{k}_{i}"] for i in range(2)] for k in range(steps)]
    got = O.optim_replay(cfg, W, Gs)
    assert set(got) == {k for k in d.files if k.startswith(name + "/") and "/step" in k or k == f"{name}/t"}
    for k, v in got.items():
        assert_bits(v, d[k], k)


@pytest.mark.parametrize("case", ["clip", "noclip"])
def test_clip_grad_norm_golden(case):
    d = load("optim")
    total, g = O.clip_grad_norm([d[f"{case}/G{i}"] for i in range(2)], d[f"{case}/max_norm"])
    assert_bits(total, d[f"{case}/total"], "total")
    for i in range(2):
        assert_bits(g[i], d[f"{case}/g{i}"], f"grad {i}")


MATMUL_CASES = [
    ("mm_2d", None, None), ("mm_fold3d", None, None), ("mm_a_t", ("t", 0, 1), None),
    ("mm_b_t", None, ("t", 0, 1)), ("mm_both_t", ("t", 0, 1), ("t", 0, 1)), ("mm_outer", None, None),
    ("mm_fold_t", ("t", 1, 2), None), ("bmm_same", None, None), ("bmm_bcast_a2d", None, None),
    ("bmm_bcast_4d", None, None), ("bmm_b_t", None, ("t", 2, 3)), ("bmm_rank", None, None),
    ("bmm_batch_t", ("t", 0, 1), None)]
LINEAR_CASES = [("lin_bias", None, True), ("lin_nobias_3d", None, False), ("lin_x_t", ("t", 0, 1), True),
                ("lin_wide", None, True)]
QLINEAR_CASES = ["q_ref_test", "q_aligned", "q_3d", "q_tiles", "q_odd_k"]


def _grad_term_counts(a, b, y):
    """Terms summed per element of ga and gb: N (times the batches a matrix of a is broadcast over)
    and M (likewise for b); a folded matmul sums gb over every row of a."""
    N = y.shape[-1]
    if b.ndim == 2:
        return N, y.size // N
    M = y.shape[-2]
    Bo = y.size // (M * N)
    Ba = a.size // (a.shape[-2] * a.shape[-1])
    Bb = b.size // (b.shape[-2] * b.shape[-1])
    return N * Bo // Ba, M * Bo // Bb


@pytest.mark.parametrize("case,aview,bview", MATMUL_CASES, ids=[c[0] for c in MATMUL_CASES])
def test_matmul_golden(case, aview, bview):
    """The reference's fp32 matmul / bmm and their grads lie within the GEMM tolerance of the fp64
    truth; a transposed operand, a wrong fold or a broadcast grad not summed would miss by O(1)."""
    d = load("linalg")
    a = make_view(d[f"{case}/a_storage"], aview)
    b = make_view(d[f"{case}/b_storage"], bview)
    y64, ty = O.matmul64(a, b)
    ga, gb, ta, tb = O.matmul_grads64(a, b, d[f"{case}/G"])
    assert d[f"{case}/out"].shape == y64.shape
    assert d[f"{case}/ga"].shape == a.shape and d[f"{case}/gb"].shape == b.shape
    na, nb = _grad_term_counts(a, b, y64)
    assert O.gemm_excess(d[f"{case}/out"], y64, ty, a.shape[-1]) <= 1.0
    assert O.gemm_excess(d[f"{case}/ga"], ga, ta, na) <= 1.0
    assert O.gemm_excess(d[f"{case}/gb"], gb, tb, nb) <= 1.0


def _fp32_dot_rows(A, B, panel):
    """fp32 products of A (M x K) and B (K x N) summed one k at a time; with `panel`, each panel of
    that many k summed from zero and added into a running total."""
    K = A.shape[1]
    acc = np.zeros((A.shape[0], B.shape[1]), np.float32)
    tot = None
    for k in range(K):
        acc = (acc + np.outer(A[:, k], B[k])).astype(np.float32)
        if panel and (k + 1) % panel == 0 and k + 1 < K:
            tot = acc.copy() if tot is None else (tot + acc).astype(np.float32)
            acc[:] = 0
    return acc if tot is None else (tot + acc).astype(np.float32)


def test_gemm_bar_separates_blocked_from_sequential_sums():
    """The GEMM bar (terms / sqrt(K) floor, no cap) tells the reference's blocked sum from a plain
    running fp32 sum: at K = 16384 a sum adding each product to the running total leaves the bound,
    while 256-product panels added into a running total (the reference's KC = 256,
    kernels_avx2.c:234-247, and the matrix-core kernels' order) stay far inside it."""
    rng = np.random.default_rng(16384)
    K = 16384
    A = rng.standard_normal((64, K)).astype(np.float32)
    B = rng.standard_normal((K, 256)).astype(np.float32)
    want = A.astype(np.float64) @ B.astype(np.float64)
    terms = np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64))
    assert O.gemm_excess(_fp32_dot_rows(A, B, 0), want, terms, K) > 1.2
    assert O.gemm_excess(_fp32_dot_rows(A, B, 256), want, terms, K) < 0.4


@pytest.mark.parametrize("case,xview,has_b", LINEAR_CASES, ids=[c[0] for c in LINEAR_CASES])
def test_linear_golden(case, xview, has_b):
    d = load("linalg")
    x = make_view(d[f"{case}/x_storage"], xview)
    W = d[f"{case}/w"]
    bias = d[f"{case}/bias"] if has_b else None
    y64, ty = O.linear64(x, W, bias)
    assert O.gemm_excess(d[f"{case}/out"], y64, ty, W.shape[1]) <= 1.0
    gx, gw, gb, tx, tw, tb = O.linear_grads64(x, W, d[f"{case}/G"])
    M = x.size // W.shape[1]
    assert O.gemm_excess(d[f"{case}/gx"], gx, tx, W.shape[0]) <= 1.0
    assert O.gemm_excess(d[f"{case}/gw"], gw, tw, M) <= 1.0
    if has_b:
        assert O.gemm_excess(d[f"{case}/gbias"], gb, tb, M) <= 1.0


@pytest.mark.parametrize("case", QLINEAR_CASES)
def test_linear_int8_golden(case):
    d = load("linalg")
    q, scale = O.quantize_rows(d[f"{case}/w"])
    assert_bits(q, d[f"{case}/q"], "weight q")
    assert_bits(scale, d[f"{case}/scale"], "weight scale")
    bias = d[f"{case}/bias"] if f"{case}/bias" in d.files else None
    y = O.linear_int8(d[f"{case}/x"], q, scale, bias)
    assert_bits(y, d[f"{case}/out"], "linear_int8")
    # the reference's own acceptance bound against the fp32 linear (test_main.c:1046-1060)
    ref32 = d[f"{case}/fp32_out"].astype(np.float64)
    rel = np.sqrt(((y - ref32) ** 2).sum() / (ref32 ** 2).sum())
    assert rel < 0.02, rel


@pytest.mark.parametrize("case", ["s8_kat", "s8_rand", "s8_extreme"])
def test_gemm_s8_golden(case):
    d = load("linalg")
    A, B = d[f"{case}/a"], d[f"{case}/b"]
    C = O.gemm_s8_nt(A, B)
    assert_bits(C, d[f"{case}/c"], case)
    assert (C == A.astype(np.int64) @ B.astype(np.int64).T).all()  # exact integer product


def test_linear_int8_epilogue_order():
    """The epilogue is ((float)acc * xs) * ws + b, each step rounded to fp32: the oracle matches that
    form on every element, and on these inputs the reassociated product (xs * ws first) and the
    contracted fma(prod, ws, b) each differ from it somewhere, so either mistake would be caught."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((200, 48)).astype(np.float32)
    wq = rng.integers(-127, 128, (24, 48)).astype(np.int8)
    ws = (rng.random(24) * 0.02).astype(np.float32)
    bias = rng.standard_normal(24).astype(np.float32)
    y = O.linear_int8(x, wq, ws, bias)
    xq, xs = O.quantize_rows(x)
    accf = (xq.astype(np.int64) @ wq.astype(np.int64).T).astype(np.float32)
    prod = (accf * xs[:, None]).astype(np.float32)
    want = ((prod * ws).astype(np.float32) + bias).astype(np.float32)
    assert_bits(y, want, "left-to-right epilogue")
    reassoc = ((accf * (xs[:, None] * ws).astype(np.float32)).astype(np.float32) + bias).astype(np.float32)
    fused = (prod.astype(np.float64) * ws + bias).astype(np.float32)
    assert not bits_equal(reassoc, y)[0] and not bits_equal(fused, y)[0]
    y0 = O.linear_int8(x, wq, ws, None)  # no bias: the + 0.0f still applies (-0 becomes +0)
    assert_bits(y0, ((prod * ws).astype(np.float32) + np.float32(0)).astype(np.float32), "no bias")
    assert not np.signbit(y0[y0 == 0]).any()


# ------------------------------------------------------------------------------------------------
# the live reference (only where oracle/_ref was built: this container, or a box it travelled to)
# ------------------------------------------------------------------------------------------------
ref_only = pytest.mark.skipif(not O.REF_LIB.exists(), reason="oracle/_ref/libnc_ref.so not built")


@ref_only
def test_transcendentals_vs_live_reference():
    import ctypes
    L = ctypes.CDLL(str(O.REF_LIB))
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(200_000).astype(np.float32) * 20,
                        np.frombuffer(rng.integers(0, 2 ** 32, 200_000, dtype=np.uint32).tobytes(), np.float32)])
    for fn in ("exp", "sigmoid", "tanh", "erf"):
        y = np.empty_like(x)
        getattr(L, f"ncref_{fn}_f32")(ctypes.c_int64(x.size), x.ctypes.data_as(ctypes.c_void_p),
                                      y.ctypes.data_as(ctypes.c_void_p))
        assert_bits(O.vmap(fn, x), y, fn)


@ref_only
@pytest.mark.parametrize("name,kind,s", UNARY)
def test_unary_vs_live_reference(name, kind, s):
    from tests.ncdrive import Engine
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    x = (rng.standard_normal(4099) * 4).astype(np.float32)
    g = rng.standard_normal(4099).astype(np.float32)
    with Engine(O.REF_LIB) as ref:
        y_ref, gx_ref = ref.unary(name, x, g, s)
    y = O.unary_fwd(kind, x, s)
    assert_bits(y, y_ref, name)
    assert_bits(O.unary_bwd(kind, x, y, g, s=s), gx_ref, name + " bwd")


@ref_only
@pytest.mark.parametrize("N,C", [(33, 257), (64, 1024), (7, 3)])
def test_loss_vs_live_reference(N, C):
    from tests.ncdrive import Engine
    rng = np.random.default_rng(N * 1000 + C)
    x = (rng.standard_normal((N, C)) * 4).astype(np.float32)
    lab = rng.integers(0, C, N).astype(np.int32)
    G = np.float32(rng.standard_normal())
    loss, prob = O.cross_entropy_fwd(x, lab)
    with Engine(O.REF_LIB) as ref:
        L = ref.lib
        for form in ("ce", "mean", "sum"):
            p = ref.param(x)
            t = ref.tensor(lab)
            out = L.nc_cross_entropy(p, t) if form == "ce" else L.nc_nll_loss(p, t, int(form == "sum"))
            got = ref.read(out)
            ref.backward_with(out, np.asarray(G))
            gx = ref.grad(p)
            if form == "ce":
                assert_bits(loss, got, "cross_entropy")
                assert_bits(O.cross_entropy_bwd(prob, lab, float(G)), gx, "cross_entropy bwd")
            else:
                assert_bits(O.nll_loss_fwd(x, lab, form == "sum"), got, f"nll {form}")
                assert_bits(O.nll_loss_bwd(x.shape, lab, float(G), form == "sum"), gx, f"nll {form} bwd")
            ref.step_end()


@ref_only
@pytest.mark.parametrize("shape,axis", [((5, 13, 9), 1), ((7, 300), 1), ((300, 7), 0), ((4, 6, 11), 2),
                                        ((3, 1000), -128)])
def test_reduce_bwd_accumulates_vs_live_reference(shape, axis):
    """sum / mean gradients added into a gradient that already holds values (a second backward): the
    reference adds scale * g, rounded, where the reduced extent is innermost (inner == 1,
    ops_reduce.c:133-135) and otherwise calls its axpy, fused multiply-adds to the end of each row
    (kernels_avx2.c:39-45).  Golden vectors start from a zero gradient, where both forms agree; this
    pins the accumulating forms, with inner rows of 9, 7 and 11 floats so the axpy's 8-wide loop has a
    tail."""
    from tests.ncdrive import Engine
    rng = np.random.default_rng(sum(shape) + axis)
    x = rng.standard_normal(shape).astype(np.float32)
    for kind in ("sum", "mean"):
        with Engine(O.REF_LIB) as ref:
            fn = ref.lib.nc_sum if kind == "sum" else ref.lib.nc_mean
            p = ref.param(x)
            Gs = []
            for _ in range(2):
                out = fn(p, axis, 0)
                G = rng.standard_normal(ref.read(out).shape).astype(np.float32)
                ref.backward_with(out, G)
                Gs.append(G)
            got = ref.grad(p).reshape(shape)
        want = O.reduce_bwd(kind, shape, axis, Gs[1], None, O.reduce_bwd(kind, shape, axis, Gs[0]))
        assert_bits(want, got, f"{kind} {shape} axis {axis}")


def _twice(ref, params, make, rng):
    """Two forward + backward passes of make(params) on the reference engine, each with its own
    upstream gradient, the second adding into the gradients the first left: (grads, [G1, G2])."""
    Gs = []
    for _ in range(2):
        out = make(*params)
        G = rng.standard_normal(ref.read(out).shape).astype(np.float32)
        ref.backward_with(out, G)
        Gs.append(G)
    return [ref.grad(p) for p in params], Gs


@ref_only
def test_bit_exact_backwards_accumulate_vs_live_reference():
    """Every bit-exact backward, run twice on the reference so that the second adds into gradients
    that already hold values: unary activations, the four broadcast binary ops (one operand reduced),
    softmax / log_softmax, max, cross entropy and nll.  The oracle's accumulating forms (gi + term,
    in the reference's association) must give the same bits; golden vectors, which start from zero
    gradients, cannot tell those forms from a fused or reassociated one."""
    from tests.ncdrive import Engine
    rng = np.random.default_rng(20261202)
    x = (rng.standard_normal((37, 29)) * 3).astype(np.float32)
    with Engine(O.REF_LIB) as ref:
        L = ref.lib
        for name, kind, s in UNARY:
            (gx,), (G1, G2) = _twice(ref, [ref.param(x)], lambda p: Engine.UNARY_CALLS[name](L, p, s), rng)
            y = O.unary_fwd(kind, x, s)
            want = O.unary_bwd(kind, x, y, G2, O.unary_bwd(kind, x, y, G1, s=s), s)
            assert_bits(want, gx.reshape(x.shape), f"{name} accumulated")
            ref.step_end()
        for bshape in ((1, 29), (37, 29)):  # b broadcast over rows (grad b reduced), and the same shape
            b = (0.5 + rng.random(bshape)).astype(np.float32)
            for op, fn in (("add", L.nc_add), ("sub", L.nc_sub), ("mul", L.nc_mul), ("div", L.nc_div)):
                (ga, gb), (G1, G2) = _twice(ref, [ref.param(x), ref.param(b)], fn, rng)
                a1, b1 = O.binary_bwd(op, x, b, G1)
                a2, b2 = O.binary_bwd(op, x, b, G2, ga0=a1, gb0=b1)
                assert_bits(a2, ga.reshape(x.shape), f"{op} b{bshape} grad a accumulated")
                # a reduced grad b sums 37 rows in the reference's row_acc order, restated by the oracle
                assert_bits(b2, gb.reshape(b.shape), f"{op} b{bshape} grad b accumulated")
                ref.step_end()
        for log_form, fn in ((False, L.nc_softmax), (True, L.nc_log_softmax)):
            (gx,), (G1, G2) = _twice(ref, [ref.param(x)], fn, rng)
            y = O.softmax_fwd(x, log_form)
            want = O.softmax_bwd(y, G2, log_form, O.softmax_bwd(y, G1, log_form))
            assert_bits(want, gx.reshape(x.shape), f"softmax log={log_form} accumulated")
            ref.step_end()
        for axis in (0, 1):
            (gx,), (G1, G2) = _twice(ref, [ref.param(x)], lambda p: L.nc_max(p, axis, 0), rng)
            _, arg = O.reduce_fwd("max", x, axis)
            want = O.reduce_bwd("max", x.shape, axis, G2, arg, O.reduce_bwd("max", x.shape, axis, G1, arg))
            assert_bits(want, gx.reshape(x.shape), f"max axis {axis} accumulated")
            ref.step_end()
        lab = rng.integers(0, x.shape[1], x.shape[0]).astype(np.int32)
        _, prob = O.cross_entropy_fwd(x, lab)
        (gx,), (G1, G2) = _twice(ref, [ref.param(x)], lambda p: L.nc_cross_entropy(p, ref.tensor(lab)), rng)
        want = O.cross_entropy_bwd(prob, lab, float(G2), O.cross_entropy_bwd(prob, lab, float(G1)))
        assert_bits(want, gx.reshape(x.shape), "cross_entropy accumulated")
        ref.step_end()
        for sm in (0, 1):
            (gx,), (G1, G2) = _twice(ref, [ref.param(x)], lambda p: L.nc_nll_loss(p, ref.tensor(lab), sm), rng)
            want = O.nll_loss_bwd(x.shape, lab, float(G2), bool(sm), O.nll_loss_bwd(x.shape, lab, float(G1), bool(sm)))
            assert_bits(want, gx.reshape(x.shape), f"nll sum={sm} accumulated")
            ref.step_end()


# ------------------------------------------------------------------------------------------------
# closed forms, invariants and the reference's own known answers
# ------------------------------------------------------------------------------------------------
def test_optim_closed_forms():
    rng = np.random.default_rng(4)
    w0 = rng.standard_normal(1000).astype(np.float32)
    g = rng.standard_normal(1000).astype(np.float32)
    # plain SGD: w - lr * g in fp32
    w, _, _ = O.optim_step("sgd", w0.copy(), g, None, None, lr=0.1)
    assert_bits(w, (w0 - np.float32(0.1) * g).astype(np.float32), "sgd")
    # Adam's first step moves each weight by ~lr in the direction of -g (bias-corrected m / sqrt(v) = sign)
    m, v = np.zeros_like(w0), np.zeros_like(w0)
    b1, b2 = np.float32(0.9), np.float32(0.999)
    w, m, v = O.optim_step("adam", w0.copy(), g, m, v, lr=0.01, beta1=b1, beta2=b2, eps=1e-8,
                           bc1=np.float32(1) - O.powf(b1, 1), bc2=np.float32(1) - O.powf(b2, 1))
    big = np.abs(g) > 1e-2
    assert np.allclose((w0 - w)[big], 0.01 * np.sign(g[big]), rtol=1e-3)
    one_m_b1, one_m_b2 = np.float64(np.float32(1) - b1), np.float64(np.float32(1) - b2)  # fp32 constants
    assert np.allclose(m, one_m_b1 * g, rtol=1e-6) and np.allclose(v, one_m_b2 * g * g, rtol=1e-6)
    # AdamW's decay multiplies the weights before the Adam update; with g = 0 only the decay acts
    z = np.zeros_like(g)
    w, _, _ = O.optim_step("adamw", w0.copy(), z, np.zeros_like(w0), np.zeros_like(w0), lr=0.1, weight_decay=0.5,
                           beta1=b1, beta2=b2, eps=1e-8, bc1=np.float32(0.1), bc2=np.float32(0.001))
    assert_bits(w, (w0 * (np.float32(1) - np.float32(0.1) * np.float32(0.5))).astype(np.float32), "adamw decay")
    # clip: the clipped grads' norm is max_norm; below the threshold nothing changes
    total, gc = O.clip_grad_norm([g, 2 * g], 1.0)
    assert abs(float(total) - float(np.sqrt(5 * (g.astype(np.float64) ** 2).sum()))) <= 1e-6 * float(total)
    assert abs(np.sqrt(sum((x.astype(np.float64) ** 2).sum() for x in gc)) - 1.0) < 1e-5
    total, gc = O.clip_grad_norm([g], 1e9)
    assert_bits(gc[0], g, "no clip")


def test_loss_closed_forms():
    rng = np.random.default_rng(5)
    # uniform logits: every row's loss is log(C), every probability 1/C
    for C in (1, 2, 7, 1000):
        loss, prob = O.cross_entropy_fwd(np.full((3, C), 2.5, np.float32), np.zeros(3, np.int32))
        assert abs(float(loss) - math.log(C)) <= 4e-7 * max(1.0, math.log(C))
        assert np.allclose(prob, 1.0 / C, rtol=2e-7)
    x = (rng.standard_normal((50, 40)) * 3).astype(np.float32)
    lab = rng.integers(0, 40, 50).astype(np.int32)
    loss, prob = O.cross_entropy_fwd(x, lab)
    X = x.astype(np.float64)
    lse = X.max(1) + np.log(np.exp(X - X.max(1, keepdims=True)).sum(1))
    want = float(np.mean(lse - X[np.arange(50), lab]))
    assert abs(float(loss) - want) <= 1e-5 * abs(want)
    # cross entropy = nll of the log-softmax (same arithmetic, same rows)
    assert O.nll_loss_fwd(O.softmax_fwd(x, log_form=True), lab) == loss
    # gradient of the mean loss: (prob - onehot) / N; each row sums to ~0
    gx = O.cross_entropy_bwd(prob, lab, 1.0)
    onehot = np.zeros_like(X)
    onehot[np.arange(50), lab] = 1.0
    assert np.allclose(gx, (prob - onehot) / 50, atol=1e-7)
    assert np.abs(gx.sum(1)).max() < 1e-7
    # nll: mean = sum / N; gradient -G at the label only, scaled by 1/N for the mean
    assert O.nll_loss_fwd(x, lab, True) == np.float32(-np.float64(x[np.arange(50), lab]).sum())
    g = O.nll_loss_bwd(x.shape, lab, 2.0, sum=False)
    assert (g[np.arange(50), lab] == np.float32(-2.0 / 50)).all() and np.count_nonzero(g) == 50
    # rows sharing a label accumulate
    g2 = O.nll_loss_bwd((2, 3), np.array([1, 1], np.int32), 1.0, sum=True)
    assert g2.tolist() == [[0, -1, 0], [0, -1, 0]]
def test_known_answers_from_reference_tests():
    # engine/tests/test_main.c:335-341
    t = np.array([-1.0, 0.5, 4.0], np.float32)
    assert abs(O.unary_fwd("hardswish", t)[1] - 0.5 * 3.5 / 6.0) <= 1e-6
    assert O.unary_fwd("relu6", t)[2] == 4.0
    assert abs(O.unary_fwd("gelu", t)[0] - (-0.15865525)) <= 1e-6
    assert abs(O.unary_fwd("gelu_tanh", t)[0] - (-0.15880801)) <= 1e-6
    assert abs(O.unary_fwd("silu", t)[1] - 0.5 / (1.0 + math.exp(-0.5))) <= 1e-6
    # :118-131 reductions
    a = np.array([[1, 5, 3], [4, 2, 6]], np.float32)
    assert O.reduce_fwd("sum", a, 0)[0][1] == 7
    assert O.reduce_fwd("sum", a, 1)[0][1] == 12
    assert abs(O.reduce_fwd("mean", a, -128)[0][0] - 3.5) <= 1e-6
    assert O.reduce_fwd("max", a, 1)[0][0] == 5
    assert O.reduce_fwd("argmax", a, 1)[0][1] == 2
    # :82-95 broadcasting
    A = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    B = np.array([10, 20, 30], np.float32)
    assert O.binary_fwd("add", A, B)[1, 2] == 36
    assert O.binary_fwd("mul", np.array([[2], [3]], np.float32), B.reshape(1, 3))[1, 1] == 60
    assert O.binary_fwd("sub", np.array(1.0, np.float32), B)[2] == -29
    # :736-745 layer norm: zero mean, unit variance
    y, _ = O.layer_norm_fwd(np.array([1, 2, 3, 6], np.float32), 4, eps=0.0)
    assert abs(y.astype(np.float64).mean()) <= 1e-6 and abs(y.astype(np.float64).var() - 1) <= 1e-5
    # :747-756 softmax of a -inf entry is exactly 0
    p = O.softmax_fwd(np.array([[0.5, -np.inf, -2.0, -np.inf]], np.float32))
    assert p[0, 1] == 0 and p[0, 3] == 0 and abs(p[0, 0] + p[0, 2] - 1) <= 1e-6


def test_transcendental_accuracy_vs_libm():
    """kernel parity bounds of engine/tests/test_main.c:818-869 against libm (math module)."""
    x = np.linspace(-100, 100, 203, dtype=np.float32)
    x[:5] = [0.0, 1e-6, -0.2, 0.249, 0.251]
    e, s, t = O.vmap("exp", x), O.vmap("sigmoid", x), O.vmap("tanh", x)
    for i, v in enumerate(x.astype(np.float64)):
        if -87 <= v <= 88:
            assert abs(e[i] - math.exp(v)) <= 1e-6 * math.exp(v)
            sv = 1 / (1 + math.exp(-v))
            assert abs(s[i] - sv) <= 1e-6 * sv
        tv = math.tanh(v)
        assert abs(t[i] - tv) <= 1e-5 * max(abs(tv), 1e-30)
    xe = np.concatenate([x, np.linspace(-4, 3.8, 40, dtype=np.float32)])
    er = O.vmap("erf", xe)
    assert max(abs(er[i] - math.erf(float(v))) for i, v in enumerate(xe)) < 5e-7
    assert abs(O.vmap("tanh", np.array([1e-6], np.float32))[0] - 1e-6) <= 1e-12
    sp = O.vmap("exp", np.array([-np.inf, np.inf, np.nan, -95.0, 100.0], np.float32))
    assert sp[0] == 0 and sp[1] == np.inf and np.isnan(sp[2]) and sp[3] == 0 and sp[4] == np.inf


def test_sum_order_is_the_avx2_tree():
    """A wrong lane pairing changes the rounding: pick values where only the exact tree gives the
    stored golden answer, and check against an fp64 sum for the magnitude."""
    x = np.array([1e8, 1, -1e8, 1, 3, 5, 7, 9, 1e8, 2, -1e8, 4, 6, 8, 10, 12, 0.5], np.float32)
    s = O.sum_f32(x)
    a0 = x[0:8].astype(np.float32)
    a1 = x[8:16].astype(np.float32)
    v = a0 + a1
    want = np.float32(np.float32(np.float32(v[0] + v[4]) + np.float32(v[2] + v[6])) +
                      np.float32(np.float32(v[1] + v[5]) + np.float32(v[3] + v[7])))
    want = np.float32(want + x[16])
    assert s == want


def test_binary_bwd_against_fp64_brute_force():
    rng = np.random.default_rng(3)
    a = rng.standard_normal((4, 1, 6)).astype(np.float32)
    b = (0.5 + rng.random((5, 1))).astype(np.float32)
    g = rng.standard_normal((4, 5, 6)).astype(np.float32)
    A, B, G = (v.astype(np.float64) for v in (a, b, g))
    for op, da, db in (("add", G, G), ("sub", G, -G), ("mul", G * B, G * A), ("div", G / B, -G * A / (B * B))):
        ga, gb = O.binary_bwd(op, a, b, g)
        want_a = da.sum(axis=1, keepdims=True)
        want_b = db.sum(axis=(0, 2)).reshape(5, 1)
        np.testing.assert_allclose(ga, want_a, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(gb, want_b, rtol=1e-5, atol=1e-5)


def test_softmax_and_layernorm_against_fp64():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((7, 300)) * 3).astype(np.float32)
    X = x.astype(np.float64)
    p = np.exp(X - X.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    np.testing.assert_allclose(O.softmax_fwd(x), p, rtol=2e-6, atol=1e-9)
    np.testing.assert_allclose(O.softmax_fwd(x, True), np.log(p), rtol=1e-5, atol=1e-5)
    g = rng.standard_normal(x.shape)
    gx = O.softmax_bwd(O.softmax_fwd(x), g)
    want = p * (g - (g * p).sum(1, keepdims=True))
    np.testing.assert_allclose(gx, want, rtol=1e-4, atol=1e-6)
    w = (1 + 0.1 * rng.standard_normal(300)).astype(np.float32)
    b = (0.1 * rng.standard_normal(300)).astype(np.float32)
    y, stats = O.layer_norm_fwd(x, 300, w, b)
    mu = X.mean(1, keepdims=True)
    xh = (X - mu) / np.sqrt(X.var(1, keepdims=True) + 1e-5)
    np.testing.assert_allclose(y, xh * w + b, rtol=1e-5, atol=1e-5)
    gx, gw, gb = O.layer_norm_bwd(x, 300, stats, g.astype(np.float32), w, True, True)
    gh = g * w
    want = (gh - gh.mean(1, keepdims=True) - xh * (gh * xh).mean(1, keepdims=True)) / np.sqrt(
        X.var(1, keepdims=True) + 1e-5)
    np.testing.assert_allclose(gx, want, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(gw, (g * xh).sum(0), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(gb, g.sum(0), rtol=1e-4, atol=1e-4)


def test_quantize_closed_form():
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((33, 65)) * 0.02).astype(np.float32)
    w[0, 0] = 1.0
    q, s = O.quantize_rows(w)
    amax = np.abs(w).max(1)
    s_want = (amax / np.float32(127)).astype(np.float32)
    assert_bits(s, s_want)
    inv = (np.float32(1) / s_want).astype(np.float32)
    q_want = np.clip(np.rint((w * inv[:, None]).astype(np.float32)), -127, 127).astype(np.int8)
    assert_bits(q, q_want)
    assert q.min() >= -127
    assert_bits(O.dequantize_rows(q, s), (q.astype(np.float32) * s[:, None]).astype(np.float32))


def test_argmax_first_index_and_nan_rule():
    x = np.array([[1, 3, 3, 2], [np.nan, 5, 6, 7], [1, np.nan, 9, 9], [-0.0, 0.0, -1, -2]], np.float32)
    got, _ = O.reduce_fwd("argmax", x, 1)
    assert list(got) == [1, 0, 2, 0]
    mx, _ = O.reduce_fwd("max", x, 1)
    assert mx[0] == 3 and np.isnan(mx[1]) and mx[2] == 9 and np.signbit(mx[3])


LIBM = [("log", 0.0), ("sqrt", 0.0), ("pow", 2.0), ("pow", 3.0), ("pow", 0.5), ("pow", -1.5), ("pow", 1.7),
        ("neg", 0.0), ("scale", -2.5), ("add_scalar", 0.75)]


@ref_only
@pytest.mark.parametrize("name,s", LIBM)
def test_libm_unary_vs_live_reference(name, s):
    """log, sqrt and pow call libm in the reference (ops_elementwise.c:233-234, 240; backward :305-306,
    312), neg / scale / add_scalar its scale and axpy kernels: forward and accumulated backward against
    the oracle bit for bit, positive inputs across the exponent range plus zero, negative, infinite,
    subnormal and NaN values."""
    from tests.ncdrive import Engine
    rng = np.random.default_rng(zlib.crc32(f"{name}/{s}".encode()))
    x = np.concatenate([np.exp(rng.uniform(-80, 80, 20_000)).astype(np.float32),
                        rng.standard_normal(2_000).astype(np.float32),
                        np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-40, 1e-45, 4.0, 0.25],
                                 np.float32)])
    with Engine(O.REF_LIB) as ref:
        (gx,), (G1, G2) = _twice(ref, [ref.param(x)], lambda p: Engine.UNARY_CALLS[name](ref.lib, p, s), rng)
        y_ref = ref.read(Engine.UNARY_CALLS[name](ref.lib, ref.param(x), s))
    y = O.unary_fwd(name, x, s)
    assert_bits(y, y_ref, f"{name} {s} fwd")
    assert_bits(O.unary_bwd(name, x, y, G2, O.unary_bwd(name, x, y, G1, s=s), s), gx, f"{name} {s} bwd accumulated")


def test_libm_unary_closed_forms():
    """sqrt of exact squares is exact; log(1) = 0, log(e^k) within an ulp of k; pow(x, 1) = x,
    pow(x, 2) within an ulp of x*x; the backward of log is g / x and of sqrt g * 0.5 / sqrt(x)."""
    rng = np.random.default_rng(9)
    r = rng.integers(1, 4096, 1000).astype(np.float32)
    assert_bits(O.unary_fwd("sqrt", r * r), r, "sqrt of squares")
    assert O.unary_fwd("log", np.array([1.0], np.float32))[0] == 0.0
    k = np.arange(-20, 21).astype(np.float32)
    lg = O.unary_fwd("log", np.exp(k.astype(np.float64)).astype(np.float32))
    assert np.all(np.abs(lg - k) <= 4 * np.spacing(np.maximum(np.abs(k), 1))), "log(e^k)"
    x = (rng.random(1000) * 100).astype(np.float32)
    assert_bits(O.unary_fwd("pow", x, 1.0), x, "pow(x, 1)")
    sq = O.unary_fwd("pow", x, 2.0)
    assert np.all(np.abs(sq - x * x) <= np.spacing(x * x)), "pow(x, 2)"
    g = rng.standard_normal(1000).astype(np.float32)
    assert_bits(O.unary_bwd("log", x, None, g), g / x, "d log")
    y = O.unary_fwd("sqrt", x)
    assert_bits(O.unary_bwd("sqrt", x, y, g), (g * np.float32(0.5)) / y, "d sqrt")
