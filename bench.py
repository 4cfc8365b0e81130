"""Benchmark of the hot path on one MI355X: achieved HBM GB/s (and % of peak) per op class, and
elements/s against the reference engine on the host CPU.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--classes all|none] [--no-cpu]

A step is one pass of the headline workload over its synthetic batch: the six activations (GELU
(erf), SiLU, Sigmoid, Tanh, Hardswish, ReLU6) each forward y = f(x) and backward gi += f'(.) * g over
2^28 fp32 elements resident in HBM.  `value` is the step's algorithmic bytes (forward 8 B/element:
read x, write y; backward 16 B/element: read x or y, read g, read+write gi) over the timed wall
time.  Every kernel launch is bracketed by HIP events on the launch stream; the per-kernel averages
give `classes` (GB/s per op class, also for the broadcast / row-reduction / int8 / full-sum
workloads unless --classes none; `gemm`: TFLOP/s against the matrix-core peaks for the fp32 and int8
linear / batched-matmul contractions) and the `roofline` of the dominant kernel; `chain` is the
launch-bound MNIST-CNN chain (add-bias, ReLU, two sums, backward) through the engine's nc.h API, in
microseconds per iteration.  `cpu_baseline` times the reference engine (oracle/_ref/libnc_ref.so, its
own threaded AVX2 path) on a bounded sample of the same work, and the same chain.  Prints one JSON
line.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_GBS = 8000.0  # MI355X HBM3E
METRIC = "achieved HBM GB/s (% of MI355X peak) per op class; elements/s vs host CPU"
ACTS = ["gelu", "silu", "sigmoid", "tanh", "hardswish", "relu6"]
N_UNARY = 1 << 28


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timeline:
    """Per-launch HIP event pairs, grouped by kernel label."""

    def __init__(self, hm):
        self.hm = hm
        self.pending = []
        self.stats = {}

    def run(self, label, nbytes, fn):
        e0, e1 = self.hm.Event(), self.hm.Event()
        e0.record()
        fn()
        e1.record()
        self.pending.append((label, nbytes, e0, e1))

    def collect(self):
        for label, nbytes, e0, e1 in self.pending:
            e1.synchronize()
            ms = e0.elapsed_ms(e1)
            s = self.stats.setdefault(label, {"bytes": nbytes, "ms": [], })
            s["ms"].append(ms)
        self.pending.clear()

    def summary(self):
        out = {}
        for label, s in self.stats.items():
            ms = float(np.median(s["ms"]))
            gbs = s["bytes"] / (ms * 1e-3) / 1e9
            out[label] = {"GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4), "us": round(ms * 1e3, 1),
                          "bytes": s["bytes"], "launches": len(s["ms"])}
        return out


def unary_workload(K, hm, n):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(n, dtype=np.float32)
    g = np.random.default_rng(2).standard_normal(n, dtype=np.float32)
    # two buffer sets, alternated between activations, so no kernel finds its inputs in the 256 MB
    # MALL from the previous one (each set is 4 GiB; consecutive uses of a set are >= 3 GiB apart)
    sets = []
    for _ in range(2):
        X, G = hm.DeviceBuffer.from_numpy(x), hm.DeviceBuffer.from_numpy(g)
        Y, GI = hm.DeviceBuffer(4 * n), hm.DeviceBuffer(4 * n)
        GI.zero()
        sets.append((X, G, Y, GI))
    del x, g
    from newch_amd.hip import BWD_READS_Y

    def step(tl):
        for i, act in enumerate(ACTS):
            X, G, Y, GI = sets[i % 2]
            tl.run(f"{act}_fwd", 8 * n, lambda a=act, X=X, Y=Y: K.unary_fwd(a, X.ptr, Y.ptr, n))
            reads_y = act in BWD_READS_Y
            tl.run(f"{act}_bwd", 16 * n,
                   lambda a=act, ry=reads_y, X=X, Y=Y, G=G, GI=GI:
                   K.unary_bwd(a, 0 if ry else X.ptr, Y.ptr if ry else 0, G.ptr, GI.ptr, n, accumulate=True))

    return step, 24 * n * len(ACTS), sets[0]


def class_workloads(K, hm):
    """Per-op-class workloads of the other configurations: (label, bytes, launcher) lists."""
    work = []
    keep = []
    # broadcast binary: a[64,512,1,64] (one 2^30-output chunk of a[256,512,1,64]) op b[1,1,512,64]
    blk = np.random.default_rng(3).standard_normal(1 << 21, dtype=np.float32)
    A = hm.DeviceBuffer.from_numpy(blk)
    Bv = hm.DeviceBuffer.from_numpy((0.5 + 1.5 * np.random.default_rng(4).random(512 * 64)).astype(np.float32))
    n_out = 1 << 30
    O = hm.DeviceBuffer(4 * n_out)
    shape = (64, 512, 512, 64)
    sa, sb, so = (32768, 64, 0, 1), (0, 0, 64, 1), (1 << 24, 1 << 15, 64, 1)
    keep += [A, Bv, O]
    fwd_bytes = 4 * n_out + 4 * (1 << 21) + 4 * 512 * 64
    for op in ("add", "mul", "div"):
        work.append((f"bcast_{op}_fwd", fwd_bytes,
                     lambda op=op: K.binary_fwd(op, shape, A.ptr, sa, Bv.ptr, sb, O.ptr, so)))
    # transposed view of a: storage [512(c),64(n),1,64] seen as [64,512,1,64] -> strides (64, 4096, 0, 1).
    # Timed as the engine runs it: the view is re-read 512x, so it is gathered to contiguous memory
    # first, then the broadcast kernel streams the output.
    AB = hm.DeviceBuffer(4 * (1 << 21))
    keep.append(AB)

    def batch_transposed():
        K.copy_strided(4, (64, 512, 1, 64), A.ptr, (64, 4096, 0, 1), AB.ptr)
        K.binary_fwd("add", shape, AB.ptr, sa, Bv.ptr, sb, O.ptr, so)
    work.append(("bcast_add_fwd_transposed_a", fwd_bytes, batch_transposed))
    # innermost-strided view of a: storage [64(n),64(w),512(c)] .transpose(1,2) .reshape(64,512,1,64)
    # -> strides (32768, 1, 0, 512).  Timed as the engine runs it: the 8 MiB operand is gathered to
    # contiguous memory, then the broadcast kernel streams the output.
    AT = hm.DeviceBuffer(4 * (1 << 21))
    keep.append(AT)

    def inner_strided():
        K.copy_strided(4, (64, 512, 1, 64), A.ptr, (32768, 1, 0, 512), AT.ptr)
        K.binary_fwd("add", shape, AT.ptr, sa, Bv.ptr, sb, O.ptr, so)
    work.append(("bcast_add_fwd_inner_strided_a", fwd_bytes, inner_strided))
    # backward of add: grad_a (sum over h) and grad_b (sum over n, c) from g = O
    GA, GB = hm.DeviceBuffer(4 * (1 << 21)), hm.DeviceBuffer(4 * 512 * 64)
    GA.zero(), GB.zero()
    sga, sgb = (32768, 64, 0, 1), (0, 0, 64, 1)
    wsb = max(K.binary_bwd_workspace(shape, sga), K.binary_bwd_workspace(shape, sgb),
              K.binary_bwd2_workspace(shape, sga, sgb))
    WS = hm.DeviceBuffer(max(wsb, 1))
    keep += [GA, GB, WS]
    # both gradients in one pass over g (g read, grad_a and grad_b read-modify-written, a and b read
    # where the op needs them)
    for op in ("add", "mul", "div"):
        ab = 0 if op == "add" else 4 * (1 << 21) + 4 * 512 * 64
        work.append((f"bcast_{op}_bwd", 4 * n_out + 8 * (1 << 21) + 8 * 512 * 64 + ab,
                     lambda op=op: K.binary_bwd2(op, shape, O.ptr, so, A.ptr, sa, Bv.ptr, sb, GA.ptr, sga, GB.ptr,
                                                 sgb, WS.ptr, wsb)))
    # one operand at a time (the path when only one operand needs a gradient)
    work.append(("bcast_add_bwd_grad_a", 4 * n_out + 8 * (1 << 21),
                 lambda: K.binary_bwd("add", 0, shape, O.ptr, so, A.ptr, sa, Bv.ptr, sb, GA.ptr, sga, WS.ptr, wsb)))
    work.append(("bcast_add_bwd_grad_b", 4 * n_out + 8 * 512 * 64,
                 lambda: K.binary_bwd("add", 1, shape, O.ptr, so, A.ptr, sa, Bv.ptr, sb, GB.ptr, sgb, WS.ptr, wsb)))
    # row reductions X[65536, 1024]
    rows, C = 65536, 1024
    X = hm.DeviceBuffer.from_numpy((np.random.default_rng(7).standard_normal((rows, C), dtype=np.float32) * 2))
    Y, G, GI = hm.DeviceBuffer(4 * rows * C), hm.DeviceBuffer(4 * rows * C), hm.DeviceBuffer(4 * rows * C)
    G.upload(np.random.default_rng(9).standard_normal((rows, C), dtype=np.float32))
    GI.zero()
    W = hm.DeviceBuffer.from_numpy((1 + 0.1 * np.random.default_rng(8).standard_normal(C)).astype(np.float32))
    Bb = hm.DeviceBuffer.from_numpy((0.1 * np.random.default_rng(8).standard_normal(C)).astype(np.float32))
    S = hm.DeviceBuffer(8 * rows)
    GW, GBb = hm.DeviceBuffer(4 * C), hm.DeviceBuffer(4 * C)
    GW.zero(), GBb.zero()
    lnws = K.layer_norm_bwd_workspace(rows, C)
    LWS = hm.DeviceBuffer(max(lnws, 1))
    M, AR = hm.DeviceBuffer(4 * rows), hm.DeviceBuffer(4 * rows)
    keep += [X, Y, G, GI, W, Bb, S, GW, GBb, LWS, M, AR]
    e = rows * C
    work += [
        ("softmax_fwd", 8 * e, lambda: K.softmax_fwd(False, rows, C, X.ptr, Y.ptr)),
        ("softmax_bwd", 16 * e, lambda: K.softmax_bwd(False, rows, C, Y.ptr, G.ptr, GI.ptr)),
        ("log_softmax_fwd", 8 * e, lambda: K.softmax_fwd(True, rows, C, X.ptr, Y.ptr)),
        ("log_softmax_bwd", 16 * e, lambda: K.softmax_bwd(True, rows, C, Y.ptr, G.ptr, GI.ptr)),
        ("layer_norm_fwd", 8 * e + 8 * rows, lambda: K.layer_norm_fwd(rows, C, X.ptr, W.ptr, Bb.ptr, 1e-5, Y.ptr, S.ptr)),
        ("layer_norm_bwd", 16 * e + 8 * rows,
         lambda: K.layer_norm_bwd(rows, C, X.ptr, W.ptr, S.ptr, G.ptr, GI.ptr, GW.ptr, GBb.ptr, LWS.ptr, lnws)),
        ("max_argmax", 4 * e + 8 * rows, lambda: K.reduce_fwd("max", rows, C, 1, X.ptr, M.ptr, AR.ptr)),
    ]
    # cross entropy over the same rows with labels ~ U[0, 1024): fwd reads x, writes prob (8 B/el);
    # bwd reads prob, read-modify-writes gi (12 B/el)
    LAB = hm.DeviceBuffer.from_numpy(np.random.default_rng(10).integers(0, C, rows).astype(np.int32))
    LS, BADF = hm.DeviceBuffer(4), hm.DeviceBuffer(8)
    GO = hm.DeviceBuffer.from_numpy(np.array([1.0], np.float32))
    lws = K.loss_workspace(rows, C)
    LWS2 = hm.DeviceBuffer(max(lws, 8))
    keep += [LAB, LS, BADF, GO, LWS2]
    work += [
        ("cross_entropy_fwd", 8 * e + 4 * rows,
         lambda: K.cross_entropy_fwd(rows, C, X.ptr, LAB.ptr, Y.ptr, LS.ptr, BADF.ptr, LWS2.ptr, lws)),
        ("cross_entropy_bwd", 12 * e + 4 * rows,
         lambda: K.cross_entropy_bwd(rows, C, Y.ptr, LAB.ptr, GO.ptr, GI.ptr, accumulate=True)),
    ]
    # int8: 48 x W[4096, 4096] quantize per row, dequantize back
    qrows, qcols = 48 * 4096, 4096
    blkw = (np.random.default_rng(11).standard_normal((4096, 4096), dtype=np.float32) * 0.02)
    Wq = hm.DeviceBuffer(4 * qrows * qcols)
    for m in range(48):
        Wq.upload(blkw, offset=m * blkw.nbytes)
    Q, SC, DQ = hm.DeviceBuffer(qrows * qcols), hm.DeviceBuffer(4 * qrows), hm.DeviceBuffer(4 * qrows * qcols)
    keep += [Wq, Q, SC, DQ]
    qe = qrows * qcols
    work += [
        ("quantize_rows", 5 * qe + 4 * qrows, lambda: K.quantize_rows(qrows, qcols, Wq.ptr, Q.ptr, SC.ptr)),
        ("dequantize_rows", 5 * qe + 4 * qrows, lambda: K.dequantize_rows(qrows, qcols, Q.ptr, SC.ptr, DQ.ptr)),
    ]
    # optimizer step over 2^26 parameters: Adam reads w, g, m, v and writes w, m, v (28 B/param), SGD
    # with momentum reads w, g, v and writes w, v (20 B/param); clip_grad_norm's fp64 sum of squares
    # reads g (4 B/param)
    npar = 1 << 26
    PW = hm.DeviceBuffer.from_numpy(np.random.default_rng(12).standard_normal(npar, dtype=np.float32))
    PG = hm.DeviceBuffer.from_numpy(np.random.default_rng(13).standard_normal(npar, dtype=np.float32))
    PM, PV = hm.DeviceBuffer(4 * npar), hm.DeviceBuffer(4 * npar)
    PM.zero(), PV.zero()
    SSD = hm.DeviceBuffer(8)
    sws = K.sumsq_workspace(npar)
    SWS = hm.DeviceBuffer(max(sws, 8))
    keep += [PW, PG, PM, PV, SSD, SWS]
    work += [
        ("adam_step", 28 * npar,
         lambda: K.optim_step("adam", npar, PW.ptr, PG.ptr, PM.ptr, PV.ptr, 1e-3, 0.0, 0.0, 0.9, 0.999, 1e-8, 1.0,
                              0.1, 0.001)),
        ("sgd_momentum_step", 20 * npar,
         lambda: K.optim_step("sgd", npar, PW.ptr, PG.ptr, PM.ptr, None, 1e-3, 0.9, 0.0)),
        ("grad_sumsq", 4 * npar, lambda: K.sumsq(npar, PG.ptr, SSD.ptr, False, SWS.ptr, sws)),
    ]
    # full sum / mean over 2^30 fp32 (the bcast output buffer holds 2^30 values)
    fws = K.reduce_workspace("sum", 1, n_out, 1)
    FWS, FS = hm.DeviceBuffer(max(fws, 1)), hm.DeviceBuffer(4)
    keep += [FWS, FS]
    work += [
        ("full_sum", 4 * n_out, lambda: K.reduce_fwd("sum", 1, n_out, 1, O.ptr, FS.ptr, 0, FWS.ptr, fws)),
        ("full_mean", 4 * n_out, lambda: K.reduce_fwd("mean", 1, n_out, 1, O.ptr, FS.ptr, 0, FWS.ptr, fws)),
    ]
    return work, keep


PEAK_F32_TFLOPS = 157.3   # MI355X dense fp32 matrix
PEAK_I8_TOPS = 5000.0     # MI355X dense int8 matrix


def gemm_workloads(K, hm):
    """Dense contractions at a transformer-linear shape: x [8192, 4096] through a [4096, 4096] weight
    (forward NT, the two backward GEMMs NN and TN), the int8 linear (row quantization + int8 MFMA GEMM
    + fused dequant/bias epilogue) and its bare int8 GEMM, and an attention-shaped batched product
    (64 x [1024, 128] @ [128, 1024], B a transposed view).  Items: label, ops per launch, peak, fn."""
    rng = np.random.default_rng(21)
    M, Kd, N = 8192, 4096, 4096
    X = hm.DeviceBuffer.from_numpy(rng.standard_normal((M, Kd), dtype=np.float32))
    W = hm.DeviceBuffer.from_numpy((rng.standard_normal((N, Kd), dtype=np.float32) * 0.02).astype(np.float32))
    G = hm.DeviceBuffer.from_numpy(rng.standard_normal((M, N), dtype=np.float32))
    Y, GX, GW = hm.DeviceBuffer(4 * M * N), hm.DeviceBuffer(4 * M * Kd), hm.DeviceBuffer(4 * N * Kd)
    WQ, WS = hm.DeviceBuffer(N * Kd), hm.DeviceBuffer(4 * N)
    K.quantize_rows(N, Kd, W.ptr, WQ.ptr, WS.ptr)
    BIAS = hm.DeviceBuffer.from_numpy(rng.standard_normal(N, dtype=np.float32))
    XQ, XS = hm.DeviceBuffer(M * Kd), hm.DeviceBuffer(4 * M)
    K.quantize_rows(M, Kd, X.ptr, XQ.ptr, XS.ptr)
    C32 = hm.DeviceBuffer(4 * M * N)
    qws = K.linear_int8_workspace(M, Kd)
    QWS = hm.DeviceBuffer(qws)
    Bh, S, D = 64, 1024, 128
    QA = hm.DeviceBuffer.from_numpy(rng.standard_normal((Bh, S, D), dtype=np.float32))
    KB = hm.DeviceBuffer.from_numpy(rng.standard_normal((Bh, S, D), dtype=np.float32))
    SC = hm.DeviceBuffer(4 * Bh * S * S)
    keep = [X, W, G, Y, GX, GW, WQ, WS, BIAS, XQ, XS, C32, QWS, QA, KB, SC]
    f = 2.0 * M * N * Kd
    work = [
        ("linear_fwd_sgemm_nt", f, PEAK_F32_TFLOPS,
         lambda: K.gemm_f32(0, 1, M, N, Kd, 1.0, X.ptr, Kd, W.ptr, Kd, 0.0, Y.ptr, N)),
        ("linear_bwd_dx_sgemm_nn", f, PEAK_F32_TFLOPS,
         lambda: K.gemm_f32(0, 0, M, Kd, N, 1.0, G.ptr, N, W.ptr, Kd, 0.0, GX.ptr, Kd)),
        ("linear_bwd_dw_sgemm_tn", f, PEAK_F32_TFLOPS,
         lambda: K.gemm_f32(1, 0, N, Kd, M, 1.0, G.ptr, N, X.ptr, Kd, 0.0, GW.ptr, Kd)),
        ("bmm_qk_t_sgemm", 2.0 * Bh * S * S * D, PEAK_F32_TFLOPS,
         lambda: K.gemm_f32_bmm(0, 1, S, S, D, QA.ptr, D, KB.ptr, D, 0.0, SC.ptr, S, [Bh], [S * D], [S * D],
                                [S * S])),
        ("gemm_s8_nt", f, PEAK_I8_TOPS,
         lambda: K.gemm_s8_nt(M, N, Kd, XQ.ptr, Kd, WQ.ptr, Kd, C32.ptr, N)),
        ("linear_int8", f, PEAK_I8_TOPS,
         lambda: K.linear_int8(M, Kd, N, X.ptr, WQ.ptr, WS.ptr, BIAS.ptr, Y.ptr, QWS.ptr, qws)),
    ]
    return work, keep


def measured_traffic(label: str):
    """HBM bytes per launch of `label` from the committed rocprofv3 PMC summary (FETCH_SIZE and
    WRITE_SIZE in KiB, scaled by what the same counters read for a plain copy of known size)."""
    p = ROOT / "profiles" / "hbm_traffic_bench.txt"
    if not p.exists():
        return None
    scale, rows = {}, {}
    for line in p.read_text().splitlines():
        parts = line.split()
        if len(parts) == 2 and parts[0] in ("fetch_scale", "write_scale"):
            scale[parts[0]] = float(parts[1])
        elif len(parts) == 4 and not line.startswith("#") and parts[1].isdigit():
            rows[parts[0]] = (float(parts[2]), float(parts[3]))
    if label not in rows or len(scale) != 2:
        return None
    f, w = rows[label]
    return int(round((f / scale["fetch_scale"] + w / scale["write_scale"]) * 1024))


def chain_latency(lib_path=None, iters: int = 200, warmup: int = 10, threads: int = 0):
    """The chain of the MNIST-CNN configuration through an nc.h engine, as the reference's Python
    layer drives it: h = relu(x + bias) for x[64,16,28,28]~U(-1,1) (seed 0) and bias[1,16,1,1]~U(-0.1,
    0.1) (the same stream, next), s = h.sum(3).sum(2), s.sum().backward(), zero_grad, step_end.
    Returns microseconds per iteration (host wall time, the device synchronised every iteration)."""
    import ctypes

    from newch_amd import abi

    L = abi.load(lib_path)
    cfg = abi.Config(0, 0, 0, threads)
    ctx = L.nc_init(ctypes.byref(cfg))
    rng = np.random.default_rng(0)
    x = rng.uniform(-1, 1, (64, 16, 28, 28)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, (1, 16, 1, 1)).astype(np.float32)

    def param(arr):
        nd, shp = abi.shape_arg(arr.shape)
        src = L.nc_from_data(ctx, abi.F32, arr.ctypes.data_as(ctypes.c_void_p), nd, shp)
        return L.nc_parameter(ctx, src, nd, shp)

    px, pb = param(x), param(b)
    sync = getattr(L, "nc_synchronize", None)

    def one():
        h = L.nc_relu(L.nc_add(px, pb))
        s = L.nc_sum(L.nc_sum(h, 3, 1), 2, 1)
        L.nc_backward(L.nc_sum(s, abi.ALL_AXES, 0))
        if sync is not None:
            sync(ctx)
        L.nc_zero_grad(px)
        L.nc_zero_grad(pb)
        L.nc_step_end(ctx)

    for _ in range(warmup):
        one()
    t0 = time.perf_counter()
    for _ in range(iters):
        one()
    el = time.perf_counter() - t0
    ok = L.nc_ok(ctx)
    L.nc_free_ctx(ctx)
    return round(el / iters * 1e6, 1) if ok else None


def cpu_baseline(budget_s: float = 12.0):
    """The reference engine on host cores: y = f(x); y.sum().backward() per activation (the
    reference's own activation benchmark, tools/bench_act.py:46-52) over a 2^22-element sample."""
    import ctypes

    from newch_amd import abi
    from oracle import pyoracle

    if not pyoracle.REF_LIB.exists():
        return None
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or min(os.cpu_count() or 1, 64)
    threads = min(threads, 64, os.cpu_count() or 1)
    L = abi.load(pyoracle.REF_LIB)
    cfg = abi.Config(0, 1, 0, threads)
    ctx = L.nc_init(ctypes.byref(cfg))
    n = 1 << 22
    x = np.random.default_rng(1).standard_normal(n, dtype=np.float32)
    nd, shp = abi.shape_arg((n,))
    src = L.nc_from_data(ctx, abi.F32, x.ctypes.data_as(ctypes.c_void_p), nd, shp)
    p = L.nc_parameter(ctx, src, nd, shp)
    calls = {"gelu": lambda t: L.nc_gelu(t, 0), "silu": L.nc_silu, "sigmoid": L.nc_sigmoid, "tanh": L.nc_tanh,
             "hardswish": L.nc_hardswish, "relu6": L.nc_relu6}
    backend = L.nc_kernel_backend(ctx).decode()
    t0 = time.perf_counter()
    reps = 0
    while True:
        for act in ACTS:
            y = calls[act](p)
            L.nc_backward(L.nc_sum(y, abi.ALL_AXES, 0))
            L.nc_step_end(ctx)
        reps += 1
        el = time.perf_counter() - t0
        if el > budget_s or reps >= 2000:
            break
    ok = L.nc_ok(ctx)
    L.nc_free_ctx(ctx)
    if not ok:
        return None
    chain_us = chain_latency(pyoracle.REF_LIB, iters=50, warmup=3, threads=threads)
    el_per_s = reps * n * len(ACTS) / el
    return {"value": round(el_per_s * 24 / 1e9, 2), "unit": "GB/s", "elements_per_s": round(el_per_s / 1e6, 1),
            "elements_unit": "M el/s", "cores": threads, "kind": "reference",
            "sample": f"2^22 fp32 elements, {reps} reps of y=f(x); y.sum().backward() for {', '.join(ACTS)} "
                      f"on the reference engine ({backend} kernel tier), "
                      f"{el:.1f} s; GB/s counts the same 24 B/element as the GPU value",
            "chain_us": chain_us,
            "chain_sample": "the MNIST-CNN chain (as `chain`), 50 iterations on the reference engine"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--classes", choices=["all", "none"], default="all")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate", action="store_true",
                    help="also launch a plain copy kernel (y = -x over the same buffers, 8 B/element) so HBM "
                         "counters can be scaled against known bytes")
    ap.add_argument("--elements", type=int, default=N_UNARY, help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one MI355X: the kernels run on one GPU's share "
                                   "and multi-GPU sharding is not implemented"}))
        sys.exit(2)

    from newch_amd import hipmem as hm
    from newch_amd.hip import Kernels

    if hm.device_count() < 1:
        sys.exit("bench.py: no HIP device visible")
    K = Kernels()
    n = args.elements
    log(f"bench: unary workload, {n} elements x {len(ACTS)} activations, warmup {args.warmup}, steps {args.steps}")
    step, step_bytes, _bufs = unary_workload(K, hm, n)
    if args.calibrate:
        X = _bufs[0]
        Y = _bufs[2]
        cal = Timeline(hm)
        for _ in range(3):
            cal.run("copy_calibration", 8 * n, lambda: K.unary_fwd("neg", X.ptr, Y.ptr, n))
        cal.collect()
        log(f"bench: copy calibration {cal.summary()['copy_calibration']}")
    warm = Timeline(hm)
    for _ in range(args.warmup):
        step(warm)
    warm.collect()
    hm.synchronize()
    tl = Timeline(hm)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(tl)
    hm.synchronize()
    wall = time.perf_counter() - t0
    tl.collect()
    classes = tl.summary()
    value = step_bytes * args.steps / wall / 1e9
    dom = max((k for k in classes), key=lambda k: classes[k]["us"])
    d = classes[dom]
    log(f"bench: unary step {wall / args.steps * 1e3:.3f} ms, {value:.1f} GB/s; dominant {dom} {d['GB/s']} GB/s")

    gemm = {}
    if args.classes == "all":
        work, keep = class_workloads(K, hm)
        for label, nbytes, fn in work:  # warm each once, then 5 timed launches
            fn()
        hm.synchronize()
        # cold cache: 1 GiB of scratch written before every timed launch evicts the 256 MB MALL
        # (outside the launch's events)
        flush = hm.DeviceBuffer(1 << 30)
        ctl = Timeline(hm)
        for _ in range(5):
            for label, nbytes, fn in work:
                K.fill(flush.ptr, 4, 0, 1 << 28)
                ctl.run(label, nbytes, fn)
        hm.synchronize()
        ctl.collect()
        extra = ctl.summary()
        for k, v in extra.items():
            log(f"bench: {k:28s} {v['GB/s']:8.1f} GB/s  {100 * v['frac']:5.1f}%  {v['us']:9.1f} us")
        classes.update(extra)
        del keep
        gwork, gkeep = gemm_workloads(K, hm)
        for label, ops, peak, fn in gwork:
            fn()
        hm.synchronize()
        gtl = Timeline(hm)
        for _ in range(5):
            for label, ops, peak, fn in gwork:
                gtl.run(label, ops, fn)
        hm.synchronize()
        gtl.collect()
        for label, ops, peak, fn in gwork:
            ms = float(np.median(gtl.stats[label]["ms"]))
            rate = ops / (ms * 1e-3) / 1e12
            gemm[label] = {"TFLOP/s" if peak == PEAK_F32_TFLOPS else "TOP/s": round(rate, 1), "peak": peak,
                           "frac": round(rate / peak, 4), "us": round(ms * 1e3, 1), "ops": ops,
                           "launches": len(gtl.stats[label]["ms"])}
            log(f"bench: {label:28s} {rate:8.1f} T/s  {100 * rate / peak:5.1f}% of {peak}  {ms * 1e3:9.1f} us")
        del gkeep

    chain_us = chain_latency()
    log(f"bench: MNIST-CNN chain fwd+bwd through the engine {chain_us} us per iteration")
    cpu = None if args.no_cpu else cpu_baseline()
    if cpu:
        log(f"bench: cpu baseline {cpu['value']} GB/s ({cpu['elements_per_s']} M el/s) on {cpu['cores']} threads")
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "unary activations fwd+bwd over 2^28 fp32 elements (x~N(0,1) seed 1, "
                               "g~N(0,1) seed 2): GELU(erf), SiLU, Sigmoid, Tanh, Hardswish, ReLU6",
                   "elements": n, "bytes_per_step": step_bytes},
        "hbm_frac": round(value / PEAK_GBS, 4),
        "elements_per_s": round(n * len(ACTS) * args.steps / wall / 1e9, 3),
        "elements_unit": "G el/s (fwd+bwd pairs)",
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": d["GB/s"], "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": d["frac"], "traffic": measured_traffic(dom), "algorithmic_bytes": d["bytes"]},
        "cpu_baseline": cpu,
        "classes": classes,
        "gemm": gemm,
        "chain": {"workload": "MNIST-CNN chain through nc.h: relu(x[64,16,28,28] + bias[1,16,1,1]), sum over "
                              "dims 3 then 2, sum().backward(), zero_grad, step_end (802,816 elements; "
                              "launch-bound)", "us_per_iter": chain_us},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
