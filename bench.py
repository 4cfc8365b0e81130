"""Benchmark of the hot path on one MI355X: achieved HBM GB/s (and % of peak) per op class, and
elements/s against the reference engine on the host CPU.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--classes all|none] [--no-cpu]
    python bench.py --only LABEL[,LABEL...]        # just those op classes (per-label profiler passes)
    python bench.py --traffic-summary DIR          # per-label HBM traffic from rocprofv3 PMC passes

A step is one pass of the headline workload over its synthetic batch: the six activations (GELU
(erf), SiLU, Sigmoid, Tanh, Hardswish, ReLU6) each forward y = f(x) and backward gi += f'(.) * g over
2^28 fp32 elements resident in HBM.  `value` is the step's algorithmic bytes (forward 8 B/element:
read x, write y; backward 16 B/element: read x or y, read g, read+write gi) over the timed wall
time.  Every kernel launch is bracketed by HIP events on the launch stream; the per-kernel medians
give `classes` (GB/s and elements/s per op class, for the broadcast / row-reduction / int8 /
full-sum workloads too unless --classes none), each with the reference engine's rate on the host
CPU beside it (`cpu`), and the `roofline` of the dominant kernel.  `gemm`: TFLOP/s against the
matrix-core peaks for the fp32 and int8 linear / batched-matmul contractions.  `engine`: the same op
classes called through the engine's nc.h API on device tensors (host wall time per call, device
synchronised), so dispatch, workspace and read-back costs show next to the kernel times.  `chain` is
the launch-bound MNIST-CNN chain (add-bias, ReLU, two sums, backward) through nc.h.  `cpu_baseline`
is the reference engine (oracle/_ref/libnc_ref.so, its own threaded AVX2 path and serial row ops) on
bounded samples of the same work.  Prints one JSON line.
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
PEAK_F32_TFLOPS = 157.3   # MI355X dense fp32 matrix
PEAK_I8_TOPS = 5000.0     # MI355X dense int8 matrix
METRIC = "achieved HBM GB/s (% of MI355X peak) per op class; elements/s vs host CPU"
ACTS = ["gelu", "silu", "sigmoid", "tanh", "hardswish", "relu6"]
N_UNARY = 1 << 28
TIMED = 10  # timed launches per op class (the median is reported)
WARM = 2  # untimed launches of each op class first
GEMM_RAMP_S = 0.25  # untimed seconds of the first contraction before the GEMM leg is timed
FLUSH_KERNEL = "k_fill16"  # the 1 GiB cache-flush fill between timed launches
CLASS_ORDER = "blocked"  # a group's timed launches class by class ("blocked") or round-robin ("interleaved")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timeline:
    """Per-launch HIP event pairs, grouped by label."""

    def __init__(self, hm):
        self.hm = hm
        self.pending = []
        self.stats = {}

    def run(self, label, nbytes, elements, fn):
        e0, e1 = self.hm.Event(), self.hm.Event()
        e0.record()
        fn()
        e1.record()
        self.pending.append((label, nbytes, elements, e0, e1))

    def collect(self):
        for label, nbytes, elements, e0, e1 in self.pending:
            e1.synchronize()
            s = self.stats.setdefault(label, {"bytes": nbytes, "elements": elements, "ms": []})
            s["ms"].append(e0.elapsed_ms(e1))
        self.pending.clear()

    def summary(self):
        out = {}
        for label, s in self.stats.items():
            ms = float(np.median(s["ms"]))
            gbs = s["bytes"] / (ms * 1e-3) / 1e9
            out[label] = {"GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4), "us": round(ms * 1e3, 1),
                          "G el/s": round(s["elements"] / (ms * 1e-3) / 1e9, 3), "bytes": s["bytes"],
                          "elements": s["elements"], "launches": len(s["ms"])}
        return out


# ------------------------------------------------------------------------------------------------
# workloads: per group, a list of (label, algorithmic bytes, elements, launcher) and the buffers
# ------------------------------------------------------------------------------------------------
def tiled(hm, K, n, seed, scale=1.0, offset=0.0):
    """A device buffer of n float32 values: a (2^20 + 7)-value random block expanded on the device
    (a strided copy with a zero stride), so large inputs cost no host memory or upload time."""
    period = (1 << 20) + 7
    blk = (np.random.default_rng(seed).standard_normal(period, dtype=np.float32) * scale + offset).astype(np.float32)
    reps = (n + period - 1) // period
    P, X = hm.DeviceBuffer.from_numpy(blk), hm.DeviceBuffer(4 * reps * period)
    K.copy_strided(4, (reps, period), P.ptr, (0, 1), X.ptr)
    hm.synchronize()
    return X


def group_unary(K, hm):
    """The headline activations over 2^28 elements, one buffer set (inputs: repeated random blocks --
    the headline step itself uses unary_workload), and a plain copy (y = -x, 8 B per element) that
    calibrates the HBM counters."""
    n = N_UNARY
    from newch_amd.hip import BWD_READS_Y
    X, G = tiled(hm, K, n, 1), tiled(hm, K, n, 2)
    Y, GI = hm.DeviceBuffer(4 * n), hm.DeviceBuffer(4 * n)
    GI.zero()
    work = []
    for act in ACTS:
        ry = act in BWD_READS_Y
        work.append((f"{act}_fwd", 8 * n, n, lambda a=act: K.unary_fwd(a, X.ptr, Y.ptr, n)))
        work.append((f"{act}_bwd", 16 * n, n, lambda a=act, ry=ry: K.unary_bwd(a, 0 if ry else X.ptr,
                                                                              Y.ptr if ry else 0, G.ptr, GI.ptr, n)))
    work.append(("copy_calibration", 8 * n, n, lambda: K.unary_fwd("neg", X.ptr, Y.ptr, n)))
    return work, [X, G, Y, GI]


def group_bcast(K, hm):
    """One 2^30-output chunk of a[256,512,1,64] op b[1,1,512,64] (a[64,512,1,64]), forward and the
    sum-to-shape backward, plus the two transposed views of a."""
    A = hm.DeviceBuffer.from_numpy(np.random.default_rng(3).standard_normal(1 << 21, dtype=np.float32))
    Bv = hm.DeviceBuffer.from_numpy((0.5 + 1.5 * np.random.default_rng(4).random(512 * 64)).astype(np.float32))
    n_out = 1 << 30
    O = hm.DeviceBuffer(4 * n_out)
    shape = (64, 512, 512, 64)
    sa, sb, so = (32768, 64, 0, 1), (0, 0, 64, 1), (1 << 24, 1 << 15, 64, 1)
    fwd_bytes = 4 * n_out + 4 * (1 << 21) + 4 * 512 * 64
    work = [(f"bcast_{op}_fwd", fwd_bytes, n_out, lambda op=op: K.binary_fwd(op, shape, A.ptr, sa, Bv.ptr, sb, O.ptr, so))
            for op in ("add", "mul", "div")]
    # transposed views of a, timed as the engine runs them: the view is re-read 512x, so it is
    # gathered to contiguous memory first, then the broadcast kernel streams the output.
    #   batch-transposed: storage [512(c),64(n),1,64] seen as [64,512,1,64] -> strides (64, 4096, 0, 1)
    #   innermost-strided: storage [64(n),64(w),512(c)] .transpose(1,2) .reshape(64,512,1,64) ->
    #   strides (32768, 1, 0, 512)
    AB, AT = hm.DeviceBuffer(4 * (1 << 21)), hm.DeviceBuffer(4 * (1 << 21))

    def batch_transposed():
        K.copy_strided(4, (64, 512, 1, 64), A.ptr, (64, 4096, 0, 1), AB.ptr)
        K.binary_fwd("add", shape, AB.ptr, sa, Bv.ptr, sb, O.ptr, so)

    def inner_strided():
        K.copy_strided(4, (64, 512, 1, 64), A.ptr, (32768, 1, 0, 512), AT.ptr)
        K.binary_fwd("add", shape, AT.ptr, sa, Bv.ptr, sb, O.ptr, so)
    work += [("bcast_add_fwd_transposed_a", fwd_bytes, n_out, batch_transposed),
             ("bcast_add_fwd_inner_strided_a", fwd_bytes, n_out, inner_strided)]
    # backward: grad_a (sum over h) and grad_b (sum over n, c) from g = O, in one pass over g
    # (g read, both grads read-modify-written, a and b read where the op needs them), or one
    # operand at a time (the path when only one operand needs a gradient)
    GA, GB = hm.DeviceBuffer(4 * (1 << 21)), hm.DeviceBuffer(4 * 512 * 64)
    GA.zero(), GB.zero()
    wsb = max(K.binary_bwd_workspace(shape, sa), K.binary_bwd_workspace(shape, sb),
              K.binary_bwd2_workspace(shape, sa, sb))
    WS = hm.DeviceBuffer(max(wsb, 1))
    for op in ("add", "mul", "div"):
        ab = 0 if op == "add" else 4 * (1 << 21) + 4 * 512 * 64
        work.append((f"bcast_{op}_bwd", 4 * n_out + 8 * (1 << 21) + 8 * 512 * 64 + ab, n_out,
                     lambda op=op: K.binary_bwd2(op, shape, O.ptr, so, A.ptr, sa, Bv.ptr, sb, GA.ptr, sa, GB.ptr,
                                                 sb, WS.ptr, wsb)))
    work += [("bcast_add_bwd_grad_a", 4 * n_out + 8 * (1 << 21), n_out,
              lambda: K.binary_bwd("add", 0, shape, O.ptr, so, A.ptr, sa, Bv.ptr, sb, GA.ptr, sa, WS.ptr, wsb)),
             ("bcast_add_bwd_grad_b", 4 * n_out + 8 * 512 * 64, n_out,
              lambda: K.binary_bwd("add", 1, shape, O.ptr, so, A.ptr, sa, Bv.ptr, sb, GB.ptr, sb, WS.ptr, wsb))]
    return work, [A, Bv, O, AB, AT, GA, GB, WS]


def group_bcast_full(K, hm):
    """The whole configuration in one call: a[256,512,1,64] + b[1,1,512,64] -> 2^32 outputs (16 GiB),
    forward and the sum-to-shape backward of both operands, which the kernel layer cuts into
    2^30-element launches."""
    A = hm.DeviceBuffer.from_numpy(np.random.default_rng(3).standard_normal(1 << 23, dtype=np.float32))
    Bv = hm.DeviceBuffer.from_numpy((0.5 + 1.5 * np.random.default_rng(4).random(512 * 64)).astype(np.float32))
    n_out = 1 << 32
    O = hm.DeviceBuffer(4 * n_out)
    shape = (256, 512, 512, 64)
    sa, sb, so = (32768, 64, 0, 1), (0, 0, 64, 1), (1 << 24, 1 << 15, 64, 1)
    fwd = lambda: K.binary_fwd("add", shape, A.ptr, sa, Bv.ptr, sb, O.ptr, so)  # noqa: E731
    GA, GB = hm.DeviceBuffer(4 * (1 << 23)), hm.DeviceBuffer(4 * 512 * 64)
    GA.zero(), GB.zero()
    wsb = K.binary_bwd2_workspace(shape, sa, sb)
    WS = hm.DeviceBuffer(max(wsb, 1))
    bwd = lambda: K.binary_bwd2("add", shape, O.ptr, so, A.ptr, sa, Bv.ptr, sb, GA.ptr, sa, GB.ptr, sb,  # noqa: E731
                                WS.ptr, wsb)
    return [("bcast_add_fwd_full", 4 * n_out + 4 * (1 << 23) + 4 * 512 * 64, n_out, fwd),
            ("bcast_add_bwd_full", 4 * n_out + 8 * (1 << 23) + 8 * 512 * 64, n_out, bwd)], [A, Bv, O, GA, GB, WS]


ROWS, COLS = 65536, 1024


def group_rows(K, hm):
    """X[65536,1024]: softmax / log_softmax and LayerNorm forward and backward, max + argmax, cross
    entropy with labels ~U[0,1024)."""
    rows, C = ROWS, COLS
    e = rows * C
    X = hm.DeviceBuffer.from_numpy(np.random.default_rng(7).standard_normal((rows, C), dtype=np.float32) * 2)
    Y, GI = hm.DeviceBuffer(4 * e), hm.DeviceBuffer(4 * e)
    G = hm.DeviceBuffer.from_numpy(np.random.default_rng(9).standard_normal((rows, C), dtype=np.float32))
    GI.zero()
    W = hm.DeviceBuffer.from_numpy((1 + 0.1 * np.random.default_rng(8).standard_normal(C)).astype(np.float32))
    Bb = hm.DeviceBuffer.from_numpy((0.1 * np.random.default_rng(8).standard_normal(C)).astype(np.float32))
    S = hm.DeviceBuffer(8 * rows)
    GW, GBb = hm.DeviceBuffer(4 * C), hm.DeviceBuffer(4 * C)
    GW.zero(), GBb.zero()
    lnws = K.layer_norm_bwd_workspace(rows, C)
    LWS = hm.DeviceBuffer(max(lnws, 1))
    M, AR = hm.DeviceBuffer(4 * rows), hm.DeviceBuffer(4 * rows)
    LAB = hm.DeviceBuffer.from_numpy(np.random.default_rng(10).integers(0, C, rows).astype(np.int32))
    LS, BADF, CS = hm.DeviceBuffer(4), hm.DeviceBuffer(8), hm.DeviceBuffer(8 * rows)
    GO = hm.DeviceBuffer.from_numpy(np.array([1.0], np.float32))
    lws = K.loss_workspace(rows, C)
    LWS2 = hm.DeviceBuffer(max(lws, 8))
    K.layer_norm_fwd(rows, C, X.ptr, W.ptr, Bb.ptr, 1e-5, Y.ptr, S.ptr)  # statistics for the backward
    work = [
        ("softmax_fwd", 8 * e, e, lambda: K.softmax_fwd(False, rows, C, X.ptr, Y.ptr)),
        ("softmax_bwd", 16 * e, e, lambda: K.softmax_bwd(False, rows, C, Y.ptr, G.ptr, GI.ptr)),
        ("log_softmax_fwd", 8 * e, e, lambda: K.softmax_fwd(True, rows, C, X.ptr, Y.ptr)),
        ("log_softmax_bwd", 16 * e, e, lambda: K.softmax_bwd(True, rows, C, Y.ptr, G.ptr, GI.ptr)),
        ("layer_norm_fwd", 8 * e + 8 * rows, e,
         lambda: K.layer_norm_fwd(rows, C, X.ptr, W.ptr, Bb.ptr, 1e-5, Y.ptr, S.ptr)),
        ("layer_norm_bwd", 16 * e + 8 * rows, e,
         lambda: K.layer_norm_bwd(rows, C, X.ptr, W.ptr, S.ptr, G.ptr, GI.ptr, GW.ptr, GBb.ptr, LWS.ptr, lnws)),
        ("max_argmax", 4 * e + 8 * rows, e, lambda: K.reduce_fwd("max", rows, C, 1, X.ptr, M.ptr, AR.ptr)),
        # forward: reads x and the labels, writes the row statistics (4 B/el + 12 B/row); backward:
        # reads x, the statistics and the labels, gi += (12 B/el + 12 B/row)
        ("cross_entropy_fwd", 4 * e + 12 * rows, e,
         lambda: K.cross_entropy_fwd(rows, C, X.ptr, LAB.ptr, CS.ptr, LS.ptr, BADF.ptr, LWS2.ptr, lws)),
        ("cross_entropy_bwd", 12 * e + 12 * rows, e,
         lambda: K.cross_entropy_bwd(rows, C, X.ptr, CS.ptr, LAB.ptr, GO.ptr, GI.ptr, accumulate=True)),
    ]
    K.cross_entropy_fwd(rows, C, X.ptr, LAB.ptr, CS.ptr, LS.ptr, BADF.ptr, LWS2.ptr, lws)  # stats for the backward
    return work, [X, Y, G, GI, W, Bb, S, GW, GBb, LWS, M, AR, LAB, LS, BADF, GO, LWS2, CS]


def w48(hm, K):
    """48 stacked W[4096,4096] ~N(0,0.02) with 0.1% of the entries x50 (seed 11)."""
    rng = np.random.default_rng(11)
    blk = rng.standard_normal((4096, 4096), dtype=np.float32) * 0.02
    idx = rng.choice(blk.size, blk.size // 1000, replace=False)
    blk.ravel()[idx] *= 50
    P = hm.DeviceBuffer.from_numpy(blk)
    Wq = hm.DeviceBuffer(48 * blk.nbytes)
    K.copy_strided(4, (48, blk.size), P.ptr, (0, 1), Wq.ptr)
    hm.synchronize()
    return Wq


def group_int8(K, hm):
    qrows, qcols = 48 * 4096, 4096
    Wq = w48(hm, K)
    Q, SC, DQ = hm.DeviceBuffer(qrows * qcols), hm.DeviceBuffer(4 * qrows), hm.DeviceBuffer(4 * qrows * qcols)
    qe = qrows * qcols
    work = [("quantize_rows", 5 * qe + 4 * qrows, qe, lambda: K.quantize_rows(qrows, qcols, Wq.ptr, Q.ptr, SC.ptr)),
            ("dequantize_rows", 5 * qe + 4 * qrows, qe, lambda: K.dequantize_rows(qrows, qcols, Q.ptr, SC.ptr, DQ.ptr))]
    return work, [Wq, Q, SC, DQ]


def group_optim(K, hm):
    """One optimizer step over 2^26 parameters: Adam reads w, g, m, v and writes w, m, v (28 B/param);
    SGD with momentum reads w, g, v and writes w, v (20 B/param); clip_grad_norm's fp64 sum of squares
    reads g (4 B/param)."""
    npar = 1 << 26
    PW = hm.DeviceBuffer.from_numpy(np.random.default_rng(12).standard_normal(npar, dtype=np.float32))
    PG = hm.DeviceBuffer.from_numpy(np.random.default_rng(13).standard_normal(npar, dtype=np.float32))
    PM, PV = hm.DeviceBuffer(4 * npar), hm.DeviceBuffer(4 * npar)
    PM.zero(), PV.zero()
    SSD = hm.DeviceBuffer(8)
    sws = K.sumsq_workspace(npar)
    SWS = hm.DeviceBuffer(max(sws, 8))
    work = [
        ("adam_step", 28 * npar, npar,
         lambda: K.optim_step("adam", npar, PW.ptr, PG.ptr, PM.ptr, PV.ptr, 1e-3, 0.0, 0.0, 0.9, 0.999, 1e-8, 1.0,
                              0.1, 0.001)),
        ("sgd_momentum_step", 20 * npar, npar,
         lambda: K.optim_step("sgd", npar, PW.ptr, PG.ptr, PM.ptr, None, 1e-3, 0.9, 0.0)),
        ("grad_sumsq", 4 * npar, npar, lambda: K.sumsq(npar, PG.ptr, SSD.ptr, False, SWS.ptr, sws)),
    ]
    return work, [PW, PG, PM, PV, SSD, SWS]


def group_sums(K, hm):
    """Full sum and mean over 2^30 fp32 elements (~N(0,1), seed 12, a 2^20 + 7-value block repeated)."""
    n = 1 << 30
    X = tiled(hm, K, n, 12)
    fws = K.reduce_workspace("sum", 1, n, 1)
    FWS, FS = hm.DeviceBuffer(max(fws, 1)), hm.DeviceBuffer(4)
    work = [("full_sum", 4 * n, n, lambda: K.reduce_fwd("sum", 1, n, 1, X.ptr, FS.ptr, 0, FWS.ptr, fws)),
            ("full_mean", 4 * n, n, lambda: K.reduce_fwd("mean", 1, n, 1, X.ptr, FS.ptr, 0, FWS.ptr, fws))]
    return work, [X, FWS, FS]


def group_gemm(K, hm):
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


GROUPS = {
    "unary": ([f"{a}_{d}" for a in ACTS for d in ("fwd", "bwd")] + ["copy_calibration"], group_unary),
    "bcast": (["bcast_add_fwd", "bcast_mul_fwd", "bcast_div_fwd", "bcast_add_fwd_transposed_a",
               "bcast_add_fwd_inner_strided_a", "bcast_add_bwd", "bcast_mul_bwd", "bcast_div_bwd",
               "bcast_add_bwd_grad_a", "bcast_add_bwd_grad_b"], group_bcast),
    "bcast_full": (["bcast_add_fwd_full", "bcast_add_bwd_full"], group_bcast_full),
    "rows": (["softmax_fwd", "softmax_bwd", "log_softmax_fwd", "log_softmax_bwd", "layer_norm_fwd",
              "layer_norm_bwd", "max_argmax", "cross_entropy_fwd", "cross_entropy_bwd"], group_rows),
    "int8": (["quantize_rows", "dequantize_rows"], group_int8),
    "optim": (["adam_step", "sgd_momentum_step", "grad_sumsq"], group_optim),
    "sums": (["full_sum", "full_mean"], group_sums),
}
GEMM_LABELS = ["linear_fwd_sgemm_nt", "linear_bwd_dx_sgemm_nn", "linear_bwd_dw_sgemm_tn", "bmm_qk_t_sgemm",
               "gemm_s8_nt", "linear_int8"]


def run_group(K, hm, builder, labels=None, setup_only=False):
    """WARM untimed launches of each op class, then TIMED launches each after a 1 GiB fill that evicts
    the 256 MB MALL (outside the launch's events): a cold-cache median per class.  The timed launches
    run class by class, so a class's time does not depend on which classes share its group or their
    order: round-robin over the classes, a short kernel ran slower after some neighbours than after
    others despite the fill (the cross-entropy forward 45.7 us after itself, 47.3-49.0 after the
    LayerNorm backward or the whole group; --class-order interleaved keeps that order for comparison).
    setup_only: build the group's inputs and stop (the profiler pass whose counters are subtracted
    from the labels')."""
    work, keep = builder(K, hm)
    if setup_only:
        hm.synchronize()
        return {}
    if labels is not None:
        work = [w for w in work if w[0] in labels]
    for _ in range(WARM):
        for w in work:
            w[3]()
    hm.synchronize()
    flush = hm.DeviceBuffer(1 << 30)
    tl = Timeline(hm)
    if CLASS_ORDER == "interleaved":
        for _ in range(TIMED):
            for label, nbytes, elements, fn in work:
                K.fill(flush.ptr, 4, 0, 1 << 28)
                tl.run(label, nbytes, elements, fn)
    else:
        for label, nbytes, elements, fn in work:
            for _ in range(TIMED):
                K.fill(flush.ptr, 4, 0, 1 << 28)
                tl.run(label, nbytes, elements, fn)
    hm.synchronize()
    tl.collect()
    del keep, flush
    return tl.summary()


def run_gemm(K, hm, labels=None):
    """Each contraction as its own block of launches (WARM untimed, then TIMED timed, back to back), so
    a kernel runs at the clocks its own power draw settles at: launches interleaved across the labels
    timed the int8 GEMM right after the fp32 GEMMs, whose power state the chip's clock management
    carries into it (136 against 124 us on one box, the fp32 GEMMs within 2% either way)."""
    work, keep = group_gemm(K, hm)
    if labels is not None:
        work = [w for w in work if w[0] in labels]
    # the matrix-core clocks ramp for ~20 ms after the bandwidth-bound classes (the first fp32 GEMM
    # launches ran 2350 -> 2080 us): the first contraction runs a quarter second untimed first
    t0 = time.perf_counter()
    while work and time.perf_counter() - t0 < GEMM_RAMP_S:
        work[0][3]()
        hm.synchronize()
    tl = Timeline(hm)
    for label, ops, peak, fn in work:
        for _ in range(WARM):
            fn()
        hm.synchronize()
        for _ in range(TIMED):
            tl.run(label, ops, 0, fn)
        hm.synchronize()
    tl.collect()
    out = {}
    for label, ops, peak, fn in work:
        ms = float(np.median(tl.stats[label]["ms"]))
        rate = ops / (ms * 1e-3) / 1e12
        out[label] = {"TFLOP/s" if peak == PEAK_F32_TFLOPS else "TOP/s": round(rate, 1), "peak": peak,
                      "frac": round(rate / peak, 4), "us": round(ms * 1e3, 1), "ops": ops,
                      "launches": len(tl.stats[label]["ms"])}
        log(f"bench: {label:28s} {rate:8.1f} T/s  {100 * rate / peak:5.1f}% of {peak}  {ms * 1e3:9.1f} us")
    del keep
    return out


def unary_workload(K, hm, n):
    """The headline step's buffers: two sets alternated between activations, so no kernel finds its
    inputs in the 256 MB MALL from the previous one (each set is 4 GiB; consecutive uses of a set are
    >= 3 GiB apart)."""
    from newch_amd.hip import BWD_READS_Y
    sets = []
    x = np.random.default_rng(1).standard_normal(n, dtype=np.float32)
    g = np.random.default_rng(2).standard_normal(n, dtype=np.float32)
    for _ in range(2):
        X, G = hm.DeviceBuffer.from_numpy(x), hm.DeviceBuffer.from_numpy(g)
        Y, GI = hm.DeviceBuffer(4 * n), hm.DeviceBuffer(4 * n)
        GI.zero()
        sets.append((X, G, Y, GI))

    def step(tl):
        for i, act in enumerate(ACTS):
            X, G, Y, GI = sets[i % 2]
            tl.run(f"{act}_fwd", 8 * n, n, lambda a=act, X=X, Y=Y: K.unary_fwd(a, X.ptr, Y.ptr, n))
            ry = act in BWD_READS_Y
            tl.run(f"{act}_bwd", 16 * n, n,
                   lambda a=act, ry=ry, X=X, Y=Y, G=G, GI=GI:
                   K.unary_bwd(a, 0 if ry else X.ptr, Y.ptr if ry else 0, G.ptr, GI.ptr, n, accumulate=True))

    return step, 24 * n * len(ACTS), sets


# ------------------------------------------------------------------------------------------------
# HBM traffic from rocprofv3 PMC passes, one pass per label and counter
# ------------------------------------------------------------------------------------------------
TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_classes.txt"


def _pmc_rows(db_dir: Path, counter: str):
    """(kernel name, value) per dispatch from the rocpd databases under db_dir."""
    import sqlite3
    rows = []
    for db in sorted(db_dir.rglob("*_results.db")):
        con = sqlite3.connect(str(db))
        try:
            rows += con.execute("select kernel_name, value from counters_collection where counter_name like ?",
                                (counter + "%",)).fetchall()
        finally:
            con.close()
    return rows


def _pmc_counts(d: Path):
    """{kernel: [dispatches, FETCH_SIZE sum, WRITE_SIZE sum]} of one pass pair d/{fetch,write}, without
    the cache-flush fills and the runtime's own copy and fill kernels."""
    out = {}
    for k_, (sub, counter) in enumerate((("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE"))):
        for k, v in _pmc_rows(d / sub, counter):
            if FLUSH_KERNEL in k or k.startswith("__amd_rocclr"):
                continue
            e = out.setdefault(k.split("(")[0], [0, 0.0, 0.0])
            if k_ == 0:
                e[0] += 1
            e[1 + k_] += v
    return out


def traffic_summary(root: Path) -> str:
    """root/<label>/{fetch,write}/: a `--only <label>` run under rocprofv3 --pmc FETCH_SIZE (WRITE_SIZE);
    root/_setup_<group>/{fetch,write}/: the same group built with --setup-only.  A label's traffic is
    its run's dispatches minus its group's setup dispatches, divided by its launches (WARM untimed +
    TIMED timed): KiB per launch, with the copy calibration's factors."""
    owner = {lab: g for g, (labels, _) in GROUPS.items() for lab in labels}
    owner.update({lab: "gemm" for lab in GEMM_LABELS})
    setup = {d.name[len("_setup_"):]: _pmc_counts(d) for d in root.iterdir() if d.name.startswith("_setup_")}
    per = {}
    for d in sorted(p for p in root.iterdir() if p.is_dir() and not p.name.startswith("_")):
        run = _pmc_counts(d)
        base = setup.get(owner.get(d.name, ""), {})
        f = w = 0.0
        kernels = []
        for k, (n, fv, wv) in run.items():
            bn, bf, bw = base.get(k, (0, 0.0, 0.0))
            if n > bn:
                kernels.append(k.replace("void ", "").replace("nchip::", ""))
            f += fv - bf
            w += wv - bw
        per[d.name] = (f / (WARM + TIMED), w / (WARM + TIMED), sorted(kernels))
    lines = []
    cal = per.get("copy_calibration")
    if cal and cal[0] and cal[1]:
        kib = 4 * N_UNARY / 1024  # the copy reads and writes 2^28 floats
        lines += [f"fetch_scale {cal[0] / kib:.4f}", f"write_scale {cal[1] / kib:.4f}"]
    lines.append(f"{'label':32s} {'launches':>8s} {'FETCH_KiB':>14s} {'WRITE_KiB':>14s}  kernels")
    for label, (f, w, ks) in per.items():
        lines.append(f"{label:32s} {WARM + TIMED:8d} {f:14.1f} {w:14.1f}  {', '.join(ks)}")
    return "\n".join(lines) + "\n"


def measured_traffic(label: str):
    """HBM bytes per launch of `label` from the committed per-label PMC summary (FETCH_SIZE and
    WRITE_SIZE in KiB per launch, scaled by what the same counters read for a plain copy)."""
    if not TRAFFIC_FILE.exists():
        return None
    scale, rows = {}, {}
    for line in TRAFFIC_FILE.read_text().splitlines():
        parts = line.split()
        if len(parts) == 2 and parts[0] in ("fetch_scale", "write_scale"):
            scale[parts[0]] = float(parts[1])
        elif len(parts) >= 4 and not line.startswith("#") and parts[1].isdigit():
            rows[parts[0]] = (float(parts[2]), float(parts[3]))
    if label not in rows or len(scale) != 2:
        return None
    f, w = rows[label]
    return int(round((f / scale["fetch_scale"] + w / scale["write_scale"]) * 1024))


# ------------------------------------------------------------------------------------------------
# the engine's nc.h API on device tensors
# ------------------------------------------------------------------------------------------------
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


def engine_leg(K, hm, classes):
    """Op classes called through nc.h on device tensors, as the reference's Python layer calls them:
    host wall time per call with the device synchronised, after WARM warm calls (the arena then reuses
    its blocks).  `kernel_us` is the same class's kernel time from `classes`."""
    import ctypes
    from ctypes import c_float, c_void_p

    from newch_amd import abi

    L = abi.load()
    ctx = L.nc_init(ctypes.byref(abi.Config(0, 0, 0, 0)))

    def check():
        if not L.nc_ok(ctx):
            raise RuntimeError(L.nc_error(ctx).decode())

    def persistent_from(buf, dt, shape):
        nd, shp = abi.shape_arg(shape)
        L.nc_persistent_begin(ctx)
        t = L.nc_from_device(ctx, dt, c_void_p(buf.ptr), nd, shp)
        L.nc_persistent_end(ctx)
        L.nc_synchronize(ctx)  # the copy has finished before the caller may free buf
        check()
        return t

    rows, C = ROWS, COLS
    Xb = hm.DeviceBuffer.from_numpy(np.random.default_rng(7).standard_normal((rows, C), dtype=np.float32) * 2)
    X = persistent_from(Xb, abi.F32, (rows, C))
    Wt = persistent_from(hm.DeviceBuffer.from_numpy((1 + 0.1 * np.random.default_rng(8).standard_normal(C))
                                                    .astype(np.float32)), abi.F32, (C,))
    Bt = persistent_from(hm.DeviceBuffer.from_numpy((0.1 * np.random.default_rng(8).standard_normal(C))
                                                    .astype(np.float32)), abi.F32, (C,))
    LAB = persistent_from(hm.DeviceBuffer.from_numpy(np.random.default_rng(10).integers(0, C, rows).astype(np.int32)),
                          abi.I32, (rows,))
    Wb = w48(hm, K)
    W48 = persistent_from(Wb, abi.F32, (48 * 4096, 4096))
    del Wb
    Ab = hm.DeviceBuffer.from_numpy(np.random.default_rng(3).standard_normal(1 << 23, dtype=np.float32))
    A = persistent_from(Ab, abi.F32, (256, 512, 1, 64))
    Bv = persistent_from(hm.DeviceBuffer.from_numpy((0.5 + 1.5 * np.random.default_rng(4).random(512 * 64))
                                                    .astype(np.float32)), abi.F32, (1, 1, 512, 64))
    del Ab
    # the linear forward of the GEMM leg's shape, bias included: x[8192,4096] W[4096,4096]^T + b
    XLb = tiled(hm, K, 8192 * 4096, 11)
    XL = persistent_from(XLb, abi.F32, (8192, 4096))
    del XLb
    WLb = tiled(hm, K, 4096 * 4096, 12, scale=0.02)
    WL = persistent_from(WLb, abi.F32, (4096, 4096))
    del WLb
    BL = persistent_from(hm.DeviceBuffer.from_numpy(np.random.default_rng(13).standard_normal(4096, dtype=np.float32)),
                         abi.F32, (4096,))
    L.nc_persistent_begin(ctx)
    Xp = L.nc_parameter(ctx, X, *abi.shape_arg((rows, C)))
    Ap = L.nc_parameter(ctx, A, *abi.shape_arg((256, 512, 1, 64)))
    Bp = L.nc_parameter(ctx, Bv, *abi.shape_arg((1, 1, 512, 64)))
    L.nc_persistent_end(ctx)
    check()
    sc = c_void_p()
    # Adam over 32 parameters of 65536 floats (gradients from one backward of the sum of their sums):
    # the engine updates them in one multi-parameter launch
    nps, pn = 32, 65536
    Pb = hm.DeviceBuffer.from_numpy(np.random.default_rng(13).standard_normal(pn, dtype=np.float32))
    pt = persistent_from(Pb, abi.F32, (pn,))
    L.nc_persistent_begin(ctx)
    params = [L.nc_parameter(ctx, pt, *abi.shape_arg((pn,))) for _ in range(nps)]
    L.nc_persistent_end(ctx)
    loss = None
    for q in params:
        t = L.nc_sum(q, 0, 0)
        loss = t if loss is None else L.nc_add(loss, t)
    L.nc_backward(loss)
    check()
    L.nc_step_end(ctx)
    plist = (c_void_p * nps)(*params)
    opt = L.nc_adam(ctx, plist, nps, abi.OptimOpts(1e-3, 0, 0, 0.9, 0.999, 1e-8))
    check()
    calls = [
        ("softmax_fwd", lambda: L.nc_softmax(X)),
        ("layer_norm_fwd", lambda: L.nc_layer_norm(X, 1, Wt, Bt, c_float(1e-5))),
        ("quantize_rows", lambda: L.nc_quantize_rows(W48, ctypes.byref(sc))),
        ("cross_entropy_fwd", lambda: L.nc_cross_entropy(X, LAB)),
        ("cross_entropy_fwd_bwd", lambda: L.nc_backward(L.nc_cross_entropy(Xp, LAB))),
        ("bcast_add_fwd_full", lambda: L.nc_add(A, Bv)),
        # the configuration's full shape through autograd: forward, full sum, its 2^32-element
        # gradient and the fused sum-to-shape backward of both operands
        ("bcast_add_fwd_sum_bwd_full", lambda: L.nc_backward(L.nc_sum(L.nc_add(Ap, Bp), abi.ALL_AXES, 0))),
        ("adam_step_32_params", lambda: L.nc_optim_step(opt)),
        # the 32 gradients' norm (one sum launch, one read-back) and their rescale (one launch)
        ("clip_grad_norm_32_params", lambda: L.nc_clip_grad_norm(plist, nps, c_float(1.0))),
        # the GEMM with the bias added in its epilogue
        ("linear_fwd_bias", lambda: L.nc_linear_fn(XL, WL, BL)),
    ]
    out = {}
    for label, fn in calls:
        ts = []
        for r in range(WARM + TIMED):
            L.nc_synchronize(ctx)
            t0 = time.perf_counter()
            fn()
            L.nc_synchronize(ctx)
            ts.append(time.perf_counter() - t0)
            check()
            for q in (Xp, Ap, Bp):
                L.nc_zero_grad(q)
            L.nc_step_end(ctx)
        us = float(np.median(ts[WARM:])) * 1e6
        k = classes.get(label if label != "cross_entropy_fwd_bwd" else "cross_entropy_fwd")
        entry = {"us": round(us, 1)}
        if k:
            kus = k["us"] + (classes["cross_entropy_bwd"]["us"] if label == "cross_entropy_fwd_bwd"
                             and "cross_entropy_bwd" in classes else 0.0)
            entry.update({"kernel_us": round(kus, 1), "GB/s": round(k["bytes"] / (us * 1e-6) / 1e9, 1)
                          if label != "cross_entropy_fwd_bwd" else None})
        out[label] = entry
        log(f"bench: engine {label:24s} {us:9.1f} us" + (f" (kernels {entry['kernel_us']} us)" if k else ""))
    L.nc_free_ctx(ctx)
    return out


# ------------------------------------------------------------------------------------------------
# CPU baseline: the reference engine per op class
# ------------------------------------------------------------------------------------------------
def cpu_baseline(classes):
    """The reference engine (oracle/_ref/libnc_ref.so) timed per op class on the host cores
    (oracle/refbench.py): each class gets a `cpu` entry; the headline value is the reference's rate
    over the headline workload's own work (each activation's forward and gi += f'(x) g backward)."""
    from oracle import pyoracle, refbench

    if not pyoracle.REF_LIB.exists():
        return None
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or min(os.cpu_count() or 1, 64)
    threads = min(threads, 64, os.cpu_count() or 1)
    ref = refbench.reference_classes(threads)
    meta = ref.pop("_meta")
    for label, (s, n, what) in ref.items():
        g = classes.get(label)
        if not g:
            continue
        per_el = g["bytes"] / g["elements"]
        gbs = per_el * n / s / 1e9
        g["cpu"] = {"GB/s": round(gbs, 2), "G el/s": round(n / s / 1e9, 4), "us": round(s * 1e6, 1),
                    "sample": what, "gpu_x": round(g["GB/s"] / gbs, 1)}
    n_cpu = ref["gelu_fwd"][1]
    t = sum(ref[f"{a}_{d}"][0] for a in ACTS for d in ("fwd", "bwd"))
    chain_us = chain_latency(pyoracle.REF_LIB, iters=50, warmup=3, threads=threads)
    return {"value": round(24 * n_cpu * len(ACTS) / t / 1e9, 2), "unit": "GB/s",
            "elements_per_s": round(n_cpu * len(ACTS) / t / 1e9, 3), "elements_unit": "G el/s (fwd+bwd pairs)",
            "cores": meta["threads"], "kind": "reference",
            "sample": f"2^{n_cpu.bit_length() - 1} fp32 elements per activation (256 MiB tensors, past the host "
                      f"caches): each of {', '.join(ACTS)} forward y = f(x) and backward gi += f'(.) g, timed on the "
                      f"reference's own code (engine/src/ops/ops_elementwise.c:229-365, {meta['backend']} tier, its "
                      f"thread pool) on {meta['threads']} threads of {meta['nproc']} ({meta['cpu']}); the same 24 "
                      f"B/element as the GPU value; every op class's own rate is in classes[*].cpu "
                      f"({meta['seconds']} s in all)",
            "chain_us": chain_us,
            "chain_sample": "the MNIST-CNN chain (as `chain`), 50 iterations on the reference engine"}


def only_mode(K, hm, labels, setup_only=False):
    """Just the named op classes (WARM untimed + TIMED timed launches each): the per-label profiler passes."""
    classes = {}
    for gname, (glabels, builder) in GROUPS.items():
        want = [x for x in glabels if x in labels]
        if want:
            classes.update(run_group(K, hm, builder, set(want), setup_only))
    if setup_only:
        if any(x in GEMM_LABELS for x in labels):
            _, keep = group_gemm(K, hm)
            hm.synchronize()
            del keep
        print(json.dumps({"setup_only": sorted(labels)}), flush=True)
        return
    gemm = run_gemm(K, hm, set(labels)) if any(x in GEMM_LABELS for x in labels) else {}
    unknown = sorted(set(labels) - set(classes) - set(gemm))
    if unknown:
        sys.exit(f"bench.py --only: unknown labels {unknown}")
    print(json.dumps({"only": sorted(labels), "classes": classes, "gemm": gemm}), flush=True)


def main():
    global CLASS_ORDER
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--classes", choices=["all", "none"], default="all")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--class-order", choices=["interleaved", "blocked"], default=CLASS_ORDER,
                    help="a group's timed launches round-robin over its classes, or class by class")
    ap.add_argument("--only", default=None, help="comma-separated op-class labels: run just those")
    ap.add_argument("--setup-only", action="store_true", help="with --only: build the inputs, launch nothing")
    ap.add_argument("--traffic-summary", default=None, help="print the per-label HBM traffic table of the "
                    "PMC passes under this directory (no GPU work)")
    args = ap.parse_args()
    CLASS_ORDER = args.class_order
    if args.traffic_summary:
        sys.stdout.write(traffic_summary(Path(args.traffic_summary)))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one MI355X: the kernels run on one GPU's share "
                                   "and multi-GPU sharding is not implemented"}))
        sys.exit(2)

    from newch_amd import hipmem as hm
    from newch_amd.hip import Kernels

    if hm.device_count() < 1:
        sys.exit("bench.py: no HIP device visible")
    K = Kernels()
    if args.only:
        only_mode(K, hm, set(args.only.split(",")), args.setup_only)
        return
    n = N_UNARY
    log(f"bench: unary workload, {n} elements x {len(ACTS)} activations, warmup {args.warmup}, steps {args.steps}")
    step, step_bytes, sets = unary_workload(K, hm, n)
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
    del sets
    value = step_bytes * args.steps / wall / 1e9
    dom = max(classes, key=lambda k: classes[k]["us"])
    d = classes[dom]
    log(f"bench: unary step {wall / args.steps * 1e3:.3f} ms, {value:.1f} GB/s; dominant {dom} {d['GB/s']} GB/s")

    gemm, engine = {}, {}
    if args.classes == "all":
        for gname, (glabels, builder) in GROUPS.items():
            if gname == "unary":
                continue
            extra = run_group(K, hm, builder)
            for k, v in extra.items():
                log(f"bench: {k:30s} {v['GB/s']:8.1f} GB/s  {100 * v['frac']:5.1f}%  {v['us']:9.1f} us  "
                    f"{v['G el/s']:8.2f} G el/s")
            classes.update(extra)
        gemm = run_gemm(K, hm)
        engine = engine_leg(K, hm, classes)

    chain_us = chain_latency()
    log(f"bench: MNIST-CNN chain fwd+bwd through the engine {chain_us} us per iteration")
    cpu = None if args.no_cpu else cpu_baseline(classes)
    if cpu:
        log(f"bench: cpu baseline {cpu['value']} GB/s ({cpu['elements_per_s']} G el/s) on {cpu['cores']} threads")
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
        "engine": engine,
        "chain": {"workload": "MNIST-CNN chain through nc.h: relu(x[64,16,28,28] + bias[1,16,1,1]), sum over "
                              "dims 3 then 2, sum().backward(), zero_grad, step_end (802,816 elements; "
                              "launch-bound)", "us_per_iter": chain_us},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
