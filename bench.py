#!/usr/bin/env python3
"""Benchmark of the tinytorch hot path on one MI355X.

Headline (BASELINE.json metric): fp32 GEMM TFLOP/s at 4096^3 as a fraction
of the fp32 MFMA peak, plus the CNN forward+backward step time.

  * A "step" of the headline is one C = A*B at M = N = K = 4096, fp32 in,
    fp32 MFMA accumulate, fp32 out, operands uniform[-1,1] from fixed seeds
    and resident in HBM before timing.  W untimed steps, then exactly K
    steps between two stream synchronisations; `value` = 2*4096^3*K / time.
  * roofline.achieved uses HIP events recorded on the library's stream (the
    stream the GEMM kernel runs on) around the K launches.
  * extra.cnn_step: config 4 (B=128, 3x32x32, conv32 -> relu -> pool ->
    conv64 -> relu -> pool -> FC 4096->10, softmax-CE) forward + full
    backward + an SGD update of every weight, inputs and weights resident,
    graph rebuilt every step through the C ABI (ctypes): ms per step over K
    back-to-back steps, the reference protocol's median (5 warmup, median of
    20 synced steps), TFLOP/s on the step's 4.11 GFLOP against the fp32 MFMA
    peak, and the reference CPU step beside it.  extra.mlp_step: the same
    for config 2.
  * extra.*: the other BASELINE configs (1024^3, 4096^3 NT/TN backward GEMMs,
    8192^3, ragged, tall-skinny, MLP step); extra.conv_kernels: the direct
    convolution kernels of the CNN step alone (TFLOP/s vs the MFMA peak);
    extra.hbm_kernels: the bandwidth kernels (im2col/col2im serve only the
    convolutions whose input slab does not fit LDS; the step runs the pool
    and relu backwards as the one maxpool_relu_bwd pass).
  * cpu_baseline: the reference's own AVX2+FMA OpenMP sgemm, compiled from
    its sources into oracle/_ref (or the oracle restatement when that build
    is missing), on this host's cores, on a bounded sample (median of 9 runs
    of the same 4096^3 workload after 2 warmups); beside it the reference
    CNN and MLP steps (5 warmup + median of 20) and one 4096^3 matmul
    backward on the reference autograd (config 3).

One JSON line on stdout.  --gpus N > 1 exits: this build targets one GPU.
"""
import argparse
import ctypes
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3   # MI355X dense fp32 matrix peak
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="headline only")
    ap.add_argument("--cnn-only", action="store_true",
                    help="only time the config-4 CNN training step (for kernel traces of it)")
    ap.add_argument("--mlp-only", action="store_true",
                    help="only time the config-2 MLP training step (for kernel traces of it)")
    ap.add_argument("--gemm-shapes", action="store_true",
                    help="only time the secondary GEMM shapes (configs 1, 3, 5; for kernel "
                         "traces of them)")
    ap.add_argument("--gemm-shape", choices=None, default=None,
                    help="only time one secondary GEMM shape, by its extra.* name")
    ap.add_argument("--conv-kernels", action="store_true",
                    help="only time the convolution kernels alone (extra.conv_kernels; for kernel "
                         "traces of them)")
    ap.add_argument("--hbm-kernels", action="store_true",
                    help="only time the bandwidth kernels alone (extra.hbm_kernels; for kernel "
                         "traces and HBM counters of them)")
    ap.add_argument("--phases", action="store_true",
                    help="per-phase kernel timestamps of the CNN step's kernels and the 64x64 "
                         "GEMM (needs `make probe`: build/probe/libtinytorch.so)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="only run a plain 1 GiB device copy kernel 5 times (the known-size "
                         "reference for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


# ---- seeded synthetic inputs; numpy only ----

def uniform(shape, lo, hi, seed):
    return np.random.default_rng(seed).uniform(lo, hi, shape).astype(np.float32)


def he_normal(shape, fan_in, seed):
    return (np.random.default_rng(seed).standard_normal(shape) *
            np.sqrt(2.0 / fan_in)).astype(np.float32)


def cnn_inputs(B=128, seed=0x5EED):
    """config 4: x U[0,1] Bx3x32x32, labels U{0..9}, He-normal conv/FC, zero biases"""
    x = uniform((B, 3, 32, 32), 0.0, 1.0, seed + 1)
    y = np.random.default_rng(seed + 2).integers(0, 10, B).astype(np.int32)
    wfc = he_normal((4097, 10), 4096, seed + 12)
    wfc[4096] = 0.0
    P = dict(w1=he_normal((32, 3, 3, 3), 27, seed + 10), b1=np.zeros(32, np.float32),
             w2=he_normal((64, 32, 3, 3), 288, seed + 11), b2=np.zeros(64, np.float32), wfc=wfc)
    return x, y, P


def mlp_inputs(B=256, seed=0x5EED):
    """config 2: x U[0,1] Bx784, labels U{0..9}, He-normal weights, zero bias rows"""
    x = uniform((B, 784), 0.0, 1.0, seed + 1)
    y = np.random.default_rng(seed + 2).integers(0, 10, B).astype(np.int32)
    Ws = []
    for i, (fi, fo) in enumerate(((784, 512), (512, 256), (256, 10))):
        w = he_normal((fi + 1, fo), fi, seed + 10 + i)
        w[fi] = 0.0
        Ws.append(w)
    return x, y, Ws


def read_traffic():
    """HBM bytes per launch of the 4096^3 GEMM from the committed rocprofv3
    PMC summary (FETCH_SIZE + WRITE_SIZE, copy-kernel calibrated)."""
    p = os.path.join(ROOT, "profiles", "sgemm_nn_4096_pmc.md")
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.strip().startswith("traffic_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


class Gemm:
    def __init__(self, L, M, N, K, ta=0, tb=0, seed=0x5EED):
        from tinytorch_amd.hip import DevBuf
        self.L, self.M, self.N, self.K, self.ta, self.tb = L, M, N, K, ta, tb
        A = uniform((K, M) if ta else (M, K), -1, 1, seed + 1)
        B = uniform((N, K) if tb else (K, N), -1, 1, seed + 2)
        self.dA, self.dB, self.dC = DevBuf.from_np(A), DevBuf.from_np(B), DevBuf(M * N)
        self.lda = M if ta else K
        self.ldb = K if tb else N

    def launch(self):
        rc = self.L.tt_k_gemm(self.M, self.N, self.K, self.dA.ptr, self.lda, self.ta,
                              self.dB.ptr, self.ldb, self.tb, self.dC.ptr, self.N)
        if rc != 0:
            raise RuntimeError(f"tt_k_gemm failed: {rc}")

    def flops(self):
        return 2.0 * self.M * self.N * self.K

    def free(self):
        for b in (self.dA, self.dB, self.dC):
            b.free()


def prewarm(fn, seconds=0.3):
    """Untimed device warm-up: the GPU leaves its idle clocks only after some
    milliseconds of sustained work (first launches after idle run ~40% slower)."""
    from tinytorch_amd.hip import sync
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(4):
            fn()
        sync()


def time_gemm(L, g, steps, warmup):
    from tinytorch_amd.hip import StreamTimer, sync
    prewarm(g.launch)
    for _ in range(warmup):
        g.launch()
    sync()
    tm = StreamTimer()
    t0 = time.perf_counter()
    tm.start()
    for _ in range(steps):
        g.launch()
    ev_ms = tm.stop_ms()
    sync()
    wall_ms = (time.perf_counter() - t0) * 1e3
    return wall_ms / steps, ev_ms / steps


class CnnStep:
    """Config 4 training step on device-resident tensors through the C ABI."""

    def __init__(self, L, B=128):
        self.L = L
        x, y, P = cnn_inputs(B=B)
        self.B = B
        self.labels = np.ascontiguousarray(y, dtype=np.int32)
        self.lab_p = self.labels.ctypes.data_as(ctypes.POINTER(ctypes.c_int))
        self.t = {k: self._tensor(v) for k, v in dict(x=x, **P).items()}
        self.flat = (ctypes.c_long * 2)(B, P["wfc"].shape[0] - 1)

    def _tensor(self, a):
        from tinytorch_amd import F32P
        a = np.ascontiguousarray(a, np.float32)
        shp = (ctypes.c_long * a.ndim)(*a.shape)
        t = self.L.tt_fromdata(a.ctypes.data_as(F32P), shp, a.ndim)
        assert t
        return t

    def step(self, lr=0.0, probe=None):
        """One step; `probe(L, loss)` (tests only) runs after the SGD update,
        before the graph is released."""
        L, t = self.L, self.t
        nodes = []

        def k(n):
            assert n, "op returned NULL"
            nodes.append(n)
            return n
        X = k(L.ag_leaf(t["x"], 0))
        w1, b1, w2, b2, wfc = (k(L.ag_leaf(t[n], 1)) for n in ("w1", "b1", "w2", "b2", "wfc"))
        h = k(L.ag_conv2d(X, w1, b1, 1, 1, 1, 1))
        h = k(L.ag_maxpool2d(k(L.ag_relu(h)), 2, 2, 2, 2))
        h = k(L.ag_conv2d(h, w2, b2, 1, 1, 1, 1))
        h = k(L.ag_maxpool2d(k(L.ag_relu(h)), 2, 2, 2, 2))
        h = k(L.ag_padones(k(L.ag_reshape(h, self.flat, 2))))
        logits = k(L.ag_matmul(h, wfc))
        loss = k(L.ag_softmax_ce(logits, self.lab_p, self.B))
        L.ag_backward(loss)
        ws = (ctypes.c_void_p * 5)(w1, b1, w2, b2, wfc)
        assert L.ag_sgd_step_many(ws, 5, ctypes.c_float(lr)) == 0
        if probe is not None:
            probe(L, loss)
        for n in nodes:
            L.ag_release(n)


class MlpStep:
    """Config 2 training step (784->512->256->10, B=256) through the C ABI."""

    def __init__(self, L, B=256):
        self.L = L
        x, y, Ws = mlp_inputs(B=B)
        self.B = B
        self.labels = np.ascontiguousarray(y, dtype=np.int32)
        self.lab_p = self.labels.ctypes.data_as(ctypes.POINTER(ctypes.c_int))
        from tinytorch_amd import F32P
        self.t = []
        for a in [x] + Ws:
            shp = (ctypes.c_long * 2)(*a.shape)
            self.t.append(L.tt_fromdata(np.ascontiguousarray(a).ctypes.data_as(F32P), shp, 2))

    def step(self, lr=0.0, probe=None):
        """One step; `probe(L, loss)` as in CnnStep.step."""
        L = self.L
        nodes = []

        def k(n):
            assert n
            nodes.append(n)
            return n
        X = k(L.ag_leaf(self.t[0], 0))
        W = [k(L.ag_leaf(t, 1)) for t in self.t[1:]]
        h = k(L.ag_relu(k(L.ag_matmul(k(L.ag_padones(X)), W[0]))))
        h = k(L.ag_relu(k(L.ag_matmul(k(L.ag_padones(h)), W[1]))))
        logits = k(L.ag_matmul(k(L.ag_padones(h)), W[2]))
        loss = k(L.ag_softmax_ce(logits, self.lab_p, self.B))
        L.ag_backward(loss)
        ws = (ctypes.c_void_p * 3)(*W)
        assert L.ag_sgd_step_many(ws, 3, ctypes.c_float(lr)) == 0
        if probe is not None:
            probe(L, loss)
        for n in nodes:
            L.ag_release(n)


# Algorithmic work of one training step (SURVEY 8(d) counts): the CNN's
# convolution and classifier GEMMs forward + backward (conv1 dX is not part
# of the step: its input is the image), and the MLP's minimal 617 MFLOP
# (2*256*(785*512 + 513*256 + 257*10) forward, twice that backward without
# the first layer's input gradient).
CNN_STEP_GFLOP = 4.11
MLP_STEP_GFLOP = 0.617


def step_figures(stepper, gflop, steps):
    """ms: K back-to-back steps between two syncs (throughput); median_ms:
    the reference protocol, 5 warmup steps then the median of 20 steps each
    bracketed by a sync (bench/bench_cpu.py:74-82)."""
    from tinytorch_amd.hip import sync
    ms = time_steps(stepper, steps, 5)

    def one():
        stepper.step()
        sync()
    med_ms = median_time(one, 5, 20) * 1e3
    tf = gflop / (ms * 1e-3) / 1e3
    return dict(ms=round(ms, 4), median_ms=round(med_ms, 4), gflop=gflop, tflops=round(tf, 2),
                frac_of_fp32_mfma_peak=round(tf / PEAK_FP32_MFMA_TFLOPS, 4))


def time_steps(stepper, steps, warmup):
    from tinytorch_amd.hip import sync
    prewarm(stepper.step)
    for _ in range(warmup):
        stepper.step()
    sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        stepper.step()
    sync()
    return (time.perf_counter() - t0) * 1e3 / steps


def bandwidth_kernels(L, reps=50):
    """The HBM-bound kernels of the CNN step at config-4 sizes, each timed with
    HIP events over `reps` launches; algorithmic bytes = every input element
    read once + every output element written once."""
    from tinytorch_amd.hip import DevBuf, StreamTimer, check, sync
    rng = np.random.default_rng(7)
    B = 128
    out = {}

    def run(name, fn, nbytes):
        check(fn(), name)
        prewarm(fn, 0.05)
        tm = StreamTimer()
        tm.start()
        for _ in range(reps):
            fn()
        ms = tm.stop_ms() / reps
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = dict(us=round(ms * 1e3, 2), bytes=int(nbytes), gb_s=round(gbs, 1),
                         frac_of_hbm_peak=round(gbs / PEAK_HBM_GBS, 4))

    # conv1 / conv2 activations of config 4
    for tag, (C, H, F) in (("conv1", (3, 32, 32)), ("conv2", (32, 16, 64))):
        x = DevBuf.from_np(rng.uniform(0, 1, B * C * H * H).astype(np.float32))
        Kc, Ncol = C * 9, B * H * H
        col = DevBuf(Kc * Ncol)
        run(f"im2col_{tag}", lambda: L.tt_k_im2col(x.ptr, col.ptr, B, C, H, H, 3, 3, 1, 1, 1, 1, H, H),
            4 * (B * C * H * H + Kc * Ncol))
        if tag == "conv2":
            run("col2im_conv2", lambda: L.tt_k_col2im(col.ptr, x.ptr, B, C, H, H, 3, 3, 1, 1, 1, 1, H, H),
                4 * (B * C * H * H + Kc * Ncol))
        n = B * F * H * H  # conv output / relu / pool input
        a = DevBuf.from_np(rng.standard_normal(n).astype(np.float32))
        g = DevBuf.from_np(rng.standard_normal(n).astype(np.float32))
        y = DevBuf(n)
        run(f"relu_fwd_{tag}", lambda: L.tt_k_relu_fwd(a.ptr, y.ptr, n), 8 * n)
        run(f"relu_bwd_{tag}", lambda: L.tt_k_relu_bwd(a.ptr, g.ptr, y.ptr, n), 12 * n)
        Ho = H // 2
        no = B * F * Ho * Ho
        p = DevBuf(no)
        run(f"maxpool_fwd_{tag}", lambda: L.tt_k_maxpool_fwd(a.ptr, p.ptr, B, F, H, H, 2, 2, 2, 2, Ho, Ho),
            4 * (n + no))
        run(f"maxpool_bwd_{tag}", lambda: L.tt_k_maxpool_bwd(a.ptr, p.ptr, y.ptr, B, F, H, H, 2, 2, 2, 2, Ho, Ho),
            4 * (2 * n + no))
        # the step's form: pool and relu backward in one pass (a = relu output)
        y2 = DevBuf(n)
        run(f"maxpool_relu_bwd_{tag}",
            lambda: L.tt_k_maxpool2x2_relu_bwd(a.ptr, p.ptr, y.ptr, y2.ptr, B, F, H, H, Ho, Ho),
            4 * (3 * n + no))
        y2.free()
        db = DevBuf(F)
        run(f"bias_grad_{tag}", lambda: L.tt_k_bias_grad(g.ptr, db.ptr, B, F, H * H), 4 * (n + F))
        for bb in (x, col, a, g, y, p, db):
            bb.free()
    D = 4096
    h = DevBuf.from_np(rng.standard_normal(B * D).astype(np.float32))
    hp = DevBuf(B * (D + 1))
    run("padones_fwd_fc", lambda: L.tt_k_padones_fwd(h.ptr, hp.ptr, B, D), 4 * (B * D + B * (D + 1)))
    # the launch floor of this timing: a one-element fill, timed the same way
    run("launch_floor_fill1", lambda: L.tt_k_fill(hp.ptr, 1, 0.0), 4)
    sync()
    return out


def conv_kernels(L, reps=50):
    """The direct (LDS-staged) convolution kernels at config-4 shapes (the
    separate kernels the graph takes outside the two-convolution chain) and
    the chain's two kernels the CNN step runs, each timed with HIP events over
    `reps` calls (a call of dW includes its partial reduction).  Algorithmic work: 2*F*C*HH*WW*N*Ho*Wo flops; bytes:
    every input element read once + every output element written once."""
    from tinytorch_amd.hip import DevBuf, StreamTimer, check, sync
    rng = np.random.default_rng(9)
    B = 128
    out = {}
    for tag, (C, H, F) in (("conv1", (3, 32, 32)), ("conv2", (32, 16, 64))):
        x = DevBuf.from_np(rng.uniform(0, 1, B * C * H * H).astype(np.float32))
        w = DevBuf.from_np(rng.uniform(-1, 1, F * C * 9).astype(np.float32))
        b = DevBuf.from_np(np.zeros(F, np.float32))
        g = DevBuf.from_np(rng.standard_normal(B * F * H * H).astype(np.float32))
        y, dx, dw, db = DevBuf(B * F * H * H), DevBuf(B * C * H * H), DevBuf(F * C * 9), DevBuf(F)
        geo = (B, C, H, H, F, 3, 3, 1, 1, 1, 1, H, H)
        flops = 2.0 * F * C * 9 * B * H * H
        nx, ny, nw = B * C * H * H, B * F * H * H, F * C * 9
        ops = {f"fwd_{tag}": (lambda: L.tt_k_conv2d_fwd_lds(x.ptr, w.ptr, b.ptr, y.ptr, *geo),
                              4 * (nx + nw + F + ny)),
               f"dw_db_{tag}": (lambda: L.tt_k_conv2d_dw_lds(g.ptr, x.ptr, dw.ptr, db.ptr, *geo),
                                4 * (ny + nx + nw + F))}
        if tag == "conv2":  # conv1's input is the image: no dX in the training step
            ops[f"dx_{tag}"] = (lambda: L.tt_k_conv2d_dx_lds(g.ptr, w.ptr, dx.ptr, *geo),
                                4 * (ny + nw + nx))
        for name, (fn, nbytes) in ops.items():
            check(fn(), name)
            prewarm(fn, 0.05)
            tm = StreamTimer()
            tm.start()
            for _ in range(reps):
                fn()
            ms = tm.stop_ms() / reps
            tf = flops / (ms * 1e-3) / 1e12
            out[name] = dict(us=round(ms * 1e3, 2), gflop=round(flops / 1e9, 3),
                             tflops=round(tf, 1), frac_of_mfma_peak=round(tf / PEAK_FP32_MFMA_TFLOPS, 3),
                             bytes=int(nbytes), gb_s=round(nbytes / (ms * 1e-3) / 1e9, 1))
        for bb in (x, w, b, g, y, dx, dw, db):
            bb.free()
    # the step's own kernels: both convolutions (+ relus, pools, codes, the
    # flattened and padded copies and the classifier's partial sums) in one
    # launch, and the backward grid (conv2 dX, conv1 dW through the pool
    # codes, conv2 dW; with their two weight-gradient reductions)
    x = DevBuf.from_np(rng.uniform(0, 1, B * 3 * 1024).astype(np.float32))
    w1 = DevBuf.from_np((rng.standard_normal(32 * 27) * 0.27).astype(np.float32))
    w2 = DevBuf.from_np((rng.standard_normal(64 * 288) * 0.083).astype(np.float32))
    b1, b2 = DevBuf.from_np(np.zeros(32, np.float32)), DevBuf.from_np(np.zeros(64, np.float32))
    fcw = DevBuf.from_np((rng.standard_normal(4097 * 10) / 64).astype(np.float32))
    p1, k1 = DevBuf(B * 32 * 256), DevBuf(B * 32 * 256, np.uint8)
    p2, c2, d2, k2 = DevBuf(B * 4096), DevBuf(B * 4096), DevBuf(B * 4097), DevBuf(B * 4096, np.uint8)
    s1, s2, part = DevBuf(32 * 27 + 32), DevBuf(18432 + 64), DevBuf(2 * B * 10)
    g2 = DevBuf.from_np(rng.standard_normal(B * 64 * 256).astype(np.float32))
    dx2, dw1, db1, dw2, db2 = DevBuf(B * 32 * 256), DevBuf(32 * 27), DevBuf(32), DevBuf(64 * 288), DevBuf(64)
    f1, f2 = 2.0 * 32 * 27 * B * 1024, 2.0 * 64 * 288 * B * 256
    ops = {"chain_fwd": (lambda: L.tt_k_conv2d_chain_fwd(
                             x.ptr, w1.ptr, b1.ptr, w2.ptr, b2.ptr, p1.ptr, k1.ptr, p2.ptr, c2.ptr,
                             d2.ptr, k2.ptr, s1.ptr, s2.ptr, fcw.ptr, 10, part.ptr, B, 3, 32, 32,
                             32, 64),
                         f1 + f2 + 2.0 * B * 4096 * 10,
                         4 * (B * 3 * 1024 + 32 * 27 + 64 * 288 + 4097 * 10 + B * 32 * 256 +
                              3 * B * 4096 + B * 4097 + 2 * B * 10) + B * 32 * 256 + B * 4096),
           "chain_bwd": (lambda: L.tt_k_conv2d_chain_bwd(
                             g2.ptr, w2.ptr, k1.ptr, x.ptr, dx2.ptr, dw1.ptr, db1.ptr, p1.ptr,
                             dw2.ptr, db2.ptr, B, 3),
                         f1 + 2 * f2,
                         4 * (B * 64 * 256 + 64 * 288 + B * 3 * 1024 + 2 * B * 32 * 256 + 32 * 27 +
                              32 + 64 * 288 + 64) + B * 32 * 256)}
    for name, (fn, flops, nbytes) in ops.items():
        check(fn(), name)
        prewarm(fn, 0.05)
        tm = StreamTimer()
        tm.start()
        for _ in range(reps):
            fn()
        ms = tm.stop_ms() / reps
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = dict(us=round(ms * 1e3, 2), gflop=round(flops / 1e9, 3), tflops=round(tf, 1),
                         frac_of_mfma_peak=round(tf / PEAK_FP32_MFMA_TFLOPS, 3), bytes=int(nbytes),
                         gb_s=round(nbytes / (ms * 1e-3) / 1e9, 1))
    for bb in (x, w1, w2, b1, b2, fcw, p1, k1, p2, c2, d2, k2, s1, s2, part, g2, dx2, dw1, db1,
               dw2, db2):
        bb.free()
    sync()
    return out


def cpu_threads():
    n = os.environ.get("OMP_NUM_THREADS")
    try:
        n = int(n)
    except (TypeError, ValueError):
        n = len(os.sched_getaffinity(0))
    return max(1, min(n, len(os.sched_getaffinity(0))))


def median_time(fn, warmup, reps):
    """the reference's timing protocol (bench/bench_cpu.py:74-82): `warmup`
    untimed calls, then the median of `reps` timed ones, in seconds"""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline(threads):
    """The reference CPU path on this host: its AVX2 OpenMP sgemm at 4096^3,
    its autograd CNN and MLP training steps, and its 4096^3 matmul backward
    (dA = dC B^T and dB = A^T dC, the naive loops of src/autograd.c:66-103)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import orc  # the CPU baseline leg is the only part of bench.py that uses oracle/
    kind = "reference" if orc.ref_available() else "port"
    n = 4096
    A = uniform((n, n), -1, 1, 0x5EED + 1)
    B = uniform((n, n), -1, 1, 0x5EED + 2)
    C = np.zeros((n, n), np.float32)

    def run():
        if kind == "reference":
            rc = orc.ref().tt_sgemm_rowmajor(n, n, n, A.ctypes.data, B.ctypes.data, C.ctypes.data,
                                            threads)
        else:
            rc = orc.orc().orc_sgemm(n, n, n, A.ctypes.data, B.ctypes.data, C.ctypes.data, threads)
        assert rc == 0
    gflops = 2.0 * n ** 3 / median_time(run, 2, 9) / 1e9
    # CNN and MLP steps on the reference autograd path (forward, softmax,
    # NumPy CE seed, backward), warmup 5 + median of 20
    x, y, P = cnn_inputs()
    step = (lambda: orc.ref_cnn_step(x, y, **P)) if kind == "reference" else \
        (lambda: orc.cnn_step(x, y, nthreads=threads, **P))
    cnn_s = median_time(step, 5, 20)
    xm, ym, Ws = mlp_inputs()
    mstep = (lambda: orc.ref_mlp_step(xm, ym, *Ws)) if kind == "reference" else \
        (lambda: orc.mlp_step(xm, ym, *Ws, nthreads=threads))
    mlp_s = median_time(mstep, 5, 20)
    out = dict(value=round(gflops, 2), unit="GFLOP/s", cores=threads, kind=kind,
               sample="sgemm 4096^3 NN fp32 (config 3 shape), 2 warmup + median of 9 runs; "
                      "reference AVX2+FMA OpenMP kernel (src/gemm.c) built from its sources",
               cnn_step_ms=round(cnn_s * 1e3, 2),
               mlp_step_ms=round(mlp_s * 1e3, 3),
               steps_sample="config-4 CNN and config-2 MLP fwd+bwd on the reference autograd "
                            "path, 5 warmup + median of 20 (bench/bench_cpu.py:74-82)")
    if kind == "reference":
        # config 3 on the reference autograd: one forward and one backward of a
        # 4096^3 matmul whose seed is dC ~ N(0,1); backward = dA + dB
        G = np.random.default_rng(0x5EED + 3).standard_normal((n, n)).astype(np.float32)
        g = orc.RefGraph()
        nA, nB = g.leaf(A), g.leaf(B)
        t0 = time.perf_counter()
        out_n = g.add(orc.ref().ag_matmul(nA, nB))
        t1 = time.perf_counter()
        g.backward(out_n, G)
        t2 = time.perf_counter()
        g.release()
        out["matmul_bwd_4096_s"] = round(t2 - t1, 3)
        out["matmul_bwd_4096_gflops"] = round(2 * 2.0 * n ** 3 / (t2 - t1) / 1e9, 2)
        out["matmul_fwd_4096_s"] = round(t1 - t0, 3)
        out["bwd_sample"] = ("config 3: one ag_matmul forward + one backward (dA and dB, "
                             "the reference's naive matmul_nt / matmul_tn) at 4096^3, 1 run")
    return out


# secondary GEMM shapes (3 and 5): name -> (M, N, K, transA, transB)
GEMM_SHAPES = {"sgemm_1024": (1024, 1024, 1024, 0, 0),
               "sgemm_4096_nt_dA": (4096, 4096, 4096, 0, 1),
               "sgemm_4096_tn_dB": (4096, 4096, 4096, 1, 0),
               "sgemm_8192": (8192, 8192, 8192, 0, 0),
               "sgemm_ragged_1000x1003x997": (1000, 1003, 997, 0, 0),
               "sgemm_tall_65536x64x4096": (65536, 64, 4096, 0, 0)}


def gemm_shapes(L, only=None):
    out = {}
    for name, (M, N, K, ta, tb) in GEMM_SHAPES.items():
        if only and name != only:
            continue
        gg = Gemm(L, M, N, K, ta, tb)
        steps = max(10, min(200, int(3e12 / gg.flops())))
        _, ms = time_gemm(L, gg, steps, 2)
        out[name] = dict(tflops=round(gg.flops() / (ms * 1e-3) / 1e12, 2), ms=round(ms, 4),
                         frac_of_peak=round(gg.flops() / (ms * 1e-3) / 1e12 /
                                            PEAK_FP32_MFMA_TFLOPS, 4))
        gg.free()
        log(name, out[name])
    return out


PROBE_LIB = os.path.join(ROOT, "build", "probe", "libtinytorch.so")


def phase_split(ts, kid, blocks, points, names):
    """Per-phase durations (us) of kernel `kid`'s workgroups `blocks` from the
    probe timestamps (100 MHz): the median over the workgroups of each span
    between consecutive points, and the span of the whole set."""
    t = ts[kid][blocks].astype(np.int64)
    out = {"workgroups": int(t.shape[0]),
           "span_us": round(float(t[:, points[-1]].max() - t[:, points[0]].min()) * 0.01, 2)}
    for (a, b), nm in zip(zip(points[:-1], points[1:]), names):
        out[nm] = round(float(np.median(t[:, b] - t[:, a])) * 0.01, 2)
    return out


def phases(L):
    """Phase timestamps (probe.h) of thread 0 of every workgroup: the config-4
    CNN step's convolution kernels and classifier backward (the last of 30
    steps) and gemm_mid_kernel at 1024^3 and 1000x1003x997 (the last of 50
    launches)."""
    from tinytorch_amd.hip import sync
    def read(name):
        f = getattr(L, "tt_probe_read_" + name)
        f.restype = ctypes.c_int
        f.argtypes = [ctypes.c_void_p, ctypes.c_int]
        buf = np.zeros(4 * 1024 * 16, np.uint64)
        if f(buf.ctypes.data, buf.size) != 0:
            raise RuntimeError("tt_probe_read_" + name)
        return buf.reshape(4, 1024, 16)
    st = CnnStep(L)
    for _ in range(30):
        st.step()
    sync()
    conv, head = read("conv"), read("head")
    nchain = 2 * st.B
    out = {
        "conv_chain_fwd_kernel": phase_split(conv, 0, slice(0, nchain), [0, 1, 2, 3, 4],
                                             ["staging", "conv1_relu_pool", "conv2",
                                              "relu_pool_fc_epilogue"]),
        "conv_chain_bwd_dw2_kernel/chain": phase_split(conv, 1, slice(0, nchain),
                                                       [0, 1, 2, 3, 15],
                                                       ["staging", "conv2_dx", "pool1_relu_bwd",
                                                        "conv1_dw_partials"]),
        "conv_chain_bwd_dw2_kernel/conv2_dw": phase_split(conv, 1, slice(nchain, 2 * nchain),
                                                          [0, 5, 6, 15],
                                                          ["staging", "mfma_issue",
                                                           "wave_sums_partials"]),
    }
    t1 = conv[1][:2 * nchain].astype(np.int64)
    out["conv_chain_bwd_dw2_kernel/grid_span_us"] = round(float(t1[:, 15].max() - t1[:, 0].min()) * 0.01, 2)
    nbw = int(np.count_nonzero(head[0, :, 2]))
    out["head_bwd_kernel/dw"] = phase_split(head, 0, slice(0, nbw), [0, 6, 7, 1, 2],
                                            ["partials_load", "softmax_ce", "stage_a", "dw_sums"])
    nda = int(np.count_nonzero(head[0, :, 5]))
    out["head_bwd_kernel/da_pool"] = phase_split(head, 0, slice(nbw, nbw + nda), [0, 6, 7, 4, 5],
                                                 ["partials_load", "softmax_ce", "stage_w",
                                                  "da_pool_bwd_stores"])
    for (M, N, K) in ((1024, 1024, 1024), (1000, 1003, 997)):
        g = Gemm(L, M, N, K)
        prewarm(g.launch, 0.2)
        for _ in range(50):
            g.launch()
        sync()
        gm = read("gemm")
        out[f"gemm_mid_kernel/{M}x{N}x{K}"] = phase_split(
            gm, 0, slice(0, 256), [0, 1, 2, 3, 4, 5],
            ["first_tiles", "k_loop_wave0", "wave0_sums_to_lds", "other_waves", "sum_and_store"])
        g.free()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU; --gpus {args.gpus} is not supported "
              "(a multi-GPU run would be data parallel: one process per GPU, each with B/N "
              "images, and one all-reduce of the weight gradients per step)", file=sys.stderr)
        sys.exit(2)
    import tinytorch_amd
    if args.phases:
        if not os.path.exists(PROBE_LIB):
            sys.exit(f"bench.py: {PROBE_LIB} is not built; run `make probe`")
        tinytorch_amd.LIB_PATH = PROBE_LIB
    tinytorch_amd.require_gpu()
    L = tinytorch_amd.lib()
    if args.phases:
        print(json.dumps(phases(L)))
        return
    log("device", tinytorch_amd.device_name())
    if args.cnn_only:
        ms = time_steps(CnnStep(L), args.steps, args.warmup)
        print(json.dumps({"cnn_step_ms": round(ms, 4), "steps": args.steps, "warmup": args.warmup}))
        return
    if args.mlp_only:
        ms = time_steps(MlpStep(L), args.steps, args.warmup)
        print(json.dumps({"mlp_step_ms": round(ms, 4), "steps": args.steps, "warmup": args.warmup}))
        return
    if args.conv_kernels:
        print(json.dumps(conv_kernels(L)))
        return
    if args.hbm_kernels:
        print(json.dumps(bandwidth_kernels(L)))
        return
    if args.gemm_shapes or args.gemm_shape:
        if args.gemm_shape and args.gemm_shape not in GEMM_SHAPES:
            sys.exit(f"bench.py: unknown --gemm-shape {args.gemm_shape}; one of {list(GEMM_SHAPES)}")
        print(json.dumps(gemm_shapes(L, args.gemm_shape)))
        return
    if args.copy_calib:
        from tinytorch_amd.hip import DevBuf, check, sync
        n = 256 << 20  # floats: 1 GiB read + 1 GiB written per launch (4x the MALL)
        src, dst = DevBuf(n), DevBuf(n)
        src.fill(1.0)
        for _ in range(5):
            check(L.tt_k_copy(dst.ptr, src.ptr, n), "tt_k_copy")
        sync()
        print(json.dumps({"copy_calib_bytes_each_way": n * 4, "launches": 5}))
        return

    g = Gemm(L, 4096, 4096, 4096)
    wall_ms, ev_ms = time_gemm(L, g, args.steps, args.warmup)
    value = g.flops() / (wall_ms * 1e-3) / 1e12
    achieved = g.flops() / (ev_ms * 1e-3) / 1e12
    g.free()
    log(f"sgemm 4096^3: wall {wall_ms:.3f} ms/step ({value:.1f} TFLOP/s), "
        f"events {ev_ms:.3f} ms/launch ({achieved:.1f} TFLOP/s)")
    traffic = read_traffic()

    extra = {}
    if not args.no_extra:
        extra.update(gemm_shapes(L))
        cnn = CnnStep(L)
        extra["cnn_step"] = step_figures(cnn, CNN_STEP_GFLOP, 20)
        extra["cnn_step_ms"] = extra["cnn_step"]["ms"]
        log("cnn step", extra["cnn_step"])
        mlp = MlpStep(L)
        extra["mlp_step"] = step_figures(mlp, MLP_STEP_GFLOP, 50)
        extra["mlp_step_ms"] = extra["mlp_step"]["ms"]
        log("mlp step", extra["mlp_step"])
        extra["conv_kernels"] = conv_kernels(L)
        for k, v in extra["conv_kernels"].items():
            log(f"{k:22s} {v['us']:8.2f} us {v['tflops']:6.1f} TFLOP/s ({100 * v['frac_of_mfma_peak']:.1f}% of fp32 MFMA)")
        extra["hbm_kernels"] = bandwidth_kernels(L)
        for k, v in extra["hbm_kernels"].items():
            log(f"{k:22s} {v['us']:8.2f} us {v['gb_s']:8.1f} GB/s ({100 * v['frac_of_hbm_peak']:.1f}% of 8 TB/s)")

    cpu = None
    if not args.no_cpu:
        threads = cpu_threads()
        log(f"cpu baseline on {threads} threads ...")
        cpu = cpu_baseline(threads)
        log("cpu", cpu)

    if cpu and extra.get("cnn_step"):
        for key, cpu_key in (("cnn_step", "cnn_step_ms"), ("mlp_step", "mlp_step_ms")):
            extra[key]["cpu_ms"] = cpu[cpu_key]
            extra[key]["speedup_vs_cpu"] = round(cpu[cpu_key] / extra[key]["ms"], 1)
        if "matmul_bwd_4096_s" in cpu:
            gpu_ms = extra["sgemm_4096_nt_dA"]["ms"] + extra["sgemm_4096_tn_dB"]["ms"]
            extra["matmul_bwd_4096"] = dict(ms=round(gpu_ms, 4), cpu_ms=round(
                cpu["matmul_bwd_4096_s"] * 1e3, 1), speedup_vs_cpu=round(
                cpu["matmul_bwd_4096_s"] * 1e3 / gpu_ms, 1))

    out = {
        "metric": "fp32 GEMM TFLOP/s @4096^3 (% MFMA peak) + CNN fwd+bwd step ms",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (uniform[-1,1] operands from fixed seeds)",
        "config": {"workload": "sgemm C=A*B fp32 row-major, M=N=K=4096",
                   "frac_of_fp32_mfma_peak": round(value / PEAK_FP32_MFMA_TFLOPS, 4)},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3),
                     "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
