#!/usr/bin/env python3
"""Benchmark of the MI355X HIP backend's hot path (one GPU).

Headline (`value`): fused Q4_0 dequant-matvec throughput in GB/s on the decode
shape of the benchmark configuration 2: W = Q4_0 [K=4096, M=14336], x = F32
[4096, 1], y = F32 [14336, 1]. One step = one fused kernel launch over one
batch. Algorithmic bytes per step = W blocks + x + y = 33,103,872 B.

The same run also measures, each against its roofline (`extra`):
  - bulk dequant of all five formats on 4096 x 11008 (configuration 1), GB/s;
  - the fused kernel for Q4_0/Q5_0 at N = 1 and 16 (configuration 2), Q4_0 at
    N = 64, and configuration 0's product (Q8_0 [4096, 4096] times 8 columns);
  - the F32 mul_mat forward + both backward products of a 4096x4096 linear
    layer over 512 tokens (configuration 3) and the batched broadcast product
    with a permuted src1 (configuration 4), TFLOP/s on the FP32 MFMA roofline.

Timing: steps are enqueued on one stream and captured into a HIP graph (host
launch overhead stays out of the timed region); HIP events on that stream
bracket each timed replay of the K launches, and the headline is the median
over --replays replays (the spread is reported beside it). Inputs rotate over buffer sets totalling more
than 512 MB so the 256 MB Infinity Cache cannot hold them between steps.

cpu_baseline: the reference's own CPU path for the headline workload, compiled
from its sources into oracle/_ref (gguf_tensor_to_f32 into the F32 weight, then
mul_mat on its serial CPU Device), on one host core (kind "reference"; its y is
checked bit for bit against the oracle). Where oracle/_ref is absent, the
oracle's restatement of the same path (kind "port"). extra.cpu_baseline_port
times the restatement on one core, extra.cpu_baseline_all_cores on every core
this process may use (sched_getaffinity), and extra.host names the CPU model.
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "train.cpp_amd"

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
FP32_MFMA_PEAK_TFS = 157.3   # MI355X dense FP32 matrix, TFLOP/s
METRIC = "Q4_0 dequant-matvec GB/s (% HBM peak); F32 mul_mat TFLOP/s (% MFMA peak)"


def load_pkg():
    spec = importlib.util.spec_from_file_location("traincpp_amd", PKG / "__init__.py",
                                                  submodule_search_locations=[str(PKG)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["traincpp_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


# ---------------------------------------------------------------- HIP runtime (events, streams, graphs)

class Hip:
    def __init__(self):
        self.rt = C.CDLL("libamdhip64.so")
        V, P = C.c_void_p, C.POINTER(C.c_void_p)
        for name, args in {
            "hipStreamCreate": [P], "hipStreamDestroy": [V], "hipStreamSynchronize": [V],
            "hipEventCreate": [P], "hipEventRecord": [V, V], "hipEventSynchronize": [V],
            "hipEventElapsedTime": [C.POINTER(C.c_float), V, V], "hipEventDestroy": [V],
            "hipStreamBeginCapture": [V, C.c_int], "hipStreamEndCapture": [V, P],
            "hipGraphInstantiate": [P, V, V, V, C.c_size_t], "hipGraphLaunch": [V, V],
            "hipGraphExecDestroy": [V], "hipGraphDestroy": [V], "hipDeviceSynchronize": [],
        }.items():
            fn = getattr(self.rt, name)
            fn.argtypes = args
            fn.restype = C.c_int

    def ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed with hipError_t {rc}")

    def stream(self):
        s = C.c_void_p()
        self.ok(self.rt.hipStreamCreate(C.byref(s)), "hipStreamCreate")
        return s.value

    def event(self):
        e = C.c_void_p()
        self.ok(self.rt.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e.value

    def elapsed_ms(self, a, b):
        f = C.c_float()
        self.ok(self.rt.hipEventElapsedTime(C.byref(f), a, b), "hipEventElapsedTime")
        return f.value


class Timer:
    """Times `steps` calls of fn(i) enqueued on one stream, as a HIP graph replay
    when capture works (falls back to plain stream launches). `replays` timed
    replays of the same graph; run() returns their median ms per step and keeps
    every replay's figure in `last_replays`.

    Each timed replay runs behind an untimed replay of the captured graph that
    is still executing: the start event completes when that replay's last launch
    does, and the timed launches, enqueued meanwhile, follow at once. The timed
    `steps` launches go once as plain stream launches and once as a second
    graph replay; run() reports the faster of the two medians (`self.mode` says
    which). A graph launch costs ~6 us of GPU time of its own (measured on the
    headline: 7.64 us per launch for 20-launch replays back to back, 7.30 us for
    200-launch replays, 7.39 us for 20 stream launches behind a replay), 4 % of a
    20-step replay; stream launches avoid it unless the host cannot enqueue
    them as fast as the GPU runs them. A replay started from an idle stream,
    submission latency included, is measured too (`last_replays_outer`)."""

    def __init__(self, hip: Hip, use_graph: bool = True, replays: int = 1):
        self.hip = hip
        self.stream = hip.stream()
        self.e0, self.e1 = hip.event(), hip.event()
        self.use_graph = use_graph
        self.replays = replays
        self.last_replays: list[float] = []
        self.last_replays_outer: list[float] = []
        self.last_replays_graph: list[float] = []
        self.last_replays_stream: list[float] = []
        self.mode = ""

    def run(self, fn, steps: int, warmup: int, replays: int | None = None) -> tuple[float, str]:
        hip, rt, s = self.hip, self.hip.rt, self.stream
        for i in range(warmup):
            fn(i, s)
        hip.ok(rt.hipStreamSynchronize(s), "sync")
        mode = "stream"
        exec_ = None
        if self.use_graph:
            graph, gexec = C.c_void_p(), C.c_void_p()
            try:
                hip.ok(rt.hipStreamBeginCapture(s, 2), "hipStreamBeginCapture")  # relaxed mode
                # step i of every replay uses input set i % sets (see rotation_sets)
                for i in range(steps):
                    fn(i, s)
                hip.ok(rt.hipStreamEndCapture(s, C.byref(graph)), "hipStreamEndCapture")
                hip.ok(rt.hipGraphInstantiate(C.byref(gexec), graph, None, None, 0), "hipGraphInstantiate")
                exec_ = gexec.value
                # untimed replays for at least 20 ms, so an idle GPU's clocks have
                # ramped up before the timed replay (the first replay after a pause
                # measured up to 5 % slower)
                t_end = time.perf_counter() + 0.02
                while True:
                    hip.ok(rt.hipGraphLaunch(exec_, s), "hipGraphLaunch")
                    hip.ok(rt.hipStreamSynchronize(s), "sync")
                    if time.perf_counter() >= t_end:
                        break
                mode = "graph"
            except RuntimeError:
                exec_ = None
        def timed(behind, body):
            hip.ok(rt.hipDeviceSynchronize(), "sync")
            if behind:
                hip.ok(rt.hipGraphLaunch(exec_, s), "hipGraphLaunch (untimed)")
            hip.ok(rt.hipEventRecord(self.e0, s), "record")
            body()
            hip.ok(rt.hipEventRecord(self.e1, s), "record")
            hip.ok(rt.hipEventSynchronize(self.e1), "sync")
            hip.ok(rt.hipDeviceSynchronize(), "sync")
            return hip.elapsed_ms(self.e0, self.e1) / steps

        def launches():
            for i in range(steps):
                fn(i, s)

        def replay():
            hip.ok(rt.hipGraphLaunch(exec_, s), "hipGraphLaunch")

        outer, in_stream, in_graph = [], [], []
        for _ in range(replays or self.replays):
            if exec_ is None:
                outer.append(timed(False, launches))
                continue
            outer.append(timed(False, replay))
            in_stream.append(timed(True, launches))
            in_graph.append(timed(True, replay))
        if exec_ is not None:
            rt.hipGraphExecDestroy(exec_)
            if np.median(in_stream) <= np.median(in_graph):
                per_step, mode = in_stream, "stream launches behind a graph replay"
            else:
                per_step, mode = in_graph, "graph replay behind a graph replay"
        else:
            per_step = outer
        self.mode = mode
        self.last_replays = per_step
        self.last_replays_outer = outer
        self.last_replays_graph = in_graph
        self.last_replays_stream = in_stream
        return float(np.median(per_step)), mode


# ---------------------------------------------------------------- workloads

def rotation_count(bytes_per_set: int, floor: int = 3, target: int = 512 << 20) -> int:
    return max(floor, -(-target // max(bytes_per_set, 1)) + 1)


def rotation_sets(bytes_per_set: int, steps: int) -> int:
    """Input sets for a timed graph of `steps` launches in which step i reads set
    i % sets. The smallest divisor of `steps` that is at least rotation_count(), so
    that a replay ends on the last set and the next replay starts on set 0: between
    two reads of one set, every other set is read, more than 512 MB (twice the
    Infinity Cache), across replay boundaries too. With fewer steps than that
    count, every step of a replay reads its own set."""
    need = rotation_count(bytes_per_set)
    # (with fewer steps than `need`, a replay reads `steps` different sets and the
    # next replay reads them again)
    for d in range(need, steps + 1):
        if steps % d == 0:
            return d
    return need


def qmatvec_case(H, synth, timer, t, K, M, N, steps, warmup, cfg=2):
    blk = synth.block_bytes(synth.quant_blocks(t, K * M // 32, synth.config_seed(cfg, t)))
    x = synth.normal(synth.config_seed(cfg, 100 + N), K * N)
    alg_bytes = blk.nbytes + x.nbytes + M * N * 4
    sets = rotation_sets(alg_bytes, steps)
    ws = [H.DeviceBuffer(blk.nbytes).upload(blk) for _ in range(sets)]
    xs = [H.DeviceBuffer(x.nbytes).upload(x) for _ in range(sets)]
    ys = [H.DeviceBuffer(M * N * 4) for _ in range(sets)]
    nb1_w = (K // 32) * H.BLOCK_BYTES[t]

    def step(i, s):
        j = i % sets
        H.qmatvec(t, ws[j].ptr, K, M, nb1_w, xs[j].ptr, N, K * 4, ys[j].ptr, M * 4, s)

    ms, mode = timer.run(step, steps, warmup)
    reps = list(timer.last_replays)
    outer = list(timer.last_replays_outer)
    other = list(timer.last_replays_graph if timer.last_replays is timer.last_replays_stream
                 else timer.last_replays_stream)
    for b in ws + xs + ys:
        b.free()
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    flops = 2.0 * K * M * N
    return {"ms": ms, "bytes": alg_bytes, "GB/s": gbs, "frac_hbm": gbs / HBM_PEAK_GBS,
            "TFLOP/s": flops / (ms * 1e-3) / 1e12, "sets": sets, "timing": mode,
            "replays_us": [round(r * 1e3, 3) for r in reps],
            "replays_with_submission_us": [round(r * 1e3, 3) for r in outer],
            "replays_other_method_us": [round(r * 1e3, 3) for r in other]}, blk, x


def dequant_case(H, synth, timer, t, n_blocks, steps, warmup):
    blk = synth.block_bytes(synth.quant_blocks(t, n_blocks, synth.config_seed(1, t)))
    alg_bytes = blk.nbytes + n_blocks * 32 * 4
    sets = rotation_sets(alg_bytes, steps)
    srcs = [H.DeviceBuffer(blk.nbytes).upload(blk) for _ in range(sets)]
    dsts = [H.DeviceBuffer(n_blocks * 128) for _ in range(sets)]

    def step(i, s):
        j = i % sets
        H.dequant(t, srcs[j].ptr, n_blocks, dsts[j].ptr, s)

    ms, mode = timer.run(step, steps, warmup)
    for b in srcs + dsts:
        b.free()
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    return {"ms": ms, "bytes": alg_bytes, "GB/s": gbs, "frac_hbm": gbs / HBM_PEAK_GBS, "sets": sets,
            "timing": mode}


def mul_mat_config3(H, synth, timer, steps, warmup):
    """Y = mul_mat(W, X); dX = mul_mat(transpose(W), dY); dW^T = mul_mat(transpose(dY), transpose(X))."""
    K = M = 4096
    T = 512
    n = K * M // 32
    q = synth.block_bytes(synth.quant_blocks(7, n, synth.config_seed(3, 0)))  # Q5_1 weights
    qd = H.DeviceBuffer(q.nbytes).upload(q)
    Wd = H.DeviceBuffer(K * M * 4)
    H.dequant(7, qd.ptr, n, Wd.ptr)  # W is the GPU dequant of the Q5_1 blocks
    H.sync()
    Xd = H.DeviceBuffer(K * T * 4).upload(synth.normal(synth.config_seed(3, 1), K * T))
    dYd = H.DeviceBuffer(K * T * 4).upload(synth.normal(synth.config_seed(3, 2), K * T, 0.0, 1e-2))
    Yd = H.DeviceBuffer(M * T * 4)
    dXd = H.DeviceBuffer(K * T * 4)
    dWd = H.DeviceBuffer(K * M * 4)
    f4 = 4
    W = H.tensor(Wd.ptr, [K, M, 1, 1], [f4, K * f4, K * M * f4, K * M * f4])
    Wt = H.tensor(Wd.ptr, [M, K, 1, 1], [K * f4, f4, K * M * f4, K * M * f4])
    X = H.tensor(Xd.ptr, [K, T, 1, 1], [f4, K * f4, K * T * f4, K * T * f4])
    Xt = H.tensor(Xd.ptr, [T, K, 1, 1], [K * f4, f4, K * T * f4, K * T * f4])
    dY = H.tensor(dYd.ptr, [M, T, 1, 1], [f4, M * f4, M * T * f4, M * T * f4])
    dYt = H.tensor(dYd.ptr, [T, M, 1, 1], [M * f4, f4, M * T * f4, M * T * f4])
    Y = H.tensor(Yd.ptr, [M, T, 1, 1], H.contiguous_nb([M, T, 1, 1]))
    dX = H.tensor(dXd.ptr, [K, T, 1, 1], H.contiguous_nb([K, T, 1, 1]))
    dWt = H.tensor(dWd.ptr, [M, K, 1, 1], H.contiguous_nb([M, K, 1, 1]))
    prods = {"fwd Y=W.X": (W, X, Y), "bwd dX=W^T.dY": (Wt, dY, dX), "bwd dW^T=dY^T.X^T": (dYt, Xt, dWt)}
    out = {}
    total_ms = 0.0
    for name, (a, b, d) in prods.items():
        ms, mode = timer.run(lambda i, s, a=a, b=b, d=d: H.mul_mat_f32(a, b, d, s), steps, warmup)
        fl = 2.0 * K * M * T
        out[name] = {"ms": ms, "TFLOP/s": fl / (ms * 1e-3) / 1e12,
                     "frac_mfma": fl / (ms * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFS, "timing": mode}
        total_ms += ms
    fl = 3 * 2.0 * K * M * T
    out["fwd+bwd"] = {"ms": total_ms, "TFLOP/s": fl / (total_ms * 1e-3) / 1e12,
                      "frac_mfma": fl / (total_ms * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFS}
    for b in (qd, Wd, Xd, dYd, Yd, dXd, dWd):
        b.free()
    return out


def mul_mat_config4(H, synth, timer, steps, warmup):
    A = synth.normal(synth.config_seed(4, 0), 128 * 1024 * 8 * 4)
    B = synth.normal(synth.config_seed(4, 1), 128 * 32 * 512 * 4)
    Ad = H.DeviceBuffer(A.nbytes).upload(A)
    Bd = H.DeviceBuffer(B.nbytes).upload(B)
    Dd = H.DeviceBuffer(1024 * 512 * 32 * 4 * 4)
    a = H.tensor(Ad.ptr, [128, 1024, 8, 4], H.contiguous_nb([128, 1024, 8, 4]))
    b = H.tensor(Bd.ptr, [128, 512, 32, 4], [4, 16384, 512, 8388608])  # permute(base[128,32,512,4],0,2,1,3)
    d = H.tensor(Dd.ptr, [1024, 512, 32, 4], H.contiguous_nb([1024, 512, 32, 4]))
    ms, mode = timer.run(lambda i, s: H.mul_mat_f32(a, b, d, s), steps, warmup)
    fl = 2.0 * 128 * 1024 * 512 * 128
    for x in (Ad, Bd, Dd):
        x.free()
    return {"ms": ms, "TFLOP/s": fl / (ms * 1e-3) / 1e12, "frac_mfma": fl / (ms * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFS,
            "timing": mode}


def linear_step(H, synth, timer, steps, warmup):
    """One training step of configuration 3's Linear layer with bias and the loss
    L = sum(mul(y, g)): the kernels HipDevice::graph_compute runs for the graph
    the reference's autograd builds (src/core/trc_autograd.cpp: graph_reset's
    fills, then mul_mat, add, mul, sum, repeat, mul, repeat_back, acc, dW, the
    transposed mul_mat of dX, acc), in that order through the C ABI on one
    stream. dW's chain (the transposed product dW^T, its transpose, cont and the
    acc into W's accumulator) runs as graph_compute fuses it: one product
    mul_mat(X^T, dY^T) added into the accumulator (trc_hip_mul_mat_acc_f32).
    Reported per step, with the products' share."""
    K = M = 4096
    T = 512
    f4 = 4
    n = K * M // 32
    q = synth.block_bytes(synth.quant_blocks(7, n, synth.config_seed(3, 0)))
    qd = H.DeviceBuffer(q.nbytes).upload(q)
    bufs = {}

    def buf(name, nfloat):
        bufs[name] = H.DeviceBuffer(max(nfloat, 4) * 4)
        return bufs[name]

    Wd = buf("W", K * M)
    H.dequant(7, qd.ptr, n, Wd.ptr)
    H.sync()
    qd.free()
    Xd = buf("X", K * T).upload(synth.normal(synth.config_seed(3, 1), K * T))
    bd = buf("b", M).upload(synth.normal(synth.config_seed(3, 3), M))
    Gd = buf("G", M * T).upload(synth.normal(synth.config_seed(3, 2), M * T, 0.0, 1e-2))
    for name, nf in (("MM", M * T), ("Y", M * T), ("YG", M * T), ("L", 1), ("dL", 1), ("R", M * T), ("DY", M * T),
                     ("DB", M), ("DX", K * T), ("gW", K * M), ("gX", K * T),
                     ("gb", M)):
        buf(name, nf)

    def t(name, ne, nb=None):
        return H.tensor(bufs[name].ptr, ne, nb if nb is not None else H.contiguous_nb(ne))

    W, X, b, G = t("W", [K, M, 1, 1]), t("X", [K, T, 1, 1]), t("b", [M, 1, 1, 1]), t("G", [M, T, 1, 1])
    MM, Y, YG = t("MM", [M, T, 1, 1]), t("Y", [M, T, 1, 1]), t("YG", [M, T, 1, 1])
    L, dL, R, DY = t("L", [1, 1, 1, 1]), t("dL", [1, 1, 1, 1]), t("R", [M, T, 1, 1]), t("DY", [M, T, 1, 1])
    DB, gb = t("DB", [M, 1, 1, 1]), t("gb", [M, 1, 1, 1])
    DYt = t("DY", [T, M, 1, 1], [M * f4, f4, M * T * f4, M * T * f4])
    Xt = t("X", [T, K, 1, 1], [K * f4, f4, K * T * f4, K * T * f4])
    gW = t("gW", [K, M, 1, 1])
    Wt = t("W", [M, K, 1, 1], [K * f4, f4, K * M * f4, K * M * f4])
    DX, gX = t("DX", [K, T, 1, 1]), t("gX", [K, T, 1, 1])

    def step(i, s):
        # graph_reset: gradient accumulators to 0, the loss gradient to 1
        H.fill_f32(bufs["gW"].ptr, 0.0, K * M, s)
        H.fill_f32(bufs["gX"].ptr, 0.0, K * T, s)
        H.fill_f32(bufs["gb"].ptr, 0.0, M, s)
        H.fill_f32(bufs["dL"].ptr, 1.0, 1, s)
        # forward
        H.mul_mat_f32(W, X, MM, s)
        H.add_f32(MM, b, Y, s)
        H.mul_f32(Y, G, YG, s)
        H.sum_f32(YG, L, s)
        # backward
        H.repeat_f32(dL, R, s)
        H.mul_f32(R, G, DY, s)
        H.repeat_back_f32(DY, DB, s)
        H.acc_f32(gb, DB, gb, M * f4, M * f4, M * f4, 0, True, s)
        H.mul_mat_acc_f32(Xt, DYt, gW, s)
        H.mul_mat_f32(Wt, DY, DX, s)
        H.acc_f32(gX, DX, gX, K * f4, K * T * f4, K * T * f4, 0, True, s)

    ms, mode = timer.run(step, steps, warmup)
    prods = {}
    for name, (a, bb, d, fn) in {"fwd": (W, X, MM, H.mul_mat_f32), "dW (added into its accumulator)":
                                 (Xt, DYt, gW, H.mul_mat_acc_f32), "dX": (Wt, DY, DX, H.mul_mat_f32)}.items():
        pm, _ = timer.run(lambda i, s, a=a, bb=bb, d=d, fn=fn: fn(a, bb, d, s), steps, warmup)
        prods[name] = round(pm * 1e3, 2)
    for v in bufs.values():
        v.free()
    fl = 3 * 2.0 * K * M * T
    return {"us": ms * 1e3, "products_us": prods, "products_sum_us": round(sum(prods.values()), 2),
            "other_kernels_us": round(ms * 1e3 - sum(prods.values()), 2), "TFLOP/s": fl / (ms * 1e-3) / 1e12,
            "frac_mfma": fl / (ms * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFS, "timing": mode, "kernel_launches": 16}


def mul_mat_config0(H, synth, timer, N, steps, warmup):
    """Configuration 0's product after the GGUF warm start: W F32 [4096, 4096] (the
    GPU dequant of the Q8_0 blocks) times X F32 [4096, N] through
    trc_hip_mul_mat_f32. HBM-bound: algorithmic bytes = W + X + Y."""
    K = M = 4096
    n = K * M // 32
    raw = synth.block_bytes(synth.quant_blocks(H.TYPE_Q8_0, n, synth.config_seed(0, 8)))
    x = synth.normal(synth.config_seed(0, 100 + N), K * N)
    alg_bytes = K * M * 4 + x.nbytes + M * N * 4
    sets = rotation_sets(alg_bytes, steps)
    qd = H.DeviceBuffer(raw.nbytes).upload(raw)
    ws = [H.DeviceBuffer(K * M * 4) for _ in range(sets)]
    for w in ws:
        H.dequant(H.TYPE_Q8_0, qd.ptr, n, w.ptr)
    H.sync()
    qd.free()
    xs = [H.DeviceBuffer(x.nbytes).upload(x) for _ in range(sets)]
    ys = [H.DeviceBuffer(M * N * 4) for _ in range(sets)]
    ts = [(H.tensor(w.ptr, [K, M, 1, 1], H.contiguous_nb([K, M, 1, 1])),
           H.tensor(xb.ptr, [K, N, 1, 1], H.contiguous_nb([K, N, 1, 1])),
           H.tensor(yb.ptr, [M, N, 1, 1], H.contiguous_nb([M, N, 1, 1]))) for w, xb, yb in zip(ws, xs, ys)]

    def step(i, s):
        a, b, d = ts[i % sets]
        H.mul_mat_f32(a, b, d, s)

    ms, mode = timer.run(step, steps, warmup)
    reps = list(timer.last_replays)
    for b in ws + xs + ys:
        b.free()
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    fl = 2.0 * K * M * N
    return {"us": ms * 1e3, "bytes": alg_bytes, "GB/s": gbs, "frac_hbm": gbs / HBM_PEAK_GBS,
            "TFLOP/s": fl / (ms * 1e-3) / 1e12, "sets": sets, "timing": mode,
            "replays_us": [round(r * 1e3, 3) for r in reps],
            "kernel": "k_mm_skinny (train.cpp_amd/csrc/hip/mul_mat.hip)"}


# ---------------------------------------------------------------- CPU baseline (reference path, oracle/)

def cpu_baseline(blk: np.ndarray, x: np.ndarray, K: int, M: int, budget_s: float, threads: int = 1):
    """The reference path for the headline workload on this host: dequantize the
    whole Q4_0 weight (gguf_tensor_to_f32) then the serial mul_mat loop. threads = 1
    follows the reference's serial design; more threads split blocks and output
    rows (same bits, every output keeps its serial k order)."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O
    lib = O.oracle()
    wf = np.empty(K * M, dtype=np.float32)
    xv = x.reshape(1, 1, 1, K)
    y = np.empty((1, 1, 1, M), dtype=np.float32)
    ane, anb = [K, M, 1, 1], [4, 4 * K, 4 * K * M, 4 * K * M]
    bne, bnb = [K, 1, 1, 1], [4, 4 * K, 4 * K, 4 * K]
    dne, dnb = [M, 1, 1, 1], [4, 4 * M, 4 * M, 4 * M]
    # one untimed pass first: it touches the output pages
    assert lib.orc_dequant(2, blk.ctypes.data, K * M // 32, wf.ctypes.data, threads) == 0
    reps, t0 = 0, time.perf_counter()
    while True:
        assert lib.orc_dequant(2, blk.ctypes.data, K * M // 32, wf.ctypes.data, threads) == 0
        assert lib.orc_mul_mat(wf.ctypes.data, O.NE(*ane), O.NB(*anb), xv.ctypes.data, O.NE(*bne), O.NB(*bnb),
                               y.ctypes.data, O.NE(*dne), O.NB(*dnb), threads) == 0
        reps += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = (time.perf_counter() - t0) / reps
    alg = blk.nbytes + x.nbytes + M * 4
    return {"value": alg / dt / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"full headline workload (Q4_0 W[4096,14336] dequant to F32 + mul_mat with x[4096,1]), "
                      f"{reps} repetitions, {dt * 1e3:.1f} ms each, oracle/oracle.cpp -O3 -ffp-contract=off, "
                      f"{threads} thread{'s' if threads > 1 else ''}"}


def cpu_baseline_reference(blk: np.ndarray, x: np.ndarray, K: int, M: int, budget_s: float):
    """The reference's own CPU path for the headline workload (oracle/_ref, built
    from its sources): gguf_tensor_to_f32 of the Q4_0 weight into the F32
    tensor's CPU buffer, then mul_mat on the reference CPU Device, repeated for
    budget_s seconds on one thread. None where oracle/_ref is absent. Its y must
    equal the oracle's bit for bit."""
    import tempfile
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O
    if not O.have_ref():
        return None
    with tempfile.TemporaryDirectory() as d:
        y, dt, reps = O.ref_headline(2, blk, x, K, M, budget_s, os.path.join(d, "w.gguf"))
    W = O.dequant(2, blk, threads=8).reshape(1, 1, M, K)
    want = O.mul_mat(W, x.reshape(1, 1, 1, K), threads=8).reshape(-1)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), "reference path differs from the oracle"
    alg = blk.nbytes + x.nbytes + M * 4
    return {"value": alg / dt / 1e9, "unit": "GB/s", "cores": 1, "kind": "reference",
            "sample": f"full headline workload (Q4_0 W[4096,14336] to F32 by the reference's gguf_tensor_to_f32, "
                      f"then mul_mat with x[4096,1] on its CPU Device), {reps} repetitions, {dt * 1e3:.1f} ms "
                      f"each, reference sources built by oracle/Makefile (-O3 -std=c++20, no -march), 1 thread; "
                      f"y bit-identical to the oracle"}


def cpu_host_info() -> dict:
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "cores_available": len(os.sched_getaffinity(0)), "os_cpu_count": os.cpu_count()}


def gguf_load_cfg0_reference_route(H, synth, threads: int, reps: int = 5):
    """The reference's gguf_load_tensor route for configuration 0 on this host:
    dequantize the Q8_0 blocks on the host into an F32 vector, then upload the
    64 MiB F32 weight. The dequant is the reference's own gguf_tensor_to_f32
    (oracle/_ref, 1 thread, mean over ~1 s) where it is built, else the oracle's
    restatement; the upload is timed here (median of `reps`)."""
    import tempfile
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O
    K = M = 4096
    n = K * M // 32
    raw = synth.block_bytes(synth.quant_blocks(H.TYPE_Q8_0, n, synth.config_seed(0, 8)))
    if O.have_ref():
        with tempfile.TemporaryDirectory() as d:
            f32, dq, _ = O.ref_dequant_timed(H.TYPE_Q8_0, raw, 1.0, os.path.join(d, "w.gguf"))
        code = "reference gguf_tensor_to_f32 (oracle/_ref)"
    else:
        f32 = np.empty(K * M, np.float32)
        t0 = time.perf_counter()
        assert O.oracle().orc_dequant(H.TYPE_Q8_0, raw.ctypes.data, n, f32.ctypes.data, threads) == 0
        dq = time.perf_counter() - t0
        code = "oracle/oracle.cpp"
    w = H.DeviceBuffer(K * M * 4)
    times = []
    for r in range(reps + 1):
        t0 = time.perf_counter()
        w.upload(f32)
        times.append(time.perf_counter() - t0)
    w.free()
    up = float(np.median(times[1:]))
    return {"ms": (dq + up) * 1e3, "dequant_ms": dq * 1e3, "upload_ms": up * 1e3, "threads": 1,
            "sample": f"Q8_0 4096x4096 blocks in memory -> host dequant ({code}) -> 64 MiB H2D"}


def cpu_other_paths(synth, budget_s: float, threads: int):
    """The reference CPU path of the other two hot paths on this host: H1 =
    gguf_tensor_to_f32's quant branch on configuration 1's Q4_0 blocks, in
    memory; H3 = configuration 3's forward product on a bounded slice of 8 of
    its 512 output columns (1/64), extrapolated to the whole product. One thread
    runs the reference's own code (oracle/_ref, where built; "code": "reference"),
    `threads` threads the oracle's restatement split over threads (same bits;
    "code": "port")."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O
    lib = O.oracle()
    out = {}

    def timed(fn):
        fn()  # untimed: first touch of the output pages
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            if time.perf_counter() - t0 >= budget_s:
                return (time.perf_counter() - t0) / reps, reps

    import tempfile
    ref = O.have_ref()
    n = 4096 * 11008 // 32
    blk = synth.block_bytes(synth.quant_blocks(2, n, synth.config_seed(1, 2)))
    wf = np.empty(n * 32, dtype=np.float32)
    for nt in sorted({1, threads}):
        if nt == 1 and ref:  # the reference's own serial gguf_tensor_to_f32
            with tempfile.TemporaryDirectory() as d:
                _, dt, reps = O.ref_dequant_timed(2, blk, budget_s, os.path.join(d, "w.gguf"))
        else:
            dt, reps = timed(lambda nt=nt: lib.orc_dequant(2, blk.ctypes.data, n, wf.ctypes.data, nt))
        out[f"dequant_cfg1_q4_0_{nt}t"] = {"GB/s": (blk.nbytes + n * 128) / dt / 1e9, "ms": dt * 1e3,
                                           "threads": nt, "reps": reps,
                                           "code": "reference" if nt == 1 and ref else "port"}
    del wf
    K = M = 4096
    T, cols = 512, 8
    W = synth.normal(synth.config_seed(3, 0), K * M)
    X = synth.normal(synth.config_seed(3, 1), K * T)
    Y = np.empty(M * T, dtype=np.float32)
    ane, anb = [K, M, 1, 1], [4, 4 * K, 4 * K * M, 4 * K * M]
    bne, bnb = [K, T, 1, 1], [4, 4 * K, 4 * K * T, 4 * K * T]
    dne, dnb = [M, T, 1, 1], [4, 4 * M, 4 * M * T, 4 * M * T]
    for nt in sorted({1, threads}):
        if nt == 1 and ref:  # the reference's own CPU Device on the first `cols` columns of X
            _, dt, reps = O.ref_mul_mat_timed(W, K, M, X[: K * cols], cols, budget_s)
        else:
            dt, reps = timed(lambda nt=nt: lib.orc_mul_mat_cols(W.ctypes.data, O.NE(*ane), O.NB(*anb),
                                                                X.ctypes.data, O.NE(*bne), O.NB(*bnb), Y.ctypes.data,
                                                                O.NE(*dne), O.NB(*dnb), 0, cols, nt))
        fl = 2.0 * K * M * cols
        out[f"mul_mat_cfg3_fwd_{nt}t"] = {"TFLOP/s": fl / dt / 1e12, "ms_slice": dt * 1e3,
                                          "ms_whole_product_extrapolated": dt * 1e3 * T / cols, "threads": nt,
                                          "reps": reps, "sample": f"{cols} of {T} output columns",
                                          "code": "reference" if nt == 1 and ref else "port"}
    return out


def read_traffic():
    """HBM bytes per launch of the headline kernel from the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel factor)."""
    p = ROOT / "profiles" / "qmatvec_q4_0_n1_traffic.json"
    if not p.exists():
        return None
    try:
        return float(json.loads(p.read_text())["traffic_bytes_per_launch"])
    except Exception:
        return None


def write_gguf_q8_0(path: str, raw: np.ndarray, K: int, M: int) -> int:
    """A one-tensor GGUF v3 file (tensor "w", Q8_0 [K, M], 32-byte alignment); returns
    the byte offset of the tensor data."""
    import struct
    head = bytearray(b"GGUF") + struct.pack("<IQQ", 3, 1, 1)
    key, val = b"general.architecture", b"linear"
    head += struct.pack("<Q", len(key)) + key + struct.pack("<iQ", 8, len(val)) + val
    head += struct.pack("<Q", 1) + b"w" + struct.pack("<IqqIQ", 2, K, M, 8, 0)
    head += bytes(-len(head) % 32)
    with open(path, "wb") as f:
        f.write(head)
        f.write(raw.tobytes())
        f.write(bytes(-raw.nbytes % 32))
    return len(head)


def gguf_load_cfg0(H, synth, reps: int = 7):
    """Configuration 0's warm start through the C ABI as hip_gguf_load_tensor does
    it: the Q8_0 blocks of a GGUF file (page-cache resident) mapped with mmap,
    uploaded raw (17.8 MB) and dequantized in HBM into the F32 weight (64 MiB).
    Median wall time over `reps` loads after one untimed load."""
    import tempfile
    K = M = 4096
    n = K * M // 32
    raw = synth.block_bytes(synth.quant_blocks(H.TYPE_Q8_0, n, synth.config_seed(0, 8)))
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "cfg0.gguf")
        off = write_gguf_q8_0(path, raw, K, M)
        blocks = H.DeviceBuffer(raw.nbytes)
        w = H.DeviceBuffer(K * M * 4)
        times = []
        for r in range(reps + 1):
            t0 = time.perf_counter()
            mm = np.memmap(path, dtype=np.uint8, mode="r", offset=off, shape=(raw.nbytes,))
            blocks.upload(mm)
            H.dequant(H.TYPE_Q8_0, blocks.ptr, n, w.ptr)
            H.sync()
            times.append(time.perf_counter() - t0)
            del mm
        blocks.free()
        w.free()
    t = float(np.median(times[1:]))
    return {"ms": t * 1e3, "ms_replays": [round(v * 1e3, 3) for v in times[1:]],
            "bytes_uploaded": int(raw.nbytes), "f32_bytes_in_hbm": K * M * 4,
            "file": "page-cache resident GGUF v3, mmap + pageable H2D + trc_hip_dequant"}


def copy_calibration(H, timer, steps, warmup):
    """A plain device copy of a known size (256 MiB read + 256 MiB written) through
    trc_hip_cpy: the reference point that scales the HBM traffic counters."""
    n = 64 << 20  # floats
    src = H.DeviceBuffer(n * 4)
    dst = H.DeviceBuffer(n * 4)
    H.fill_f32(src.ptr, 1.0, n)
    a = H.tensor(src.ptr, [n, 1, 1, 1], H.contiguous_nb([n, 1, 1, 1]))
    b = H.tensor(dst.ptr, [n, 1, 1, 1], H.contiguous_nb([n, 1, 1, 1]))
    ms, mode = timer.run(lambda i, s: H.cpy(a, b, s), steps, warmup)
    src.free()
    dst.free()
    return {"bytes_read": n * 4, "bytes_written": n * 4, "ms": ms, "GB/s": 2 * n * 4 / (ms * 1e-3) / 1e9,
            "timing": mode}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--replays", type=int, default=7,
                    help="timed replays of the headline's graph of --steps launches; the median is reported")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--headline-only", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only time a 256 MiB device copy (reference for the traffic counters)")
    ap.add_argument("--only", choices=["dequant", "mul_mat", "qmm", "cfg0", "qmm_sweep", "mm0", "mm0_sweep", "step"],
                    help="only time one hot path and print its figures (for counter runs): dequant = the five "
                         "formats on configuration 1, mul_mat = configurations 3 and 4, qmm = Q4_0 N=16 on "
                         "configuration 2, qmm_sweep = Q4_0 on configuration 2 for N from 1 to 64, mm0 = "
                         "configuration 0's F32 product (8 columns), mm0_sweep = the same for N from 1 to 64, step = "
                         "configuration 3's Linear training step")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this backend is measured on one GPU; multi-GPU runs are not part of this "
                                   "build (sharding across GPUs is designed, not built)", "n_gpus": args.gpus}))
        sys.exit(2)

    pkg = load_pkg()
    from traincpp_amd import hip as H
    from traincpp_amd import synth
    props = H.init(0)
    hip = Hip()
    timer = Timer(hip, use_graph=not args.no_graph, replays=3)
    K, M = 4096, 14336
    if args.calibrate_copy:
        print(json.dumps({"calibration": "copy", **copy_calibration(H, timer, args.steps, args.warmup)}), flush=True)
        return
    if args.only:
        part = {"only": args.only}
        if args.only == "dequant":
            for name, t in H.QUANT_TYPES.items():
                part[name] = dequant_case(H, synth, timer, t, 4096 * 11008 // 32, args.steps, args.warmup)
        elif args.only == "mul_mat":
            part["cfg3"] = mul_mat_config3(H, synth, timer, args.steps, args.warmup)
            part["cfg4"] = mul_mat_config4(H, synth, timer, args.steps, args.warmup)
        elif args.only == "qmm":
            part["q4_0 N=16"], _, _ = qmatvec_case(H, synth, timer, H.TYPE_Q4_0, K, M, 16, args.steps, args.warmup)
        elif args.only == "step":
            part["linear_step"] = linear_step(H, synth, timer, args.steps, args.warmup)
        elif args.only == "mm0":
            part["N=8"] = mul_mat_config0(H, synth, timer, 8, args.steps, args.warmup)
        elif args.only == "mm0_sweep":
            for n in (8, 1, 2, 3, 4, 16, 24, 32, 48, 64):
                r = mul_mat_config0(H, synth, timer, n, args.steps, args.warmup)
                part[f"N={n}"] = {"us": round(r["us"], 2), "frac_hbm": round(r["frac_hbm"], 4),
                                  "TFLOP/s": round(r["TFLOP/s"], 2), "replays_us": r["replays_us"]}
        elif args.only == "cfg0":
            part["q8_0 4096x4096 N=8"], _, _ = qmatvec_case(H, synth, timer, H.TYPE_Q8_0, 4096, 4096, 8, args.steps,
                                                           args.warmup, cfg=0)
        else:
            for n in (1, 2, 3, 4, 8, 12, 16, 17, 24, 32, 33, 48, 64):
                r, _, _ = qmatvec_case(H, synth, timer, H.TYPE_Q4_0, K, M, n, args.steps, args.warmup)
                part[f"q4_0 N={n}"] = {"us": round(r["ms"] * 1e3, 2), "frac_hbm": round(r["frac_hbm"], 4),
                                       "TFLOP/s": round(r["TFLOP/s"], 2)}
        print(json.dumps(part), flush=True)
        return

    t_wall = time.perf_counter()
    timer.replays = args.replays
    head, blk, x = qmatvec_case(H, synth, timer, H.TYPE_Q4_0, K, M, 1, args.steps, args.warmup)
    timer.replays = 3
    wall = time.perf_counter() - t_wall
    reps = head["replays_us"]
    traffic = read_traffic()
    roofline = {"bound": "hbm", "achieved": head["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": head["GB/s"] / HBM_PEAK_GBS, "traffic": traffic,
                "kernel": "k_qmatvec_dot<Q4_0> (train.cpp_amd/csrc/hip/qmatvec.hip)",
                "algorithmic_bytes_per_launch": head["bytes"]}

    extra = {"device": f"{props.name.decode()} {props.arch.decode()} CUs={props.compute_units}"}
    if not args.headline_only:
        s, w = max(20, args.steps // 2), max(5, args.warmup // 2)
        extra["qmatvec"] = {}
        for name, t in (("q4_0", H.TYPE_Q4_0), ("q5_0", H.TYPE_Q5_0)):
            for N in (1, 16):
                if name == "q4_0" and N == 1:
                    r = head
                else:
                    r, _, _ = qmatvec_case(H, synth, timer, t, K, M, N, s, w)
                extra["qmatvec"][f"{name} N={N}"] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}
        # skinny GEMM at the top of the fused range (one pass over W per 32 columns)
        r, _, _ = qmatvec_case(H, synth, timer, H.TYPE_Q4_0, K, M, 64, s, w)
        extra["qmatvec"]["q4_0 N=64"] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}
        # configuration 0's product: Q8_0 W[4096,4096] times x with 8 columns, fused
        r, _, _ = qmatvec_case(H, synth, timer, H.TYPE_Q8_0, 4096, 4096, 8, s, w, cfg=0)
        extra["qmatvec_cfg0_q8_0_4096x4096_n8"] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}
        # configuration 0 as the reference runs it: the F32 weight of the warm start times 8 columns
        r = mul_mat_config0(H, synth, timer, 8, s, w)
        extra["mul_mat_cfg0_f32_4096x4096x8"] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}
        extra["dequant_4096x11008"] = {}
        for name, t in H.QUANT_TYPES.items():
            r = dequant_case(H, synth, timer, t, 4096 * 11008 // 32, s, w)
            extra["dequant_4096x11008"][name] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}
        extra["mul_mat_cfg3_linear_4096x4096x512"] = mul_mat_config3(H, synth, timer, max(10, s // 4), 3)
        extra["mul_mat_cfg4_batched_permuted"] = mul_mat_config4(H, synth, timer, max(10, s // 4), 3)
        extra["linear_step_cfg3_fwd_bwd"] = linear_step(H, synth, timer, max(10, s // 4), 3)
        extra["gguf_load_cfg0_hip_route"] = gguf_load_cfg0(H, synth)

    host = cpu_host_info()
    port = cpu_baseline(blk, x, K, M, args.cpu_budget / 2)
    cpu = cpu_baseline_reference(blk, x, K, M, args.cpu_budget)
    if cpu is None:
        cpu = port
    else:
        extra["cpu_baseline_port"] = port
    cpu["cpu_model"] = host["cpu_model"]
    extra["cpu_vs_gpu_speedup"] = head["GB/s"] / cpu["value"]
    extra["host"] = host
    if not args.headline_only:
        # the same path on every core this process may run on, outputs split over threads
        nt = max(1, host["cores_available"])
        extra["cpu_baseline_all_cores"] = cpu_baseline(blk, x, K, M, args.cpu_budget / 4, nt)
        extra["cpu_other_paths"] = cpu_other_paths(synth, args.cpu_budget / 5, nt)
        extra["cpu_other_paths"]["gguf_load_cfg0_reference_route"] = gguf_load_cfg0_reference_route(H, synth, 1)

    line = {
        "metric": METRIC,
        "value": round(head["GB/s"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded splitmix64: Q4_0 blocks with d~U[2e-4,1e-3] fp16, nibbles U{0..15}; x~N(0,1))",
        "config": {"workload": "cfg2 decode: fused Q4_0 dequant-matvec, W[K=4096,M=14336] x F32 x[4096,1]",
                   "K": K, "M": M, "N": 1, "rotating_sets": head["sets"], "timing": head["timing"],
                   "x_arithmetic": "x in 24-bit block fixed point (a power-of-two scale per 32-element block), "
                                   "exact int32 digit dot products against the quants, f32 block scaling and "
                                   "accumulation",
                   "headline_stat": f"median of {len(reps)} timed runs of {args.steps} launches each, "
                                    "each enqueued behind an untimed graph replay of the same steps "
                                    f"({head['timing']})",
                   "replays_us": reps, "spread_us": round(max(reps) - min(reps), 3),
                   "replays_other_method_us": head["replays_other_method_us"],
                   "replays_from_idle_graph_us": head["replays_with_submission_us"],
                   "wall_s_headline": round(wall, 3)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
