#!/usr/bin/env python3
"""Benchmark of the MI355X tensor-module backend (one GPU).

Headline (`value`): fp32 GEMM C = A.B at M=N=K=4096, GFLOP/s of the whole
timed loop, inputs resident in HBM.  The `suite` object carries the other
benchmark workloads measured the same way (MLP forward, GEMM sweep, conv2d,
small CNN, elementwise and softmax bandwidth), each with its own roofline
entry.

Timing: W warmup steps, device sync, then exactly K steps between two HIP
events on the library stream (the stream every kernel is launched on),
device sync after.  Suite entries warm up for at least 50 ms (the GPU clock
ramps after idle time) and time at least 10 ms of work (microsecond kernels
would otherwise measure host launch jitter).  The suite runs first, so the
headline's W + K steps run on a GPU that has been under load for seconds, at
the clock it holds under sustained work (with --no-suite they follow the
idle host setup instead); the CPU baseline runs last.
`roofline.achieved` = algorithmic FLOP (or bytes) of the dominant kernel per
launch / its average launch time from those events.

The CPU baseline times the oracle (a loop-for-loop restatement of the
reference's CPU kernels, single thread) on a bounded row slab of the same
workload, on this host, in this run.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-suite]
       [--no-cpu] [--workload NAME] [--vendor]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from camel_amd import _hip as H  # noqa: E402
from camel_amd import datagen as D  # noqa: E402

P = C.c_void_p
METRIC = "fp32 GEMM/conv GFLOP/s + % MFMA peak; elementwise GB/s + % HBM peak, 1 GPU"
PEAK_MFMA_F32_TFLOPS = 157.3  # MI355X dense fp32 matrix, vendor figure
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E, vendor figure
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.txt")
COUNTER_FILE = os.path.join(ROOT, "profiles", "mfma_counters.txt")


def _counter_entry(key: str):
    """MFMA-pipe utilisation of a workload from profiles/mfma_counters.txt:
    sum SQ_VALU_MFMA_BUSY_CYCLES / (4 SIMDs x sum SQ_BUSY_CU_CYCLES) over the
    call's kernels, with provenance (commit, kernels), read by rocprofv3
    --pmc passes."""
    try:
        with open(COUNTER_FILE) as f:
            for line in f:
                if not line.startswith(key + ":"):
                    continue
                fields = line.split(":", 1)[1].split()
                src = {"file": "profiles/mfma_counters.txt",
                       "counters": "SQ_VALU_MFMA_BUSY_CYCLES, SQ_BUSY_CU_CYCLES"}
                for fld in fields[1:]:
                    if "=" in fld:
                        k, v = fld.split("=", 1)
                        if k in ("commit", "kernels"):
                            src[k] = v.split(";") if k == "kernels" else v
                return float(fields[0]), src
    except OSError:
        pass
    return None, None


def _traffic_entry(key: str):
    """(HBM bytes per call, provenance) from profiles/traffic.txt, measured with
    two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE); provenance names the
    commit the counters were read at and the kernels they cover."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if not line.startswith(key + ":"):
                    continue
                fields = line.split(":", 1)[1].split()
                src = {"file": "profiles/traffic.txt", "counters": "FETCH_SIZE, WRITE_SIZE"}
                for fld in fields[4:]:
                    if "=" in fld:
                        k, v = fld.split("=", 1)
                        src[k] = v.split(";") if k == "kernels" else v
                return float(fields[0]), src
    except OSError:
        pass
    return None, None


def _progress(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# Suite entries (not the headline, which runs exactly --warmup / --steps) warm
# up for at least this long, so the GPU clock has ramped after idle host work,
# and time at least this much GPU work, so launches of microsecond kernels do
# not measure host issue jitter.
SUITE_MIN_WARM_S = 0.05
SUITE_MIN_TIMED_S = 0.01
_suite_mode = False


def _time_loop(fn, steps: int, warmup: int):
    adaptive = _suite_mode
    t0 = time.perf_counter()
    n_warm = 0
    while n_warm < warmup or (adaptive and time.perf_counter() - t0 < SUITE_MIN_WARM_S):
        fn()
        n_warm += 1
        if adaptive and n_warm % 8 == 0:
            H.sync()
    H.sync()
    if adaptive:
        per_step = (time.perf_counter() - t0) / max(1, n_warm)
        steps = max(steps, int(SUITE_MIN_TIMED_S / max(per_step, 1e-6)) + 1)
    t = H.Timer()
    wall0 = time.perf_counter()
    t.begin()
    for _ in range(steps):
        fn()
    ms = t.end()
    H.sync()
    wall = time.perf_counter() - wall0
    return ms / steps, wall


def sgemm_call(da, db, dc, M, N, K, dbias=None, flags=0):
    return lambda: H.call("camel_hip_sgemm", P(da.ptr), P(db.ptr), P(dc.ptr), M, N, K,
                          P(dbias.ptr) if dbias is not None else None, flags)


def _with_traffic(line: dict, key):
    if key is not None:
        nbytes, src = _traffic_entry(key)
        line["traffic"] = nbytes
        if src is not None:
            line["traffic_source"] = src
        if line["bound"] == "mfma":
            busy, src = _counter_entry(key)
            if busy is not None:
                line["mfma_busy"] = busy
                line["mfma_busy_source"] = src
    return line


def roofline_mfma(flop: float, ms: float, traffic_key=None):
    ach = flop / (ms * 1e-3) / 1e12
    return _with_traffic({"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_MFMA_F32_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(ach / PEAK_MFMA_F32_TFLOPS, 4),
                          "traffic": None}, traffic_key)


def roofline_hbm(nbytes: float, ms: float, traffic_key=None):
    ach = nbytes / (ms * 1e-3) / 1e9
    return _with_traffic({"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS,
                          "unit": "GB/s", "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": None},
                         traffic_key)


# ---------------------------------------------------------------- workloads

def wl_gemm(n_m, n_n, n_k, steps, warmup, seed=D.SEED_GEMM):
    a = D.uniform(seed + n_m, (n_m, n_k), -1.0, 1.0)
    b = D.uniform(seed + n_m + 1, (n_k, n_n), -1.0, 1.0)
    da, db, dc = H.to_device(a), H.to_device(b), H.DeviceBuffer(n_m * n_n * 4)
    ms, wall = _time_loop(sgemm_call(da, db, dc, n_m, n_n, n_k), steps, warmup)
    flop = 2.0 * n_m * n_n * n_k
    return {"ms": ms, "wall_s": wall, "flop": flop, "value": flop / (ms * 1e-3) / 1e9,
            "unit": "GFLOP/s", "a": a, "b": b}


def wl_gemm_host(n, steps, warmup, seed=D.SEED_GEMM):
    """The headline GEMM with host operands: H2D of A and B, the GEMM, D2H of C
    per call (pageable host memory, synchronous copies), timed by wall clock.
    The PCIe-inclusive rate of a caller that hands host buffers per call."""
    a = D.uniform(seed + n, (n, n), -1.0, 1.0)
    b = D.uniform(seed + n + 1, (n, n), -1.0, 1.0)
    da, db, dc = H.DeviceBuffer(a.nbytes), H.DeviceBuffer(b.nbytes), H.DeviceBuffer(a.nbytes)
    c = np.empty((n, n), np.float32)

    def step():
        da.upload(a)
        db.upload(b)
        sgemm_call(da, db, dc, n, n, n)()
        H.call("camel_hip_d2h", P(c.ctypes.data), P(dc.ptr), C.c_size_t(c.nbytes))

    for _ in range(warmup):
        step()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    return {"ms": ms, "flop": 2.0 * n ** 3, "bytes_pcie": 3.0 * a.nbytes}


def wl_skinny(steps, warmup):
    # M=16, N=K=4096: B (64 MiB) fits the 256 MiB MALL, so rotate 6 buffer sets
    # (>= 400 MiB) to measure HBM rather than cache.
    sets = []
    for s in range(6):
        a = D.uniform(D.SEED_GEMM + 16 + 10 * s, (16, 4096), -1.0, 1.0)
        b = D.uniform(D.SEED_GEMM + 17 + 10 * s, (4096, 4096), -1.0, 1.0)
        sets.append((H.to_device(a), H.to_device(b), H.DeviceBuffer(16 * 4096 * 4)))
    it = [0]

    def step():
        da, db, dc = sets[it[0] % len(sets)]
        it[0] += 1
        sgemm_call(da, db, dc, 16, 4096, 4096)()

    ms, wall = _time_loop(step, steps, warmup)
    flop = 2.0 * 16 * 4096 * 4096
    nbytes = 4.0 * (16 * 4096 + 4096 * 4096 + 16 * 4096)
    return {"ms": ms, "flop": flop, "bytes": nbytes}


def wl_mlp(steps, warmup, fused=True):
    """MLP forward: dense 784->1024->1024->10 (+relu) then row softmax, batch 1024.
    fused: the calls the operator layer's chain makes for it (its plan is
    dense_relu, then dense_relu+dense+softmax as camel_hip_dense_head);
    otherwise one call per layer and the softmax kernel."""
    B = 1024
    dims = [784, 1024, 1024, 10]
    x = D.uniform(D.SEED_MLP, (B, dims[0]), 0.0, 1.0)
    ws = [D.normal(D.SEED_MLP + 1 + i, (dims[i], dims[i + 1]), std=float(np.sqrt(1.0 / dims[i])))
          for i in range(3)]
    bs = [np.zeros(dims[i + 1], np.float32) for i in range(3)]
    dx = H.to_device(x)
    dws = [H.to_device(w) for w in ws]
    dbs = [H.to_device(b) for b in bs]
    acts = [H.DeviceBuffer(B * d * 4) for d in dims[1:]]
    dp = H.DeviceBuffer(B * 10 * 4)

    relu_bias = H.EPI_BIAS | H.EPI_RELU

    def step():
        if fused:
            sgemm_call(dx, dws[0], acts[0], B, dims[1], dims[0], dbs[0], relu_bias)()
            H.call("camel_hip_dense_head", P(acts[0].ptr), P(dws[1].ptr), P(dbs[1].ptr),
                   P(dws[2].ptr), P(dbs[2].ptr), P(dp.ptr), B, dims[1], dims[2], dims[3],
                   relu_bias, H.EPI_BIAS, 1)
            return
        src = dx
        for i in range(3):
            flags = H.EPI_BIAS | (H.EPI_RELU if i < 2 else 0)
            sgemm_call(src, dws[i], acts[i], B, dims[i + 1], dims[i], dbs[i], flags)()
            src = acts[i]
        H.call("camel_hip_softmax_rows", P(acts[2].ptr), P(dp.ptr), B, 10)

    ms, wall = _time_loop(step, steps, warmup)
    flop = sum(2.0 * B * dims[i] * dims[i + 1] for i in range(3))
    return {"ms": ms, "flop": flop, "x": x, "ws": ws, "bs": bs, "dp": dp}


def wl_conv(steps, warmup):
    """conv2d 64x64x56x56 -> 128, 3x3, s1 p1, bias + relu."""
    x = D.normal(D.SEED_CONV_X, (64, 64, 56, 56))
    w = D.normal(D.SEED_CONV_W, (128, 64, 3, 3), std=float(np.sqrt(2.0 / (9 * 64))))
    b = np.zeros(128, np.float32)
    dx, dw, db = H.to_device(x), H.to_device(w), H.to_device(b)
    dy = H.DeviceBuffer(64 * 128 * 56 * 56 * 4)
    call = lambda: H.call("camel_hip_conv2d", P(dx.ptr), P(dw.ptr), P(db.ptr), P(dy.ptr), 64, 64,
                          56, 56, 128, 3, 3, 1, 1, H.EPI_BIAS | H.EPI_RELU)
    ms, wall = _time_loop(call, steps, warmup)
    flop = 2.0 * (64 * 56 * 56) * 128 * (64 * 9)
    return {"ms": ms, "flop": flop, "x": x, "w": w, "b": b}


def wl_cnn(steps, warmup, fused=True):
    """Small CNN forward, batch 512 (valid 3x3 convs, 2x2 pool).
    fused: conv1 + relu + conv2 + relu + pool are one kernel
    (camel_hip_conv2d_pair_pool2: conv1's output stays in LDS; conv2's weights
    packed once at setup), and dense1 + relu + dense2 + softmax one head
    (camel_hip_dense_head: the dense2 kernel adds dense1's split-K partials);
    otherwise every layer is its own call."""
    B = 512
    x = D.uniform(D.SEED_CNN, (B, 1, 28, 28), 0.0, 1.0)
    w1 = D.normal(D.SEED_CNN + 1, (32, 1, 3, 3), std=float(np.sqrt(2.0 / 9)))
    w2 = D.normal(D.SEED_CNN + 2, (64, 32, 3, 3), std=float(np.sqrt(2.0 / 288)))
    w3 = D.normal(D.SEED_CNN + 3, (9216, 128), std=float(np.sqrt(2.0 / 9216)))
    w4 = D.normal(D.SEED_CNN + 4, (128, 10), std=float(np.sqrt(2.0 / 128)))
    z = lambda n: H.to_device(np.zeros(n, np.float32))
    dx, d1, d2, d3, d4 = (H.to_device(t) for t in (x, w1, w2, w3, w4))
    b1, b2, b3, b4 = z(32), z(64), z(128), z(10)
    a1 = H.DeviceBuffer(B * 32 * 26 * 26 * 4)
    a2 = H.DeviceBuffer(B * 64 * 24 * 24 * 4)
    a3 = H.DeviceBuffer(B * 64 * 12 * 12 * 4)
    a4 = H.DeviceBuffer(B * 128 * 4)
    a5 = H.DeviceBuffer(B * 10 * 4)
    dp = H.DeviceBuffer(B * 10 * 4)
    EPI = H.EPI_BIAS | H.EPI_RELU
    # conv2's weights packed once for the implicit GEMM (weight pre-packing)
    d2p = H.DeviceBuffer(64 * 32 * 9 * 4)
    H.call("camel_hip_conv2d_pack_weights", P(d2.ptr), P(d2p.ptr), 64, 32, 3, 3)

    def step():
        if fused:
            H.call("camel_hip_conv2d_pair_pool2", P(dx.ptr), P(d1.ptr), P(b1.ptr), P(d2p.ptr),
                   P(b2.ptr), P(a3.ptr), B, 28, 28, 32, 64, EPI, EPI | H.CONV_W_PACKED)
            H.call("camel_hip_dense_head", P(a3.ptr), P(d3.ptr), P(b3.ptr), P(d4.ptr), P(b4.ptr),
                   P(dp.ptr), B, 9216, 128, 10, EPI, H.EPI_BIAS, 1)
            return
        H.call("camel_hip_conv2d", P(dx.ptr), P(d1.ptr), P(b1.ptr), P(a1.ptr), B, 1, 28, 28, 32, 3, 3, 1, 0, EPI)
        H.call("camel_hip_conv2d", P(a1.ptr), P(d2.ptr), P(b2.ptr), P(a2.ptr), B, 32, 26, 26, 64, 3, 3, 1, 0, EPI)
        H.call("camel_hip_maxpool2d", P(a2.ptr), P(a3.ptr), B, 64, 24, 24, 2, 2, 2)
        sgemm_call(a3, d3, a4, B, 128, 9216, b3, EPI)()
        sgemm_call(a4, d4, a5, B, 10, 128, b4, H.EPI_BIAS)()
        H.call("camel_hip_softmax_rows", P(a5.ptr), P(dp.ptr), B, 10)

    ms, wall = _time_loop(step, steps, warmup)
    flop = 2.0 * B * (26 * 26 * 32 * 9 + 24 * 24 * 64 * 288 + 9216 * 128 + 128 * 10)
    return {"ms": ms, "flop": flop}


def _big_input(seed, n, lo=-1.0, hi=1.0):
    # 1 GiB buffers: generate 16 Mi seeded values and tile them (bandwidth is
    # independent of the values; the buffers still exceed the 256 MiB MALL).
    base = D.uniform(seed, (1 << 24,), lo, hi)
    return np.tile(base, n // base.size)


def wl_eltwise(steps, warmup):
    n = 1 << 28
    a = _big_input(D.SEED_ELT, n)
    b = _big_input(D.SEED_ELT + 1, n)
    da, db, dc = H.to_device(a), H.to_device(b), H.DeviceBuffer(n * 4)
    del a, b
    out = {}
    for name, op in (("add", H.OP_ADD), ("mul", H.OP_MUL)):
        call = lambda op=op: H.call("camel_hip_binary", op, H.DT_F32, P(da.ptr), H.DT_F32, P(db.ptr),
                                    H.DT_F32, P(dc.ptr), n)
        ms, _ = _time_loop(call, steps, warmup)
        out[name] = {"ms": ms, "bytes": 12.0 * n}
    call = lambda: H.call("camel_hip_relu", P(da.ptr), P(dc.ptr), n)
    ms, _ = _time_loop(call, steps, warmup)
    out["relu"] = {"ms": ms, "bytes": 8.0 * n}
    return out


def wl_copy(steps, warmup):
    """1 GiB device-to-device copy: the known-size transfer that calibrates the
    FETCH_SIZE / WRITE_SIZE counters (reads 1 GiB, writes 1 GiB per launch)."""
    n = 1 << 28
    da, db = H.DeviceBuffer(n * 4), H.DeviceBuffer(n * 4)
    H.call("camel_hip_fill", H.DT_F32, P(da.ptr), n, 1.0)
    call = lambda: H.call("camel_hip_d2d", P(db.ptr), P(da.ptr), C.c_size_t(n * 4))
    ms, _ = _time_loop(call, steps, warmup)
    return {"ms": ms, "bytes": 8.0 * n}


def wl_softmax(steps, warmup):
    rows, cols = 262144, 1024
    base = D.normal(D.SEED_ELT + 2, (1 << 24,))
    x = np.tile(base, rows * cols // base.size)
    dx, dy = H.to_device(x), H.DeviceBuffer(rows * cols * 4)
    del x
    call = lambda: H.call("camel_hip_softmax_rows", P(dx.ptr), P(dy.ptr), rows, cols)
    ms, _ = _time_loop(call, steps, warmup)
    return {"ms": ms, "bytes": 8.0 * rows * cols}


# ------------------------------------------------------------- CPU baseline
#
# The oracle (a loop-for-loop restatement of the reference's CPU kernels:
# ijk matmul with fp64 accumulation and per-element dtype dispatch,
# operators.cpp:757-766; tensorBinary, runtime.cpp:775-793; the mnist.cml
# softmax composition; conv2d as direct loops in matmul order), single
# thread, on this host, in this run -- a reported baseline per suite row,
# full where it finishes in seconds, otherwise a labelled slab of the same
# workload whose cost per row / image / element is the same as the whole's.

def _oracle():
    from oracle import ffi as O  # the CPU baseline leg is bench.py's only user of the oracle
    return O


def _cpu_line(value: float, unit: str, sample: str, spent: float) -> dict:
    n = os.cpu_count()
    return {"value": round(value, 4), "unit": unit, "cores": 1, "nproc": n, "kind": "port",
            "sample": f"{sample}; {spent:.2f} s on 1 of {n} host cores"}


def _timed(fn):
    t0 = time.perf_counter()
    out = fn()
    return out, time.perf_counter() - t0


def cpu_baseline_gemm(a, b, budget_s: float = 12.0, max_rows: int | None = None):
    """Oracle ijk matmul (reference operators.cpp:757-766) on a row slab, 1 thread:
    as many leading rows as fit the budget (all of them for small problems)."""
    O = _oracle()
    M, K = a.shape
    N = b.shape[1]
    _, per_row = _timed(lambda: O.matmul_rows(a, b, 0, 1))
    rows = max(1, min(M, int(budget_s / max(per_row, 1e-6)), max_rows or M))
    _, spent = _timed(lambda: O.matmul_rows(a, b, 0, rows))
    what = "all rows" if rows == M else f"rows 0-{rows - 1} (slab, extrapolated per row)"
    return _cpu_line(2.0 * rows * N * K / spent / 1e9, "GFLOP/s",
                     f"{what} of the {M}x{N}x{K} fp32 matmul through the oracle (ijk, fp64 "
                     f"accumulate, per-element dtype dispatch)", spent)


def cpu_baseline_mlp(x, ws, bs):
    """The whole MLP forward (config 2) through the oracle: three dense layers
    (matmul + bias, relu as x*(x>0)) and the mnist.cml softmax composition."""
    O = _oracle()

    def run():
        h = x
        for i in range(3):
            h = O.dense(h, ws[i], bs[i], i < 2)
        return O.softmax_rows(h)

    _, spent = _timed(run)
    flop = sum(2.0 * x.shape[0] * w.shape[0] * w.shape[1] for w in ws)
    return _cpu_line(flop / spent / 1e9, "GFLOP/s",
                     f"full MLP forward, batch {x.shape[0]} (784->1024->1024->10 + softmax)", spent)


def cpu_baseline_conv(x, w, b, images: int = 1):
    """conv2d config 4 through the oracle's direct loops on an image slab."""
    O = _oracle()
    _, spent = _timed(lambda: O.conv2d_images(x, w, b, True, 0, images, 1, 1))
    N, Cin, H_, W_ = x.shape
    Co = w.shape[0]
    flop = 2.0 * images * H_ * W_ * Co * Cin * 9
    return _cpu_line(flop / spent / 1e9, "GFLOP/s",
                     f"images 0-{images - 1} of {N} (slab, extrapolated per image) of the "
                     f"{N}x{Cin}x{H_}x{W_} -> {Co} 3x3 conv + bias + relu", spent)


def cpu_baseline_cnn(images: int = 32):
    """The CNN forward (config 5) through the oracle on an image slab: conv,
    conv, 2x2 pool, dense, dense, softmax, per image as the batch would run."""
    O = _oracle()
    x = D.uniform(D.SEED_CNN, (images, 1, 28, 28), 0.0, 1.0)
    w1 = D.normal(D.SEED_CNN + 1, (32, 1, 3, 3), std=float(np.sqrt(2.0 / 9)))
    w2 = D.normal(D.SEED_CNN + 2, (64, 32, 3, 3), std=float(np.sqrt(2.0 / 288)))
    w3 = D.normal(D.SEED_CNN + 3, (9216, 128), std=float(np.sqrt(2.0 / 9216)))
    w4 = D.normal(D.SEED_CNN + 4, (128, 10), std=float(np.sqrt(2.0 / 128)))
    z = lambda n: np.zeros(n, np.float32)

    def run():
        h = O.conv2d(x, w1, z(32), True)
        h = O.conv2d(h, w2, z(64), True)
        h = O.maxpool2d(h, 2, 2).reshape(images, 9216)
        h = O.dense(h, w3, z(128), True)
        return O.softmax_rows(O.dense(h, w4, z(10), False))

    _, spent = _timed(run)
    flop = 2.0 * images * (26 * 26 * 32 * 9 + 24 * 24 * 64 * 288 + 9216 * 128 + 128 * 10)
    return _cpu_line(flop / spent / 1e9, "GFLOP/s",
                     f"images 0-{images - 1} of 512 (slab, extrapolated per image) of the CNN "
                     f"forward", spent)


def cpu_baseline_bandwidth(kind: str, n: int = 1 << 24):
    """Elementwise / softmax through the oracle on the first n elements of the
    same seeded inputs, in the suite line's unit (GB/s of algorithmic bytes)."""
    O = _oracle()
    if kind == "softmax":
        x = D.normal(D.SEED_ELT + 2, (n // 1024, 1024))
        _, spent = _timed(lambda: O.softmax_rows(x))
        return _cpu_line(8.0 * n / spent / 1e9, "GB/s",
                         f"rows 0-{n // 1024 - 1} of 262144 (slab) of the 1024-column row softmax "
                         f"(mnist.cml composition)", spent)
    a = D.uniform(D.SEED_ELT, (n,), -1.0, 1.0)
    if kind == "relu":
        _, spent = _timed(lambda: O.relu(a))
        nbytes = 8.0 * n
    else:
        b = D.uniform(D.SEED_ELT + 1, (n,), -1.0, 1.0)
        op = O.ADD if kind == "add" else O.MUL
        _, spent = _timed(lambda: O.binary(op, a, b))
        nbytes = 12.0 * n
    return _cpu_line(nbytes / spent / 1e9, "GB/s",
                     f"first {n} of 2^28 elements (slab) of {kind}", spent)


# ------------------------------------------------------------ vendor line

def vendor_suite() -> dict:
    """The same workloads through PyTorch-ROCm's vendor libraries on this GPU
    (hipBLASLt / rocBLAS GEMMs, MIOpen convolutions, torch's elementwise and
    softmax kernels), fp32 with TF32-style shortcuts off, timed with events on
    torch's current stream after >= 50 ms of warm-up.  A reference point for
    the kernels of this library, not part of its product path."""
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    dev = torch.device("cuda", 0)
    dt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    def time_us(fn, iters):
        t0 = time.perf_counter()
        n = 0
        while n < 5 or time.perf_counter() - t0 < SUITE_MIN_WARM_S:
            fn()
            n += 1
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(iters):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / iters * 1e3

    out = {}
    for n in (256, 1024, 2048, 4096, 8192):
        a = dt(D.uniform(D.SEED_GEMM + n, (n, n), -1.0, 1.0))
        b = dt(D.uniform(D.SEED_GEMM + n + 1, (n, n), -1.0, 1.0))
        c = torch.empty(n, n, device=dev)
        us = time_us(lambda: torch.matmul(a, b, out=c), 10 if n >= 4096 else 200)
        key = "matmul_256" if n == 256 else f"sgemm_{n}"
        out[key] = {"us": round(us, 2), "TFLOP/s": round(2.0 * n ** 3 / us / 1e6, 2)}
        del a, b, c
    a = dt(D.uniform(D.SEED_GEMM + 16, (16, 4096), -1.0, 1.0))
    bs = [dt(D.uniform(D.SEED_GEMM + 17 + 10 * s, (4096, 4096), -1.0, 1.0)) for s in range(6)]
    c = torch.empty(16, 4096, device=dev)
    it = [0]

    def skinny():
        torch.matmul(a, bs[it[0] % 6], out=c)
        it[0] += 1
    us = time_us(skinny, 600)
    out["sgemm_16x4096x4096"] = {"us": round(us, 2),
                                 "TB/s": round(4.0 * (2 * 16 * 4096 + 4096 * 4096) / us / 1e6, 3)}
    del a, bs, c
    dims = [784, 1024, 1024, 10]
    x = dt(D.uniform(D.SEED_MLP, (1024, 784), 0.0, 1.0))
    ws = [dt(D.normal(D.SEED_MLP + 1 + i, (dims[i], dims[i + 1]), std=float(np.sqrt(1.0 / dims[i]))))
          for i in range(3)]
    bz = [torch.zeros(d, device=dev) for d in dims[1:]]

    def mlp():
        h = torch.relu(torch.addmm(bz[0], x, ws[0]))
        h = torch.relu(torch.addmm(bz[1], h, ws[1]))
        return torch.softmax(torch.addmm(bz[2], h, ws[2]), dim=1)
    us = time_us(mlp, 300)
    out["mlp_forward"] = {"us": round(us, 2), "TFLOP/s": round(3.813e9 / us / 1e6, 2)}
    xc = dt(D.normal(D.SEED_CONV_X, (64, 64, 56, 56)))
    wc = dt(D.normal(D.SEED_CONV_W, (128, 64, 3, 3), std=float(np.sqrt(2.0 / 576))))
    bc = torch.zeros(128, device=dev)
    us = time_us(lambda: torch.relu(torch.nn.functional.conv2d(xc, wc, bc, padding=1)), 30)
    out["conv2d_3x3"] = {"us": round(us, 2), "TFLOP/s": round(29.596e9 / us / 1e6, 2)}
    del xc, wc
    xi = dt(D.uniform(D.SEED_CNN, (512, 1, 28, 28), 0.0, 1.0))
    w1 = dt(D.normal(D.SEED_CNN + 1, (32, 1, 3, 3), std=float(np.sqrt(2.0 / 9))))
    w2 = dt(D.normal(D.SEED_CNN + 2, (64, 32, 3, 3), std=float(np.sqrt(2.0 / 288))))
    w3 = dt(D.normal(D.SEED_CNN + 3, (9216, 128), std=float(np.sqrt(2.0 / 9216))))
    w4 = dt(D.normal(D.SEED_CNN + 4, (128, 10), std=float(np.sqrt(2.0 / 128))))
    z = {k: torch.zeros(k, device=dev) for k in (32, 64, 128, 10)}

    def cnn():
        h = torch.relu(torch.nn.functional.conv2d(xi, w1, z[32]))
        h = torch.relu(torch.nn.functional.conv2d(h, w2, z[64]))
        h = torch.nn.functional.max_pool2d(h, 2).reshape(512, 9216)
        h = torch.relu(torch.addmm(z[128], h, w3))
        return torch.softmax(torch.addmm(z[10], h, w4), dim=1)
    us = time_us(cnn, 50)
    out["cnn_forward"] = {"us": round(us, 2), "TFLOP/s": round(12.28e9 / us / 1e6, 2)}
    n = 1 << 28
    ea = torch.rand(n, device=dev) * 2 - 1
    eb = torch.rand(n, device=dev) * 2 - 1
    ec = torch.empty(n, device=dev)
    for name, fn, nb in (("eltwise_add", lambda: torch.add(ea, eb, out=ec), 12.0),
                         ("eltwise_mul", lambda: torch.mul(ea, eb, out=ec), 12.0),
                         ("eltwise_relu", lambda: torch.clamp_min(ea, 0.0, out=ec), 8.0)):
        us = time_us(fn, 20)
        out[name] = {"us": round(us, 2), "TB/s": round(nb * n / us / 1e6, 3)}
    del ea, eb, ec
    sx = torch.randn(262144, 1024, device=dev)
    us = time_us(lambda: torch.softmax(sx, dim=1), 20)
    out["softmax_262144x1024"] = {"us": round(us, 2), "TB/s": round(8.0 * 262144 * 1024 / us / 1e6, 3)}
    return {"vendor": out, "torch": torch.__version__}


# ------------------------------------------------------------------- main

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--no-suite", action="store_true", help="headline GEMM only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--unfused", action="store_true",
                    help="mlp / cnn workloads: one call per layer (no fused kernels)")
    ap.add_argument("--vendor", action="store_true",
                    help="time the same workloads through PyTorch-ROCm's vendor libraries instead")
    ap.add_argument("--workload", default="gemm4096",
                    choices=["gemm4096", "gemm1024", "gemm2048", "gemm8192", "mlp", "conv2d",
                             "cnn", "eltwise", "softmax", "skinny", "copy"])
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only; multi-GPU runs are not supported "
              "(use --gpus 1)", file=sys.stderr)
        return 2

    if args.vendor:
        print(json.dumps(vendor_suite()))
        return 0

    H.call("camel_hip_init", 0)
    steps, warmup = args.steps, args.warmup

    if args.workload in ("gemm1024", "gemm2048", "gemm8192"):
        # one square GEMM alone (profiling)
        n = int(args.workload[4:])
        r = wl_gemm(n, n, n, steps, warmup)
        print(json.dumps({"workload": args.workload, "ms": r["ms"], "value": r["value"],
                          "unit": "GFLOP/s"}))
        return 0

    if args.workload != "gemm4096":
        # single-workload mode (used for profiling one kernel at a time)
        fn = {"mlp": wl_mlp, "conv2d": wl_conv, "cnn": wl_cnn, "eltwise": wl_eltwise,
              "softmax": wl_softmax, "skinny": wl_skinny, "copy": wl_copy}[args.workload]
        res = fn(steps, warmup, fused=False) if args.unfused and args.workload in ("mlp", "cnn") \
            else fn(steps, warmup)
        keep = {k: v for k, v in res.items() if isinstance(v, (int, float, dict))}
        print(json.dumps({"workload": args.workload, **keep}))
        return 0

    if not args.no_suite:
        global _suite_mode
        _suite_mode = True
        suite = {}
        # CPU baselines of the suite rows run after all GPU work (see below).
        cpu_jobs = []
        s_steps, s_warm = max(5, steps // 5), 2
        for n in (1024, 2048, 8192):
            r = wl_gemm(n, n, n, s_steps if n < 8192 else 5, s_warm)
            suite[f"sgemm_{n}"] = {"value": round(r["value"], 1), "unit": "GFLOP/s",
                                   "ms": round(r["ms"], 4),
                                   "roofline": roofline_mfma(r["flop"], r["ms"], f"sgemm_{n}")}
            cpu_jobs.append((f"sgemm_{n}", lambda a=r["a"], b=r["b"], n=n: cpu_baseline_gemm(
                a, b, budget_s=4.0 if n == 1024 else 2.0)))
        r = wl_gemm(256, 256, 256, s_steps, s_warm)
        suite["matmul_256"] = {"value": round(r["value"], 1), "unit": "GFLOP/s",
                               "ms": round(r["ms"], 4),
                               "note": "BASELINE config 1 (plumbing anchor): launch-latency bound",
                               "roofline": roofline_mfma(r["flop"], r["ms"])}
        cpu_jobs.append(("matmul_256", lambda a=r["a"], b=r["b"]: cpu_baseline_gemm(a, b)))
        r = wl_gemm_host(4096, 5, 2)
        suite["sgemm_4096_host_operands"] = {
            "value": round(r["flop"] / (r["ms"] * 1e-3) / 1e9, 1), "unit": "GFLOP/s",
            "ms": round(r["ms"], 4), "pcie_bytes": r["bytes_pcie"],
            "note": "H2D A, B + GEMM + D2H C per call; PCIe-inclusive, not the headline value",
            "roofline": roofline_mfma(r["flop"], r["ms"])}
        r = wl_skinny(s_steps * 4, s_warm)
        suite["sgemm_16x4096x4096"] = {
            "value": round(r["flop"] / (r["ms"] * 1e-3) / 1e9, 1), "unit": "GFLOP/s",
            "ms": round(r["ms"], 4),
            "roofline": roofline_hbm(r["bytes"], r["ms"], "skinny")}
        cpu_jobs.append(("sgemm_16x4096x4096", lambda: cpu_baseline_gemm(
            D.uniform(D.SEED_GEMM + 16, (16, 4096), -1.0, 1.0),
            D.uniform(D.SEED_GEMM + 17, (4096, 4096), -1.0, 1.0))))
        r = wl_mlp(s_steps * 2, s_warm)
        suite["mlp_forward"] = {"value": round(r["flop"] / (r["ms"] * 1e-3) / 1e9, 1),
                                "unit": "GFLOP/s", "ms": round(r["ms"], 4),
                                "roofline": roofline_mfma(r["flop"], r["ms"], "mlp")}
        cpu_jobs.append(("mlp_forward", lambda x=r["x"], ws=r["ws"], bs=r["bs"]:
                         cpu_baseline_mlp(x, ws, bs)))
        r = wl_mlp(s_steps * 2, s_warm, fused=False)
        suite["mlp_forward_unfused"] = {"value": round(r["flop"] / (r["ms"] * 1e-3) / 1e9, 1),
                                        "unit": "GFLOP/s", "ms": round(r["ms"], 4),
                                        "note": "one call per layer, no fused kernels",
                                        "roofline": roofline_mfma(r["flop"], r["ms"])}
        r = wl_conv(s_steps, s_warm)
        suite["conv2d_3x3"] = {"value": round(r["flop"] / (r["ms"] * 1e-3) / 1e9, 1),
                               "unit": "GFLOP/s", "ms": round(r["ms"], 4),
                               "roofline": roofline_mfma(r["flop"], r["ms"], "conv2d")}
        cpu_jobs.append(("conv2d_3x3", lambda x=r["x"], w=r["w"], b=r["b"]:
                         cpu_baseline_conv(x, w, b, images=2)))
        r = wl_cnn(s_steps, s_warm)
        suite["cnn_forward"] = {"value": round(r["flop"] / (r["ms"] * 1e-3) / 1e9, 1),
                                "unit": "GFLOP/s", "ms": round(r["ms"], 4),
                                "roofline": roofline_mfma(r["flop"], r["ms"], "cnn")}
        cpu_jobs.append(("cnn_forward", lambda: cpu_baseline_cnn(images=32)))
        r = wl_cnn(s_steps, s_warm, fused=False)
        suite["cnn_forward_unfused"] = {"value": round(r["flop"] / (r["ms"] * 1e-3) / 1e9, 1),
                                        "unit": "GFLOP/s", "ms": round(r["ms"], 4),
                                        "note": "one call per layer, no fused kernels",
                                        "roofline": roofline_mfma(r["flop"], r["ms"])}
        e = wl_eltwise(s_steps, s_warm)
        for name, r in e.items():
            suite[f"eltwise_{name}"] = {"value": round(r["bytes"] / (r["ms"] * 1e-3) / 1e9, 1),
                                        "unit": "GB/s", "ms": round(r["ms"], 4),
                                        "roofline": roofline_hbm(r["bytes"], r["ms"],
                                                                 f"eltwise_{name}")}
            cpu_jobs.append((f"eltwise_{name}", lambda name=name: cpu_baseline_bandwidth(name)))
        r = wl_softmax(s_steps, s_warm)
        suite["softmax_262144x1024"] = {"value": round(r["bytes"] / (r["ms"] * 1e-3) / 1e9, 1),
                                        "unit": "GB/s", "ms": round(r["ms"], 4),
                                        "roofline": roofline_hbm(r["bytes"], r["ms"],
                                                                 "softmax")}
        cpu_jobs.append(("softmax_262144x1024", lambda: cpu_baseline_bandwidth("softmax")))
        for k, v in suite.items():
            _progress(f"{k}: {v['value']} {v['unit']} ({100 * v['roofline']['frac']:.1f}% of peak)")
        _suite_mode = False

    # The headline: exactly W warmup steps and K timed steps, after the suite.
    g = wl_gemm(4096, 4096, 4096, steps, warmup)
    _progress(f"sgemm 4096^3: {g['ms']:.4f} ms/step, {g['value']:.0f} GFLOP/s")
    line = {
        "metric": METRIC,
        "value": round(g["value"], 1),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(g["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded SplitMix64 U(-1,1), generated on host, resident in HBM)",
        "config": {"workload": "sgemm M=N=K=4096 (BASELINE config 3)", "M": 4096, "N": 4096,
                   "K": 4096, "layout": "row-major contiguous", "parallelism": "single GPU"},
        "roofline": roofline_mfma(g["flop"], g["ms"], "sgemm_4096"),
    }
    if not args.no_suite:
        line["suite"] = suite

    # Last, so the host-only baseline does not leave the GPU idle (and its
    # clock low) before any GPU timing.
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_gemm(g["a"], g["b"])
        _progress(f"cpu baseline: {line['cpu_baseline']['value']} GFLOP/s")
        if not args.no_suite:
            for key, job in cpu_jobs:
                line["suite"][key]["cpu_baseline"] = job()
                _progress(f"cpu baseline {key}: {line['suite'][key]['cpu_baseline']['value']} "
                          f"{line['suite'][key]['cpu_baseline']['unit']}")
    del g

    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
