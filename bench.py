#!/usr/bin/env python3
"""Benchmark of the MI355X fp32 GEMM path (one JSON line on stdout).

Headline (BASELINE.json metric): fp32 GEMM TFLOP/s at M = N = K = 4096,
row-major NN, A and B ~ N(0, 1), as a fraction of the MI355X fp32-MFMA peak.
A "step" is one GEMM launch over the resident operands.  The 784-256-10 MLP
training step rate is reported beside it.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--sweep FILE]

Timing: W untimed launches, then K launches bracketed by
torch.cuda.synchronize() with HIP events recorded on the stream the kernels
are launched on (torch's current stream, whose handle is passed to the C-ABI).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix peak (256 CU x 256 FLOP/clk x 2.4 GHz)
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "sgemm_nn_4096_traffic.txt")

# --profile-mode workloads (fast_dl_amd/profiling.py): name -> (M, N, K, transB,
# batch, epilogue, rotate), or "mlp" / "idx" for the MLP step and the IDX gather.
# "headline" is the bench line's own GEMM (M = N = K = --size).
from fast_dl_amd.profiling import CONFIGS as _PROFILE_WORKLOADS  # noqa: E402

PROFILE_CONFIGS = {name: (None if name == "headline" else
                          (w.kind if w.shape is None else w.shape))
                   for name, w in _PROFILE_WORKLOADS.items()}
CLOCK_WARM = True  # --no-clock-warm turns warm_clock off (counter runs)


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-mlp", action="store_true", help="skip the MLP step rate")
    ap.add_argument("--sweep", default=None, help="write every BASELINE config's timing here")
    ap.add_argument("--profile-mode", action="store_true",
                    help="only the headline launches (for rocprofv3 runs)")
    ap.add_argument("--profile-vendor", action="store_true",
                    help="with --profile-mode: launch the same workload through PyTorch "
                         "(vendor BLAS; eager autograd step for c2_mlp) instead, for "
                         "comparison traces")
    ap.add_argument("--profile-config", default="headline", choices=sorted(PROFILE_CONFIGS),
                    help="with --profile-mode: which BASELINE configuration to launch")
    ap.add_argument("--copy-calib", action="store_true",
                    help="with --profile-mode: also run known-size copy, sum and fill kernels "
                         "that scale the FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--no-clock-warm", action="store_true",
                    help="with --profile-mode: skip the clock warm-up bursts (counter runs, "
                         "which serialize every dispatch)")
    ap.add_argument("--collect-profiles", metavar="DIR", default=None,
                    help="run every rocprofv3 pass of fast_dl_amd/profiling.py into DIR (each "
                         "as a child process of this one, which does not touch the GPU)")
    ap.add_argument("--stages", default="trace,vendor,counters",
                    help="with --collect-profiles: comma-separated stages")
    ap.add_argument("--configs", default=None,
                    help="with --collect-profiles: comma-separated configurations (default all)")
    ap.add_argument("--summarize", metavar="DIR", default=None,
                    help="write the profiles/*.txt summaries from the rocprofv3 output in DIR")
    return ap.parse_args()


def read_traffic():
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, or None."""
    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", text, re.M)
    return float(m.group(1)) if m else None


def warm_clock(fn, stream, ms=50.0, min_launch_ms=0.015):
    """Back-to-back launches of ``fn`` for about ``ms`` of GPU time: the clock
    ramps over the first ~20 ms of work, and a short kernel's few warmup
    launches would otherwise be timed on a cold clock.  Launches shorter than
    ``min_launch_ms`` are left alone: their rows are bound by host launch
    cost, which a long burst of launches beforehand was measured to raise."""
    import torch

    if not CLOCK_WARM:
        return
    fn()  # one-time costs (code load, first-touch) stay out of the estimate
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(3):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    per = start.elapsed_time(end) / 3
    if per < min_launch_ms:
        return
    for _ in range(int(ms / per) + 1):
        fn()
    torch.cuda.synchronize()


def copy_calibration(torch):
    """Known-size kernels for scaling the FETCH_SIZE / WRITE_SIZE counters, three
    launches each: a 256 MiB device copy (256 MiB read, 256 MiB written), a
    64 MiB copy, a sum over 256 MiB (read only) and a 256 MiB fill (write only).
    Two sizes and three access mixes, so a scale taken from one of them is
    cross-checked by the others."""
    big = torch.ones(64 << 20, device="cuda")  # 256 MiB
    dst = torch.empty_like(big)
    small = torch.ones(16 << 20, device="cuda")  # 64 MiB
    sdst = torch.empty_like(small)
    out = torch.empty((), device="cuda")
    for _ in range(3):
        dst.copy_(big)
    for _ in range(3):
        sdst.copy_(small)
    for _ in range(3):
        torch.sum(big, dim=0, out=out)
    for _ in range(3):
        dst.fill_(2.0)
    torch.cuda.synchronize()


def time_launches(fn, steps, warmup, stream):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per launch


def launch_percentiles(fn, steps, stream):
    """Per-launch durations from events recorded between back-to-back launches on
    ``stream``: (median, p10, p90) in ms.  Each event pair brackets one launch."""
    import torch

    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    ev[0].record(stream)
    for i in range(steps):
        fn()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    d = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
    pick = lambda q: d[min(len(d) - 1, int(q * len(d)))]  # noqa: E731
    return pick(0.5), pick(0.1), pick(0.9)


def vendor_case(torch, M, N, K, ta=0, tb=0, batch=1, epi=0, seed=0, rotate=1):
    """The same GEMM through PyTorch (rocBLAS / hipBLASLt, full fp32), for comparison only.

    Bias+ReLU is ``addmm`` followed by an in-place ``relu_`` (two launches), which
    is how a caller without a fused epilogue would write it.
    """
    torch.backends.cuda.matmul.allow_tf32 = False
    gen = torch.Generator(device="cuda").manual_seed(seed)
    a_shape = (batch, K, M) if ta else (batch, M, K)
    b_shape = (batch, N, K) if tb else (batch, K, N)
    As = [torch.randn(a_shape, generator=gen, device="cuda") for _ in range(rotate)]
    Bs = [torch.randn(b_shape, generator=gen, device="cuda") for _ in range(rotate)]
    Cs = [torch.empty((batch, M, N), device="cuda") for _ in range(rotate)]
    bias = torch.randn((N,), generator=gen, device="cuda") * 0.1
    state = {"i": 0}

    def launch():
        i = state["i"]
        state["i"] = (i + 1) % rotate
        a = As[i].transpose(1, 2) if ta else As[i]
        b = Bs[i].transpose(1, 2) if tb else Bs[i]
        if batch == 1:
            if epi in (1, 2):
                torch.addmm(bias, a[0], b[0], out=Cs[i][0])
            else:
                torch.mm(a[0], b[0], out=Cs[i][0])
        else:
            torch.bmm(a, b, out=Cs[i])
        if epi == 2:
            Cs[i].relu_()

    return launch


def gemm_case(capi, torch, M, N, K, ta=0, tb=0, batch=1, epi=0, seed=0, rotate=1):
    """Resident operands and a launcher closure for one GEMM configuration.

    rotate > 1 cycles through that many copies of the operands so the working
    set exceeds the 256 MB Infinity Cache (HBM-bound shapes).  The call is the
    one the dl:: operations make: fdl_sgemm_ex_ws with the workspace
    fdl_sgemm_workspace_size asks for when it asks for one, else fdl_sgemm_ex.
    """
    gen = torch.Generator(device="cuda").manual_seed(seed)
    a_shape = (batch, K, M) if ta else (batch, M, K)
    b_shape = (batch, N, K) if tb else (batch, K, N)
    As = [torch.randn(a_shape, generator=gen, device="cuda") for _ in range(rotate)]
    Bs = [torch.randn(b_shape, generator=gen, device="cuda") for _ in range(rotate)]
    Cs = [torch.empty((batch, M, N), device="cuda") for _ in range(rotate)]
    bias = torch.randn((N,), generator=gen, device="cuda") * 0.1
    lda = M if ta else K
    ldb = K if tb else N
    stream = torch.cuda.current_stream().cuda_stream
    state = {"i": 0}
    ws_bytes = capi.workspace_size(ta, tb, M, N, K, batch)
    ws = torch.empty((ws_bytes // 4,), device="cuda") if ws_bytes else None

    def launch():
        i = state["i"]
        state["i"] = (i + 1) % rotate
        args = (ta, tb, M, N, K, As[i].data_ptr(), lda, M * K, Bs[i].data_ptr(), ldb, K * N,
                Cs[i].data_ptr(), N, M * N, batch, bias.data_ptr() if epi in (1, 2) else None,
                None, epi)
        if ws is None:
            capi.sgemm_ex(*args, stream)
        else:
            capi.sgemm_ex_ws(*args, ws.data_ptr(), ws_bytes, stream)

    return launch, As[0], Bs[0], Cs[0]


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(n, rows):
    """Restated reference CPU loop (oracle/gemm_cpu, 1 thread) on a row block.

    The reference has no threading, so the loop runs on one core; the process
    is pinned to a single CPU for the timed call and unpinned afterwards.  The
    loop's cost per row is uniform, so the rate of a row block is the rate of
    the whole product.
    """
    import numpy as np

    import oracle

    g = np.random.default_rng(0)
    A = g.standard_normal((rows, n)).astype(np.float32)
    B = g.standard_normal((n, n)).astype(np.float32)
    saved = os.sched_getaffinity(0)
    core = min(saved)
    os.sched_setaffinity(0, {core})
    try:
        t0 = time.perf_counter()
        oracle.gemm_cpu(A, B)
        dt = time.perf_counter() - t0
    finally:
        os.sched_setaffinity(0, saved)
    flops = 2.0 * rows * n * n
    return {
        "value": flops / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": 1,
        "kind": "port",
        "extrapolated": rows < n,
        "sample": f"extrapolated from a {rows}-row block of the {n}^3 NN GEMM ({rows} of {n} "
                  f"rows timed, {dt:.2f} s; the whole product would take {dt * n / rows:.0f} s; "
                  f"gemm_cpu loop, gcc -O2 -ffp-contract=off, 1 thread pinned to cpu {core}); "
                  f"host {cpu_model()}, {len(saved)} cpus visible",
    }


def cpu_baseline_mlp(seconds=8.0):
    """The restated reference step (oracle_mlp2_train_step: the gemm_cpu loop for
    all six products of legacy/src/runtime/Network.cpp:7-34's step order, the
    softmax-CE gradient of legacy/src/ops/SoftmaxCrossEntropyLoss.cpp:39-51 and
    the SGD update of legacy/include/dl/optim/Optimizer.hpp:24-34) on BASELINE
    config 2 (784-256-10, batch 256, dX included), 1 thread pinned to one core,
    repeated for about ``seconds``: steps/s."""
    import numpy as np

    import oracle

    g = np.random.default_rng(2)
    B, I, H, C = 256, 784, 256, 10
    X = g.random((B, I), dtype=np.float32)
    labels = g.integers(0, C, B).astype(np.int64)
    W1 = g.uniform(-(6 / I) ** 0.5, (6 / I) ** 0.5, (I, H)).astype(np.float32)
    W2 = g.uniform(-(6 / H) ** 0.5, (6 / H) ** 0.5, (H, C)).astype(np.float32)
    b1, b2 = np.zeros(H, np.float32), np.zeros(C, np.float32)
    saved = os.sched_getaffinity(0)
    core = min(saved)
    os.sched_setaffinity(0, {core})
    try:
        steps, t0 = 0, time.perf_counter()
        while True:
            r = oracle.mlp2_train_step(X, labels, W1, b1, W2, b2, 0.1)
            W1, b1, W2, b2 = r["W1"], r["b1"], r["W2"], r["b2"]
            steps += 1
            if time.perf_counter() - t0 >= seconds:
                break
        dt = time.perf_counter() - t0
    finally:
        os.sched_setaffinity(0, saved)
    return {"value": steps / dt, "unit": "steps/s", "cores": 1, "kind": "port",
            "extrapolated": False,
            "sample": f"{steps} consecutive full steps of the 784-256-10 MLP at batch 256 "
                      f"(oracle_mlp2_train_step: forward, softmax-CE, backward incl. dX, SGD "
                      f"lr 0.1), {dt:.2f} s; gcc -O2 -ffp-contract=off, 1 thread pinned to cpu "
                      f"{core}; host {cpu_model()}, {len(saved)} cpus visible"}


def mlp_rate(capi, torch, steps=2000, warmup=100):
    """fdl_mlp2_train_step on BASELINE config 2 (784-256-10, batch 256), steps/s.

    2000 steps (32 ms): the host issues a step in about 12 us and the GPU runs
    one in about 16, so the queue fills after a start-up of a few hundred
    microseconds, which 200 steps did not amortise (16.9-17.6 us per step
    over 200 steps against 15.8 us over 1000 and 3000, measured in one
    process)."""
    gen = torch.Generator(device="cuda").manual_seed(2)
    B, I, H, C = 256, 784, 256, 10
    X = torch.rand((B, I), generator=gen, device="cuda")
    labels = torch.randint(0, C, (B,), generator=gen, device="cuda", dtype=torch.int64)
    W1 = (torch.rand((I, H), generator=gen, device="cuda") * 2 - 1) * (6 / I) ** 0.5
    W2 = (torch.rand((H, C), generator=gen, device="cuda") * 2 - 1) * (6 / H) ** 0.5
    b1 = torch.zeros(H, device="cuda")
    b2 = torch.zeros(C, device="cuda")
    buf = {k: torch.empty(s, device="cuda") for k, s in dict(
        H=(B, H), logits=(B, C), G2=(B, C), G1=(B, H), dW1=(I, H), db1=(H,), dW2=(H, C),
        db2=(C,), dX=(B, I), loss=(1,)).items()}
    stream = torch.cuda.current_stream().cuda_stream
    p = {k: v.data_ptr() for k, v in buf.items()}
    args = (X.data_ptr(), labels.data_ptr(), B, I, H, C, W1.data_ptr(), b1.data_ptr(),
            W2.data_ptr(), b2.data_ptr(), 0.1, p["H"], p["logits"], p["G2"], p["G1"], p["dW1"],
            p["db1"], p["dW2"], p["db2"], p["dX"], p["loss"], stream)

    # The C function itself, its status checked, without the wrapper's
    # per-call library lookup (the Python loop is the host side of the step).
    fn = capi.load_library().fdl_mlp2_train_step

    def step():
        if fn(*args) != 0:
            raise capi.FdlError("fdl_mlp2_train_step", -1, capi.last_error())

    warm_clock(step, torch.cuda.current_stream())
    ms = time_launches(step, steps, warmup, torch.cuda.current_stream())
    loss = float(buf["loss"].item())
    # The same step captured into a HIP graph and replayed: one step per
    # graph, and GRAPH_STEPS consecutive steps per graph (one host launch for
    # all of them; ms per step = ms per replay / GRAPH_STEPS).
    graph_ms = {}
    for per in (1, GRAPH_STEPS):
        handle = capi.mlp2_graph_create_steps(per, *args)
        try:
            launch = lambda: capi.mlp2_graph_launch(handle, stream)  # noqa: E731
            warm_clock(launch, torch.cuda.current_stream())
            replays = max(steps // per, 20)
            graph_ms[per] = time_launches(launch, replays, max(warmup // per, 2),
                                          torch.cuda.current_stream()) / per
        finally:
            capi.mlp2_graph_destroy(handle)
    return 1000.0 / ms, ms, loss, graph_ms


GRAPH_STEPS = 64  # steps per graph in the multi-step replay figure


IDX_COUNT, IDX_PIXELS, IDX_BATCH = 60000, 784, 256  # MNIST train set: 60000 records of 28x28


def idx_bytes(rows, pixels=IDX_PIXELS, indexed=False):
    """Algorithmic HBM bytes of fdl_idx_gather over ``rows`` rows: 1 byte read
    and 4 written per pixel, 1 read and 8 written per label, plus an 8-byte
    index read per row when an index is used."""
    return rows * (pixels * 5 + 9 + (8 if indexed else 0))


def idx_data_rate(capi, torch, steps=30, warmup=5):
    """fdl_idx_gather on an MNIST-sized set resident in HBM (synthetic bytes).
    Two copies of the set and of the outputs alternate, so consecutive
    launches touch 470 MB, more than the 256 MB Infinity Cache."""
    gen = torch.Generator(device="cuda").manual_seed(3)
    count, px, B = IDX_COUNT, IDX_PIXELS, IDX_BATCH
    copies = 2
    imgs = [torch.randint(0, 256, (count, px), generator=gen, device="cuda",
                          dtype=torch.uint8) for _ in range(copies)]
    labs = [torch.randint(0, 10, (count,), generator=gen, device="cuda", dtype=torch.uint8)
            for _ in range(copies)]
    xs = [torch.empty((count, px), device="cuda") for _ in range(copies)]
    ys = [torch.empty(count, device="cuda", dtype=torch.int64) for _ in range(copies)]
    perm = torch.randperm(count, generator=gen, device="cuda")
    xb = torch.empty((B, px), device="cuda")
    yb = torch.empty(B, device="cuda", dtype=torch.int64)
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    it = [0]

    def whole(index=None):
        i = it[0] % copies
        it[0] += 1
        capi.idx_gather(imgs[i].data_ptr(), labs[i].data_ptr(), count, px, index, count, 255.0,
                        xs[i].data_ptr(), ys[i].data_ptr(), sh)

    def batch():
        j = (it[0] * B) % (count - B)
        it[0] += 1
        capi.idx_gather(imgs[0].data_ptr(), labs[0].data_ptr(), count, px,
                        perm.data_ptr() + 8 * j, B, 255.0, xb.data_ptr(), yb.data_ptr(), sh)

    out = {}
    for name, fn, rows, indexed in [("whole_set", whole, count, False),
                                    ("epoch_permuted", lambda: whole(perm.data_ptr()), count, True),
                                    ("batch_256", batch, B, True)]:
        warm_clock(fn, stream)
        ms = time_launches(fn, steps, warmup, stream)
        nbytes = idx_bytes(rows, indexed=indexed)
        out[name] = {"ms": ms, "gbs": nbytes / (ms / 1e3) / 1e9,
                     "frac_hbm": nbytes / (ms / 1e3) / 1e9 / PEAK_HBM_GBS, "bytes": nbytes}
    return out


def idx_epoch_rate(capi, torch, epochs=2):
    """One training epoch of the 784-256-10 MLP (batch 256, lr 0.1) over an
    MNIST-sized set resident in HBM, each step one fdl_mlp2_train_step.
    "per_batch" gathers each batch (fdl_idx_gather through a permutation)
    right before its step; "whole_epoch" gathers the epoch's 234 batches in
    one launch into a 188 MB fp32 buffer and each step reads its rows at an
    offset (dl::train::train_epoch's default).  steps/s over `epochs` epochs
    after one untimed epoch."""
    gen = torch.Generator(device="cuda").manual_seed(4)
    count, px, B, H, C = IDX_COUNT, IDX_PIXELS, IDX_BATCH, 256, 10
    imgs = torch.randint(0, 256, (count, px), generator=gen, device="cuda", dtype=torch.uint8)
    labs = torch.randint(0, C, (count,), generator=gen, device="cuda", dtype=torch.uint8)
    perm = torch.randperm(count, generator=gen, device="cuda")
    W1 = (torch.rand((px, H), generator=gen, device="cuda") * 2 - 1) * (6 / px) ** 0.5
    W2 = (torch.rand((H, C), generator=gen, device="cuda") * 2 - 1) * (6 / H) ** 0.5
    b1 = torch.zeros(H, device="cuda")
    b2 = torch.zeros(C, device="cuda")
    buf = {k: torch.empty(s, device="cuda") for k, s in dict(
        H=(B, H), logits=(B, C), G2=(B, C), G1=(B, H), dW1=(px, H), db1=(H,), dW2=(H, C),
        db2=(C,), dX=(B, px), loss=(1,)).items()}
    p = {k: v.data_ptr() for k, v in buf.items()}
    steps = count // B
    xs = torch.empty((steps * B, px), device="cuda")
    ys = torch.empty(steps * B, device="cuda", dtype=torch.int64)
    sh = torch.cuda.current_stream().cuda_stream

    def gather(row0, rows):
        capi.idx_gather(imgs.data_ptr(), labs.data_ptr(), count, px, perm.data_ptr() + 8 * row0,
                        rows, 255.0, xs.data_ptr(), ys.data_ptr(), sh)

    def step(row0):
        capi.mlp2_train_step(xs.data_ptr() + 4 * row0 * px, ys.data_ptr() + 8 * row0, B, px, H,
                             C, W1.data_ptr(), b1.data_ptr(), W2.data_ptr(), b2.data_ptr(), 0.1,
                             p["H"], p["logits"], p["G2"], p["G1"], p["dW1"], p["db1"],
                             p["dW2"], p["db2"], p["dX"], p["loss"], sh)

    def per_batch():
        for i in range(steps):
            gather(i * B, B)
            step(0)

    def whole_epoch():
        gather(0, steps * B)
        for i in range(steps):
            step(i * B)

    out = {"steps_per_epoch": steps}
    main = torch.cuda.current_stream()
    for name, fn in (("per_batch", per_batch), ("whole_epoch", whole_epoch)):
        fn()
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(main)
        for _ in range(epochs):
            fn()
        t1.record(main)
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / epochs
        out[name] = {"ms_per_epoch": ms, "steps_per_s": steps / (ms / 1e3)}
    out["final_loss"] = float(buf["loss"].item())
    return out


def cpu_baseline_idx(seconds=2.0):
    """The restated loader conversion (oracle_idx_gather, the loop of
    legacy/src/data/DataLoader.cpp:61-68 over the whole set), 1 thread."""
    import numpy as np

    import oracle

    g = np.random.default_rng(3)
    images = g.integers(0, 256, (IDX_COUNT, IDX_PIXELS), dtype=np.uint8)
    labels = g.integers(0, 10, IDX_COUNT, dtype=np.uint8)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.idx_gather(images, labels, None, batch=IDX_COUNT)
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = (time.perf_counter() - t0) / reps
    return {"gbs": idx_bytes(IDX_COUNT) / dt / 1e9, "ms": dt * 1e3, "cores": 1, "kind": "port",
            "sample": f"the whole 60000x784 set, {reps} passes (oracle_idx_gather, gcc -O2)"}


def sampled_parity(A, B, C, n, rows=16):
    """Cheap parity guard on the benchmarked output: sampled rows vs fp64 dot products."""
    import numpy as np

    import torch

    torch.cuda.synchronize()
    idx = torch.randint(0, n, (rows,), generator=torch.Generator().manual_seed(5))
    a = A[0][idx.cuda()].double().cpu().numpy()
    b = B[0].double().cpu().numpy()
    c = C[0][idx.cuda()].double().cpu().numpy()
    ref = a @ b
    bound = 2.0 * (np.sqrt(n) + 2.0) * float(np.finfo(np.float32).eps) * (np.abs(a) @ np.abs(b))
    return bool(np.all(np.abs(c - ref) <= bound))


def torch_mlp_rate(torch, steps=2000, warmup=100):
    """The same 784-256-10 step written in eager PyTorch (autograd, fused
    cross_entropy, torch.optim.SGD), for comparison only: steps/s."""
    gen = torch.Generator(device="cuda").manual_seed(2)
    B, I, H, C = 256, 784, 256, 10
    X = torch.rand((B, I), generator=gen, device="cuda")
    labels = torch.randint(0, C, (B,), generator=gen, device="cuda", dtype=torch.int64)
    W1 = ((torch.rand((I, H), generator=gen, device="cuda") * 2 - 1) * (6 / I) ** 0.5)
    W2 = ((torch.rand((H, C), generator=gen, device="cuda") * 2 - 1) * (6 / H) ** 0.5)
    params = [W1.requires_grad_(), torch.zeros(H, device="cuda", requires_grad=True),
              W2.requires_grad_(), torch.zeros(C, device="cuda", requires_grad=True)]
    opt = torch.optim.SGD(params, lr=0.1)

    def step():
        opt.zero_grad(set_to_none=False)
        h = torch.relu(torch.addmm(params[1], X, params[0]))
        loss = torch.nn.functional.cross_entropy(torch.addmm(params[3], h, params[2]), labels)
        loss.backward()
        opt.step()

    warm_clock(step, torch.cuda.current_stream())
    ms = time_launches(step, steps, warmup, torch.cuda.current_stream())
    return 1000.0 / ms, ms


def sweep(capi, torch, path):
    """Every BASELINE configuration, one line each, with the same GEMM through
    PyTorch's vendor BLAS (``vendor_ms``) timed the same way beside it."""
    out = []

    def rec(name, launch, vendor, flops, nbytes, steps=30, warmup=5):
        warm_clock(launch, torch.cuda.current_stream())
        ms = time_launches(launch, steps, warmup, torch.cuda.current_stream())
        t = ms / 1e3
        ridge = PEAK_FP32_MFMA_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
        bound = "mfma" if flops / nbytes >= ridge else "hbm"
        row = {"config": name, "ms": ms, "tflops": flops / t / 1e12, "gbs": nbytes / t / 1e9,
               "bound": bound,
               "frac": (flops / t / 1e12 / PEAK_FP32_MFMA_TFLOPS) if bound == "mfma"
               else (nbytes / t / 1e9 / PEAK_HBM_GBS)}
        if vendor is not None:
            warm_clock(vendor, torch.cuda.current_stream())
            row["vendor_ms"] = time_launches(vendor, steps, warmup, torch.cuda.current_stream())
            row["speedup_vs_vendor"] = row["vendor_ms"] / ms
        out.append(row)
        print(json.dumps(row), file=sys.stderr, flush=True)

    def b4(M, N, K, batch=1, bias=False):
        return 4.0 * batch * (M * K + K * N + M * N) + (4.0 * N if bias else 0.0)

    def both(M, N, K, **kw):
        launch, *_ = gemm_case(capi, torch, M, N, K, **kw)
        return launch, vendor_case(torch, M, N, K, **kw)

    rec("C1 256x128x784 NN", *both(256, 128, 784), 2.0 * 256 * 128 * 784, b4(256, 128, 784))
    for n in (1024, 2048, 4096, 8192):
        rec(f"C3 {n}^3 NN", *both(n, n, n), 2.0 * n ** 3, b4(n, n, n),
            steps=10 if n == 8192 else 30)
    for tb in (0, 1):
        rec(f"C4 64x(128x128x64) {'NT' if tb else 'NN'}",
            *both(128, 128, 64, tb=tb, batch=64, rotate=40), 2.0 * 64 * 128 * 128 * 64,
            b4(128, 128, 64, 64))
    for m in (1, 8):
        rec(f"C5a M={m} K=N=4096 bias+relu", *both(m, 4096, 4096, epi=2, rotate=6),
            2.0 * m * 4096 * 4096, b4(m, 4096, 4096, bias=True))
    for n in (777, 1000, 1023):
        rec(f"C5b {n}^3 bias+relu", *both(n, n, n, epi=2), 2.0 * n ** 3,
            b4(n, n, n, bias=True))
    for name, row in idx_data_rate(capi, torch).items():
        out.append({"config": f"IDX gather {name} (60000x784 bytes -> fp32)", "ms": row["ms"],
                    "gbs": row["gbs"], "bound": "hbm", "frac": row["frac_hbm"]})
        print(json.dumps(out[-1]), file=sys.stderr, flush=True)
    ep = idx_epoch_rate(capi, torch)
    out.append({"config": "MLP epoch from resident IDX bytes (234 steps of 256)",
                "per_batch_steps_per_s": ep["per_batch"]["steps_per_s"],
                "whole_epoch_steps_per_s": ep["whole_epoch"]["steps_per_s"]})
    print(json.dumps(out[-1]), file=sys.stderr, flush=True)
    sps, ms, _, gms = mlp_rate(capi, torch)
    tsps, tms = torch_mlp_rate(torch)
    out.append({"config": "C2 MLP 784-256-10 b256 step", "ms": ms, "steps_per_s": sps,
                "graph_ms": gms[1], "graph_steps_per_s": 1000.0 / gms[1],
                f"graph{GRAPH_STEPS}_ms": gms[GRAPH_STEPS],
                f"graph{GRAPH_STEPS}_steps_per_s": 1000.0 / gms[GRAPH_STEPS],
                "torch_eager_ms": tms, "torch_eager_steps_per_s": tsps})
    print(json.dumps(out[-1]), file=sys.stderr, flush=True)
    with open(path, "w") as f:
        json.dump(out, f, indent=1)


def main():
    global CLOCK_WARM
    args = parse_args()
    if args.collect_profiles or args.summarize:
        from fast_dl_amd import profiling

        if args.collect_profiles:
            rc = profiling.collect(args.collect_profiles, args.stages.split(","),
                                   args.configs.split(",") if args.configs else None)
            if rc:
                sys.exit(rc)
        if args.summarize:
            profiling.summarize(args.summarize)
        return
    CLOCK_WARM = not args.no_clock_warm
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "sharding the path over several GPUs is designed, not built", file=sys.stderr)
        sys.exit(2)
    import torch

    import fast_dl_amd.capi as capi

    capi.load_library()
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream()
    if args.profile_mode and args.profile_config != "headline":
        cfg = PROFILE_CONFIGS[args.profile_config]
        if cfg == "idx":
            rows = idx_data_rate(capi, torch, steps=args.steps, warmup=args.warmup)
            print(json.dumps({"profile_mode": True, "config": args.profile_config,
                              "rows": rows}), flush=True)
            return
        if cfg == "mlp" and args.profile_vendor:
            _, pms = torch_mlp_rate(torch, steps=args.steps, warmup=args.warmup)
        elif cfg == "mlp":
            _, pms, _, _ = mlp_rate(capi, torch, steps=args.steps, warmup=args.warmup)
        else:
            M, N, K, tb, batch, epi, rot = cfg
            if args.profile_vendor:
                plaunch = vendor_case(torch, M, N, K, tb=tb, batch=batch, epi=epi, rotate=rot)
            else:
                plaunch, *_ = gemm_case(capi, torch, M, N, K, tb=tb, batch=batch, epi=epi,
                                        rotate=rot)
            # Timed on a warmed clock, as the sweep rows are.
            warm_clock(plaunch, stream)
            pms = time_launches(plaunch, args.steps, args.warmup, stream)
        if args.copy_calib:
            copy_calibration(torch)
        print(json.dumps({"profile_mode": True, "config": args.profile_config,
                          "vendor": args.profile_vendor, "ms_per_launch": pms}), flush=True)
        return
    n = args.size
    if args.profile_mode and args.profile_vendor:
        vms = time_launches(vendor_case(torch, n, n, n), args.steps, args.warmup, stream)
        print(json.dumps({"profile_mode": True, "config": "headline", "vendor": True,
                          "ms_per_launch": vms}), flush=True)
        return
    launch, A, B, C = gemm_case(capi, torch, n, n, n, seed=0)
    if args.profile_mode:
        ms = time_launches(launch, args.steps, args.warmup, stream)
        if args.copy_calib:
            copy_calibration(torch)
        print(json.dumps({"profile_mode": True, "ms_per_launch": ms}), flush=True)
        return

    mlp = None
    if not args.no_mlp:
        sps, mlp_ms, loss, graph_ms = mlp_rate(capi, torch)
        mlp = {"steps_per_s": sps, "ms_per_step": mlp_ms,
               "graph_steps_per_s": 1000.0 / graph_ms[1], "graph_ms_per_step": graph_ms[1],
               f"graph{GRAPH_STEPS}_steps_per_s": 1000.0 / graph_ms[GRAPH_STEPS],
               f"graph{GRAPH_STEPS}_ms_per_step": graph_ms[GRAPH_STEPS],
               "final_loss": loss,
               "config": "784-256-10, batch 256, lr 0.1, full step (forward, softmax-CE, "
                         "backward incl. dX, SGD): one fdl_mlp2_train_step call (3 launches) "
                         "per step; graph = the same step replayed as a HIP graph; "
                         f"graph{GRAPH_STEPS} = {GRAPH_STEPS} consecutive steps captured in "
                         "one graph (fdl_mlp2_graph_create_steps), one replay per "
                         f"{GRAPH_STEPS} steps"}
    idx = None
    if not args.no_mlp:
        idx = idx_data_rate(capi, torch)
        idx["epoch_train"] = idx_epoch_rate(capi, torch)
        idx["workload"] = ("fdl_idx_gather over an MNIST-sized set resident in HBM: 60000 "
                           "records of 784 bytes + label bytes -> fp32 /255 rows and int64 "
                           "labels; batch_256 = one training batch through a permutation; "
                           "epoch_train = a 784-256-10 MLP epoch (234 steps of batch 256, one "
                           "fdl_mlp2_train_step each) fed by a gather per batch or by one "
                           "gather of the whole epoch")

    # The GPU clock ramps over the first ~20 ms of back-to-back large
    # launches after even 10 ms of idle or of launch-bound work (measured at
    # 4096^3: the first launches take 1.07-1.10 ms, then 0.945 ms from about
    # the 20th).  The vendor comparison runs just before the headline with a
    # 50 ms clock warm-up of its own, so both are timed on a warmed clock; the
    # headline itself is exactly `warmup` untimed and `steps` timed launches.
    vendor = vendor_case(torch, n, n, n)
    warm_clock(vendor, stream)
    vendor_ms = time_launches(vendor, args.steps, args.warmup, stream)
    ms = time_launches(launch, args.steps, args.warmup, stream)
    flops = 2.0 * n * n * n
    tflops = flops / (ms / 1e3) / 1e12
    med, p10, p90 = launch_percentiles(launch, args.steps, stream)
    parity = sampled_parity(A, B, C, n)
    if args.sweep:
        sweep(capi, torch, args.sweep)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(n, rows=64)
        if mlp is not None:
            mlp["cpu_baseline"] = cpu_baseline_mlp()
        if idx is not None:
            idx["cpu_baseline"] = cpu_baseline_idx()

    family = capi.kernel_choice(0, 0, n, n, n)
    kernel = capi.KERNEL_NAMES.get(family, "auto")
    kernel_fn = {capi.KERNEL_DMA256: "sgemm_dma_kernel", capi.KERNEL_DMA128: "sgemm_dma_kernel",
                 capi.KERNEL_DMA64: "sgemm_dma_kernel", capi.KERNEL_DMA128W8: "sgemm_dma_kernel",
                 capi.KERNEL_DMA64U: "sgemm_dma_kernel", capi.KERNEL_DMA128W8U: "sgemm_dma_kernel",
                 capi.KERNEL_SKINNY: "sgemm_skinny_kernel",
                 capi.KERNEL_SPLITK32: "sgemm_splitk32_kernel",
                 capi.KERNEL_SPLITK16: "sgemm_splitk16_kernel"}.get(family, "sgemm_tiled_kernel")
    line = {
        "metric": "fp32 GEMM TFLOP/s at M=N=K=4096 (% MI355X fp32 peak); MLP train steps/s",
        "value": tflops,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "launch_ms": {"median": med, "p10": p10, "p90": p90},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (torch.randn on device, seed 0)",
        "config": {"workload": f"sgemm NN row-major M=N=K={n}, A,B ~ N(0,1)",
                   "kernel": f"{kernel_fn} ({kernel})", "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": tflops / PEAK_FP32_MFMA_TFLOPS,
                     "traffic": read_traffic()},
        "cpu_baseline": cpu,
        "mlp_train": mlp,
        "idx_data": idx,
        "parity_sampled_rows_fp64": parity,
        "vendor_blas": {"what": "torch.mm fp32 (rocBLAS/hipBLASLt), same operands and stream",
                        "ms": vendor_ms, "tflops": flops / (vendor_ms / 1e3) / 1e12},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
