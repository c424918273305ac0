"""rocprofv3 evidence for every BASELINE configuration: collection and summaries.

    python bench.py --collect-profiles DIR [--stages trace,vendor,counters]
    python bench.py --summarize DIR

``collect`` runs rocprofv3 as a child process once per (configuration,
stage), each over ``bench.py --profile-mode --profile-config NAME``, and writes
the raw CSV output under DIR.  It never touches the GPU itself (the profiled
program is started as a child, never exec'd).  ``summarize`` reads DIR and
writes the text summaries under ``profiles/``; every figure in them comes
from those CSV files by the code below.

Stages:
  trace     kernel trace of this build's kernels per configuration
  vendor    the same workload through PyTorch's vendor BLAS (comparison)
  counters  two --pmc passes per configuration (the hardware collects only
            a few counters of each block per pass):
              A: SQ_WAVES SQ_WAVE_CYCLES SQ_WAIT_ANY SQ_INSTS_VALU_MFMA_MOPS_F32
                 GRBM_GUI_ACTIVE FETCH_SIZE
              B: SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS
                 SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE WRITE_SIZE
            each followed by known-size copy, sum and fill kernels that scale
            FETCH_SIZE and WRITE_SIZE (bench.py copy_calibration).

Derived figures (per dispatch, averaged over the timed dispatches):
  MFMA utilisation  = MOPS_F32 * 512 FLOP / (256 CUs * 256 FLOP/clk * cycles),
                      cycles = traced duration x the clock GRBM_GUI_ACTIVE / 8
                      (the counter sums 8 XCDs) gives over a long dispatch
  MFMA busy         = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs * cycles)
  LDS bank conflict = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE
  waiting           = SQ_WAIT_ANY / SQ_WAVE_CYCLES
  HBM bytes         = FETCH_SIZE * read scale + WRITE_SIZE * write scale (KiB)
"""
from __future__ import annotations

import collections
import csv
import glob
import os
import re
import subprocess
import sys
import time
from dataclasses import dataclass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROFILES = os.path.join(ROOT, "profiles")

PEAK_TFLOPS = 157.3   # MI355X fp32 MFMA, dense
PEAK_GBS = 8000.0     # MI355X HBM3E
CUS = 256
FLOP_PER_CU_CLK = 256
NOMINAL_GHZ = 2.4


@dataclass(frozen=True)
class Workload:
    label: str
    shape: tuple | None   # (M, N, K, transB, batch, epilogue, rotate) or None
    kind: str = "gemm"    # gemm | mlp | idx
    steps: int = 50
    warmup: int = 10


CONFIGS = {
    "headline": Workload("C3 4096^3 NN (bench headline)", (4096, 4096, 4096, 0, 1, 0, 1),
                         steps=50, warmup=40),
    "c1": Workload("C1 256x128x784 NN", (256, 128, 784, 0, 1, 0, 1)),
    "c3_1024": Workload("C3 1024^3 NN", (1024, 1024, 1024, 0, 1, 0, 1)),
    "c3_2048": Workload("C3 2048^3 NN", (2048, 2048, 2048, 0, 1, 0, 1)),
    "c3_8192": Workload("C3 8192^3 NN", (8192, 8192, 8192, 0, 1, 0, 1), steps=10, warmup=5),
    "c4_nn": Workload("C4 64 x (128x64 . 64x128) NN", (128, 128, 64, 0, 64, 0, 40)),
    "c4_nt": Workload("C4 64 x (128x64 . 64x128) NT", (128, 128, 64, 1, 64, 0, 40)),
    "c5a_m1": Workload("C5a M=1 K=N=4096 bias+ReLU", (1, 4096, 4096, 0, 1, 2, 6)),
    "c5a_m8": Workload("C5a M=8 K=N=4096 bias+ReLU", (8, 4096, 4096, 0, 1, 2, 6)),
    "c5b_777": Workload("C5b 777^3 bias+ReLU", (777, 777, 777, 0, 1, 2, 1)),
    "c5b_1000": Workload("C5b 1000^3 bias+ReLU", (1000, 1000, 1000, 0, 1, 2, 1)),
    "c5b_1023": Workload("C5b 1023^3 bias+ReLU", (1023, 1023, 1023, 0, 1, 2, 1)),
    "c2_mlp": Workload("C2 MLP 784-256-10 step, batch 256 (eager steps, then graph replays)",
                       None, kind="mlp"),
    "idx_data": Workload("IDX gather, 60000x784 bytes -> fp32 (whole set, permuted epoch, batch)",
                         None, kind="idx", steps=30, warmup=5),
}
ORDER = list(CONFIGS)

PASS_A = ["SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_WAIT_ANY", "SQ_INSTS_VALU_MFMA_MOPS_F32",
          "GRBM_GUI_ACTIVE", "FETCH_SIZE"]
PASS_B = ["SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_INSTS_LDS",
          "SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE", "WRITE_SIZE"]

BENCH_ARGS = "python3 <repo>/bench.py --profile-mode --profile-config {cfg} --steps {s} --warmup {w}"
TRACE_CMD = ("cd /tmp && export TMPDIR=/tmp && timeout -s KILL 150 rocprofv3 --kernel-trace --stats "
             "--output-format csv -d <DIR>/{run} -o run -- " + BENCH_ARGS)
PMC_CMD = ("cd /tmp && export TMPDIR=/tmp && timeout -s KILL 150 rocprofv3 --pmc {ctrs} "
           "--output-format csv -d <DIR>/{run} -o run -- " + BENCH_ARGS +
           " --copy-calib --no-clock-warm")
COLLECT_CMD = "python bench.py --collect-profiles <DIR> && python bench.py --summarize <DIR>"


def flops_bytes(cfg: str) -> tuple[float, float]:
    """Algorithmic FLOP 2*M*N*K*batch and bytes 4*(MK+KN+MN)*batch (+4N bias)."""
    M, N, K, _, batch, epi, _ = CONFIGS[cfg].shape
    return (2.0 * M * N * K * batch,
            4.0 * batch * (M * K + K * N + M * N) + (4.0 * N if epi in (1, 2) else 0.0))


# ----------------------------------------------------------------------- collect

def _run(argv: list[str], log: str) -> int:
    env = dict(os.environ, TMPDIR="/tmp")
    with open(log, "w") as f:
        proc = subprocess.run(argv, cwd="/tmp", env=env, stdout=f, stderr=subprocess.STDOUT)
    return proc.returncode


def _bench_argv(cfg: str, vendor: bool = False, pmc: bool = False) -> list[str]:
    w = CONFIGS[cfg]
    argv = [sys.executable, os.path.join(ROOT, "bench.py"), "--profile-mode", "--profile-config",
            cfg, "--steps", str(w.steps), "--warmup", str(w.warmup)]
    if vendor:
        argv.append("--profile-vendor")
    if pmc:
        argv += ["--copy-calib", "--no-clock-warm"]
    return argv


def collect(out_dir: str, stages: list[str], configs: list[str] | None = None) -> int:
    """Runs every rocprofv3 pass; returns the number of failed passes.  A pass
    that fails stops the collection (nothing more runs on the GPU)."""
    os.makedirs(out_dir, exist_ok=True)
    out_dir = os.path.abspath(out_dir)
    configs = configs or ORDER
    jobs = []
    for stage in stages:
        for cfg in configs:
            if stage == "trace":
                jobs.append((f"trace_{cfg}", ["--kernel-trace", "--stats"], cfg, False, False))
            elif stage == "vendor" and cfg != "idx_data":
                jobs.append((f"vendor_{cfg}", ["--kernel-trace", "--stats"], cfg, True, False))
            elif stage == "counters":
                jobs.append((f"pmcA_{cfg}", ["--pmc", *PASS_A], cfg, False, True))
                jobs.append((f"pmcB_{cfg}", ["--pmc", *PASS_B], cfg, False, True))
    for i, (name, prof_args, cfg, vendor, pmc) in enumerate(jobs):
        t0 = time.time()
        argv = ["timeout", "-s", "KILL", "150", "rocprofv3", *prof_args, "--output-format", "csv",
                "-d", os.path.join(out_dir, name), "-o", "run", "--",
                *_bench_argv(cfg, vendor=vendor, pmc=pmc)]
        log = os.path.join(out_dir, name + ".log")
        rc = _run(argv, log)
        # rocprofv3 itself can end with SIGSEGV (139) after the profiled program
        # has finished and its output files are written (seen at the tool's
        # teardown on this stack).  Such a pass counts only if the program
        # printed its closing profile_mode line and the CSV holds at least the
        # timed dispatches.
        ok = rc == 0 or (rc == 139 and _finished(log) and
                         _dispatches(os.path.join(out_dir, name)) >= CONFIGS[cfg].steps)
        print(f"[{i + 1}/{len(jobs)}] {name}: rc={rc} {time.time() - t0:.1f}s", flush=True)
        if not ok:
            print(f"stopping: {name} failed (see {name}.log)", flush=True)
            return 1
    return 0


def _finished(log: str) -> bool:
    """Whether the profiled bench.py printed its closing {"profile_mode": true, ...} line."""
    try:
        with open(log) as f:
            lines = f.read().splitlines()
    except OSError:
        return False
    for line in reversed(lines):
        if line.startswith("{") and '"profile_mode": true' in line:
            return True
    return False


def _dispatches(d: str) -> int:
    """Rows of the pass's kernel trace or counter CSV (0 when there is none)."""
    for suffix in ("kernel_trace.csv", "counter_collection.csv"):
        files = glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True)
        if files:
            with open(files[0]) as f:
                return max(0, sum(1 for _ in f) - 1)
    return 0


# ------------------------------------------------------------------- reading CSV

def _csv(d: str, suffix: str) -> list[dict]:
    files = glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True)
    if not files:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def trace(d: str) -> list[tuple[str, float]]:
    """(kernel name, duration us) per dispatch, in start order."""
    rows = _csv(d, "kernel_trace.csv")
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    return [(r["Kernel_Name"], (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
            for r in rows]


def counters(d: str) -> list[dict]:
    """One dict per dispatch: counter values summed over their instances,
    plus _name, _dur (us) and _id, in dispatch order."""
    by = collections.OrderedDict()
    for r in _csv(d, "counter_collection.csv"):
        k = int(r["Dispatch_Id"])
        e = by.setdefault(k, {"_name": r["Kernel_Name"], "_id": k,
                              "_dur": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3})
        e[r["Counter_Name"]] = e.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return [by[k] for k in sorted(by)]


def short(name: str) -> str:
    name = name.replace("fdl::(anonymous namespace)::", "").replace("(anonymous namespace)::", "")
    return re.sub(r"\s+", " ", name)


def is_ours(name: str) -> bool:
    return "fdl::" in name


def kernel_family(name: str) -> str:
    m = re.search(r"(sgemm_\w+?_kernel|mlp_head_kernel|idx_gather_kernel|\w+_kernel)", short(name))
    return m.group(1) if m else short(name)[:40]


def timed_mean(values: list[float], steps: int) -> float:
    last = values[-steps:]
    return sum(last) / len(last)


def period(names: list[str], maxp: int = 40) -> int | None:
    for p in range(1, maxp + 1):
        if len(names) >= 4 * p and all(names[-k] == names[-k - p] for k in range(1, 3 * p + 1)):
            return p
    return None


def per_iteration(tr: list[tuple[str, float]], steps: int) -> tuple[float, int, list[str]]:
    """GPU time of one iteration: the kernel-name sequence's period p, and the
    summed durations of the last steps*p dispatches / steps."""
    names = [n for n, _ in tr]
    p = period(names) or 1
    last = tr[-steps * p:]
    return sum(t for _, t in last) / steps, p, [n for n, _ in tr[-p:]]


# ---------------------------------------------------------------- calibration

@dataclass
class Calibration:
    read_scale: float
    write_scale: float
    lines: list


def calibration(rows_a: list[dict], rows_b: list[dict]) -> Calibration:
    """Scales for FETCH_SIZE / WRITE_SIZE from the known-size kernels that
    end each --copy-calib run: 3 copies of 256 MiB, 3 of 64 MiB, 3 sums over
    256 MiB and 3 fills of 256 MiB (KiB per dispatch)."""
    def pick(rows, pat, n, skip=0):
        sel = [r for r in rows if re.search(pat, r["_name"])]
        return sel[len(sel) - skip - n: len(sel) - skip] if skip else sel[-n:]

    def mean(rows, ctr):
        return sum(r[ctr] for r in rows) / len(rows)

    KI = 262144.0  # 256 MiB in KiB
    copy_a = [r for r in rows_a if "copyBuffer" in r["_name"]]
    copy_b = [r for r in rows_b if "copyBuffer" in r["_name"]]
    big_a, small_a = copy_a[-6:-3], copy_a[-3:]
    big_b, small_b = copy_b[-6:-3], copy_b[-3:]
    sum_a = pick(rows_a, r"reduce|Reduce|sum", 3)
    fill_b = pick(rows_b, r"[Ff]ill", 3)
    read_scale = KI / mean(big_a, "FETCH_SIZE")
    write_scale = KI / mean(big_b, "WRITE_SIZE")
    lines = [
        "kernel (known bytes)              counter      KiB/dispatch   scale to known",
        f"copy 256 MiB (read 256 MiB)       FETCH_SIZE   {mean(big_a, 'FETCH_SIZE'):12.0f}   "
        f"{read_scale:6.3f}   <- read scale",
        f"copy 64 MiB (read 64 MiB)         FETCH_SIZE   {mean(small_a, 'FETCH_SIZE'):12.0f}   "
        f"{KI / 4 / mean(small_a, 'FETCH_SIZE'):6.3f}",
    ]
    if sum_a:
        lines.append(f"sum over 256 MiB (read 256 MiB)   FETCH_SIZE   {mean(sum_a, 'FETCH_SIZE'):12.0f}   "
                     f"{KI / mean(sum_a, 'FETCH_SIZE'):6.3f}")
    lines += [
        f"copy 256 MiB (write 256 MiB)      WRITE_SIZE   {mean(big_b, 'WRITE_SIZE'):12.0f}   "
        f"{write_scale:6.3f}   <- write scale",
        f"copy 64 MiB (write 64 MiB)        WRITE_SIZE   {mean(small_b, 'WRITE_SIZE'):12.0f}   "
        f"{KI / 4 / mean(small_b, 'WRITE_SIZE'):6.3f}",
    ]
    if fill_b:
        lines.append(f"fill 256 MiB (write 256 MiB)      WRITE_SIZE   {mean(fill_b, 'WRITE_SIZE'):12.0f}   "
                     f"{KI / mean(fill_b, 'WRITE_SIZE'):6.3f}")
    return Calibration(read_scale, write_scale, lines)


# --------------------------------------------------------------------- summaries

def _header(title: str, cmd_lines: list[str]) -> list[str]:
    return [f"# {title}", "", "made by (from the repository root, on an MI355X):",
            f"  {COLLECT_CMD}", "which runs, per configuration:", *[f"  {c}" for c in cmd_lines], ""]


def _dominant(tr: list[tuple[str, float]], steps: int) -> tuple[str, float, int]:
    agg = collections.OrderedDict()
    for n, t in tr:
        if is_ours(n):
            agg.setdefault(n, []).append(t)
    name = max(agg, key=lambda n: sum(agg[n][-steps:]))
    return name, timed_mean(agg[name], steps), len(agg[name])


def write_traces(d: str) -> dict:
    """profiles/sgemm_baseline_configs_kernel_trace.txt and
    profiles/sgemm_nn_4096_kernel_trace.txt; returns {cfg: (kernel, timed us)}."""
    L = _header("rocprofv3 kernel traces of every BASELINE configuration (this build)",
                [TRACE_CMD.format(run="trace_<config>", cfg="<config>", s="<steps>", w="<warmup>")])
    L += ["Each run launches the configuration warmup + steps times on resident synthetic operands",
          "(HBM-bound configurations rotate operand copies past the 256 MB Infinity Cache); launches",
          "of 15 us and more follow about 50 ms of back-to-back launches that warm the clock.",
          "timed_us is the mean over the last `steps` dispatches of the kernel, the region",
          "bench.py times; rates use the algorithmic FLOP 2*M*N*K*batch and bytes",
          "4*(MK+KN+MN)*batch (+4N with a bias).", ""]
    out = {}
    for cfg in _present(d, "trace"):
        w = CONFIGS[cfg]
        tr = trace(os.path.join(d, f"trace_{cfg}"))
        agg = collections.OrderedDict()
        for n, t in tr:
            if is_ours(n):
                agg.setdefault(n, []).append(t)
        L.append(f"## {cfg}: {w.label}  (steps {w.steps}, warmup {w.warmup})")
        L.append(" calls    avg_us    min_us  timed_us  kernel")
        for n, ts in sorted(agg.items(), key=lambda x: -sum(x[1][-w.steps:])):
            L.append(f"{len(ts):6d} {sum(ts) / len(ts):9.2f} {min(ts):9.2f} "
                     f"{timed_mean(ts, w.steps):9.2f}  {short(n)[:140]}")
        if w.kind == "gemm":
            name, t, calls = _dominant(tr, w.steps)
            # a call of two launches (the skinny K split: partials, then their
            # sum) counts both
            group = [n for n, ts in agg.items() if len(ts) == calls]
            fam = kernel_family(name)
            if len(group) > 1:
                t = sum(timed_mean(agg[n], w.steps) for n in group)
                fam = " + ".join(kernel_family(n) for n in group)
            fl, by = flops_bytes(cfg)
            L.append(f"  => {fam} {t:.2f} us: {fl / t / 1e6:.2f} TFLOP/s "
                     f"({100 * fl / t / 1e6 / PEAK_TFLOPS:.1f}% of {PEAK_TFLOPS}), "
                     f"{by / t / 1e3:.0f} GB/s ({100 * by / t / 1e3 / PEAK_GBS:.1f}% of 8 TB/s)")
            out[cfg] = (name, t)
        elif w.kind == "mlp":
            step_us, p, names = per_iteration([x for x in tr if is_ours(x[0])], w.steps)
            L.append(f"  => one step = {p} kernels, {step_us:.2f} us of GPU time "
                     f"({1e6 / step_us:.0f} steps/s with no gaps between launches)")
            out[cfg] = (None, step_us)
        else:
            name, t, _ = _dominant(tr, w.steps)
            out[cfg] = (name, t)
        L.append("")
    _write("sgemm_baseline_configs_kernel_trace.txt", L)
    if "headline" not in out:
        return out

    st = _csv(os.path.join(d, "trace_headline"), "kernel_stats.csv")
    name, t = out["headline"]
    fl, _ = flops_bytes("headline")
    H = _header("rocprofv3 kernel trace: sgemm_nn_4096 (bench.py headline workload)",
                [TRACE_CMD.format(run="trace_headline", cfg="headline", s=50, w=40)])
    H += ["kernel stats (all dispatches, warmup included):",
          " calls     avg_us     min_us     max_us  name"]
    for r in st:
        if is_ours(r["Name"]):
            H.append(f"{int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:10.1f} "
                     f"{float(r['MinNs']) / 1e3:10.1f} {float(r['MaxNs']) / 1e3:10.1f}  "
                     f"{short(r['Name'])[:140]}")
    H += ["", f"headline kernel average duration over the 50 timed dispatches: {t:.1f} us",
          f"=> {fl / t / 1e6:.1f} TFLOP/s = {100 * fl / t / 1e6 / PEAK_TFLOPS:.1f}% of the "
          f"{PEAK_TFLOPS} TFLOP/s fp32-MFMA peak", ""]
    _write("sgemm_nn_4096_kernel_trace.txt", H)
    return out


def write_vendor(d: str) -> None:
    L = _header("Per-iteration GPU time of every BASELINE workload: this build vs the vendor BLAS",
                [TRACE_CMD.format(run="{trace|vendor}_<config>", cfg="<config>", s="<steps>",
                                  w="<warmup>") + "  [--profile-vendor]"])
    L += ["--profile-vendor launches the same workload through PyTorch (torch.mm / addmm + relu_ /",
          "bmm, full fp32, allow_tf32 off; for C2 the eager autograd step with torch.optim.SGD).",
          "GPU time per iteration = summed kernel durations of the last `steps` iterations / steps",
          "(launch gaps excluded on both sides); an iteration's kernels are the period of the",
          "trace's kernel-name sequence.", "",
          "workload                               ours_us  vendor_us  vendor/ours  kernels (ours | vendor)"]
    for cfg in _present(d, "vendor"):
        w = CONFIGS[cfg]
        tr = [x for x in trace(os.path.join(d, f"trace_{cfg}")) if is_ours(x[0])]
        o, po, _ = per_iteration(tr, w.steps)
        v, pv, vn = per_iteration(trace(os.path.join(d, f"vendor_{cfg}")), w.steps)
        tags = sorted({(re.search(r"(MT\w+?_MI\d+x\d+x\d+)", n) or
                        re.search(r"(\w+_kernel|__amd\w+)", n) or re.search(r"(\w+)", n)).group(1)
                       for n in vn})
        L.append(f"{w.label[:36]:36} {o:9.2f} {v:10.2f} {v / o:12.2f}  {po} | {pv}: "
                 f"{', '.join(tags)[:110]}")
    L.append("")
    _write("vendor_blas_kernel_trace.txt", L)


def _mean_rows(rows: list[dict], keys: list[str]) -> dict:
    return {k: sum(r.get(k, 0.0) for r in rows) / len(rows) for k in keys + ["_dur"]}


def write_counters(d: str, traces: dict) -> dict:
    """profiles/sgemm_configs_counters.txt, counter_calibration.txt and
    sgemm_nn_4096_traffic.txt; returns {cfg: {metric: value}}."""
    cal = calibration(counters(os.path.join(d, "pmcA_headline")),
                      counters(os.path.join(d, "pmcB_headline")))
    C = _header("Counter calibration: FETCH_SIZE and WRITE_SIZE against known-size kernels",
                [PMC_CMD.format(ctrs="<pass A | pass B>", run="pmc{A|B}_headline", cfg="headline",
                                s=50, w=40)])
    C += ["The last kernels of every counter run move known byte counts (bench.py",
          "copy_calibration).  The scale is known KiB / counted KiB; the 256 MiB copy gives the",
          "scales used, the other kernels cross-check them.", ""] + cal.lines + [""]
    _write("counter_calibration.txt", C)

    results = {}
    L = _header("Hardware counters of the dominant kernels of every BASELINE configuration",
                [PMC_CMD.format(ctrs=" ".join(PASS_A), run="pmcA_<config>", cfg="<config>",
                                s="<steps>", w="<warmup>"),
                 PMC_CMD.format(ctrs=" ".join(PASS_B), run="pmcB_<config>", cfg="<config>",
                                s="<steps>", w="<warmup>")])
    L += ["Means over each kernel's last `steps` dispatches (for C2 and the IDX rows, over all",
          "dispatches of the kernel).  Durations are the kernel traces' timed means (counter",
          "runs serialize dispatches).  HBM bytes are FETCH_SIZE and WRITE_SIZE scaled by",
          f"x{cal.read_scale:.3f} (read) and x{cal.write_scale:.3f} (write); see",
          "counter_calibration.txt.  FETCH_SIZE counts L2 misses, which the Infinity Cache may",
          "serve as well as HBM.", "",
          "cycles = traced duration x GHz, GHz = GRBM_GUI_ACTIVE/8 / counter-run duration for",
          "         dispatches of 100 us and more (else '-' and the nominal 2.4 GHz)",
          "mfma%  = MOPS_F32*512 / (256 CUs * 256 FLOP/clk * cycles)",
          "busy%  = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs * cycles)",
          "ldsc%  = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE",
          "wait%  = SQ_WAIT_ANY / SQ_WAVE_CYCLES",
          "lds/w  = SQ_INSTS_LDS per wave;  ratio = (rd + wr) / algorithmic bytes",
          "GB/s   = (rd + wr) / traced duration (HBM and Infinity Cache traffic)",
          "",
          f"{'config':10} {'kernel':24} {'us':>8} {'GHz':>5} {'mfma%':>6} {'busy%':>6} "
          f"{'ldsc%':>6} {'wait%':>6} {'lds/w':>7} {'rd_MiB':>8} {'wr_MiB':>8} {'alg_MiB':>8} "
          f"{'ratio':>6} {'GB/s':>7} {'%HBM':>6}"]
    for cfg in _present(d, "pmcB"):
        w = CONFIGS[cfg]
        ra = [r for r in counters(os.path.join(d, f"pmcA_{cfg}")) if is_ours(r["_name"])]
        rb = [r for r in counters(os.path.join(d, f"pmcB_{cfg}")) if is_ours(r["_name"])]
        fams = collections.OrderedDict()
        for r in ra:
            fams.setdefault(r["_name"], [[], []])[0].append(r)
        for r in rb:
            if r["_name"] in fams:
                fams[r["_name"]][1].append(r)
        if w.kind == "gemm":
            dom = traces[cfg][0]
            names = [dom] if dom in fams else list(fams)[:1]
        else:
            names = list(fams)
        tr = trace(os.path.join(d, f"trace_{cfg}"))
        for name in names:
            rows_a, rows_b = fams[name]
            if w.kind == "gemm":
                rows_a, rows_b = rows_a[-w.steps:], rows_b[-w.steps:]
            A = _mean_rows(rows_a, PASS_A)
            B = _mean_rows(rows_b, PASS_B)
            t_us = timed_mean([t for n, t in tr if n == name], w.steps)
            # Cycles of the kernel: its traced duration at the clock measured by
            # GRBM_GUI_ACTIVE over the counter run's dispatch when that lasts
            # 100 us or more, else at the nominal 2.4 GHz (for a few-us kernel
            # the GUI-active count also covers the dispatch around it).
            ghz = A["GRBM_GUI_ACTIVE"] / 8 / (A["_dur"] * 1e3) if A["_dur"] >= 100 else None
            cyc = t_us * 1e3 * (ghz or NOMINAL_GHZ)
            mfma = A["SQ_INSTS_VALU_MFMA_MOPS_F32"] * 512 / (CUS * FLOP_PER_CU_CLK * cyc)
            busy = B["SQ_VALU_MFMA_BUSY_CYCLES"] / (CUS * 4 * cyc)
            ldsc = B["SQ_LDS_BANK_CONFLICT"] / B["SQ_LDS_IDX_ACTIVE"] if B["SQ_LDS_IDX_ACTIVE"] else 0
            wait = A["SQ_WAIT_ANY"] / A["SQ_WAVE_CYCLES"] if A["SQ_WAVE_CYCLES"] else 0
            ldsw = B["SQ_INSTS_LDS"] / A["SQ_WAVES"] if A["SQ_WAVES"] else 0
            rd = A["FETCH_SIZE"] * cal.read_scale / 1024
            wr = B["WRITE_SIZE"] * cal.write_scale / 1024
            alg = flops_bytes(cfg)[1] / 2 ** 20 if w.kind == "gemm" else float("nan")
            gbs = (rd + wr) * 2 ** 20 / (t_us * 1e3)
            label = kernel_family(name)
            while label in results.get(cfg, {}):
                label += "'"  # same family, other instantiation (the MLP's two group launches)
            results.setdefault(cfg, {})[label] = dict(
                us=t_us, ghz=ghz, mfma=mfma, busy=busy, ldsc=ldsc, wait=wait, ldsw=ldsw, rd=rd,
                wr=wr, alg=alg, gbs=gbs, bytes=(rd + wr) * 2 ** 20)
            alg_s = f"{alg:8.2f} {(rd + wr) / alg:6.2f}" if alg == alg else f"{'-':>8} {'-':>6}"
            ghz_s = f"{ghz:5.2f}" if ghz else f"{'-':>5}"
            L.append(f"{cfg:10} {label[:24]:24} {t_us:8.2f} {ghz_s} "
                     f"{100 * mfma:6.1f} {100 * busy:6.1f} {100 * ldsc:6.2f} {100 * wait:6.1f} "
                     f"{ldsw:7.1f} {rd:8.2f} {wr:8.2f} {alg_s} {gbs:7.0f} "
                     f"{100 * gbs / PEAK_GBS:6.1f}")
    L.append("")
    _write("sgemm_configs_counters.txt", L)

    h = results["headline"]
    fam = next(iter(h))
    alg = flops_bytes("headline")[1]
    T = _header("HBM traffic per launch: sgemm_nn_4096 (bench.py headline workload)",
                [PMC_CMD.format(ctrs=" ".join(PASS_A), run="pmcA_headline", cfg="headline", s=50, w=40),
                 PMC_CMD.format(ctrs=" ".join(PASS_B), run="pmcB_headline", cfg="headline", s=50, w=40)])
    T += [f"kernel {fam}, mean over the 50 timed dispatches:",
          f"  FETCH_SIZE x{cal.read_scale:.3f} -> {h[fam]['rd']:.1f} MiB read",
          f"  WRITE_SIZE x{cal.write_scale:.3f} -> {h[fam]['wr']:.1f} MiB written",
          f"  algorithmic 4*(MK+KN+MN) = {alg / 2 ** 20:.1f} MiB; traffic / algorithmic = "
          f"{h[fam]['bytes'] / alg:.2f}",
          "  (each XCD's L2 fetches the A row-panels and B column-panels of its own tiles;",
          "   the Infinity Cache serves those re-reads)", "",
          f"traffic_bytes_per_launch: {h[fam]['bytes']:.0f}", ""]
    _write("sgemm_nn_4096_traffic.txt", T)
    return results


def _present(d: str, prefix: str) -> list[str]:
    """Configurations with a `prefix`_<config> run in d (and its trace), in ORDER."""
    return [c for c in ORDER if os.path.isdir(os.path.join(d, f"{prefix}_{c}")) and
            os.path.isdir(os.path.join(d, f"trace_{c}"))]


def _write(fname: str, lines: list[str]) -> None:
    os.makedirs(PROFILES, exist_ok=True)
    with open(os.path.join(PROFILES, fname), "w") as f:
        f.write("\n".join(lines))
    print(f"wrote profiles/{fname}", flush=True)


def summarize(d: str) -> None:
    traces = write_traces(d)
    if glob.glob(os.path.join(d, "vendor_*")):
        write_vendor(d)
    if glob.glob(os.path.join(d, "pmcA_*")):
        write_counters(d, traces)
