"""Benchmark of the fused-DAG hot path on one MI355X.

`python bench.py [--gpus 1] [--steps K] [--warmup W]` prints ONE JSON line.

Headline workload (`value`): config 2a, the fused row softmax region over
f32 [16384, 1024] logits ~ N(0, sigma=2); one step = one launch of the
softmax region over the whole tensor, inputs resident in HBM. Five
input/output buffer pairs (640 MiB) rotate so the 256 MB Infinity Cache
cannot hold the working set. Algorithmic bytes per launch = 16384*1024*4
read + the same written = 134 217 728 B; `value` = those bytes / the
average launch time, timed with HIP events recorded on the library stream
(the stream every launcher enqueues on) around exactly K launches.

`roofline.traffic` is the HBM bytes one softmax launch moves, from two
rocprofv3 --pmc runs of this script (FETCH_SIZE, then WRITE_SIZE), each
scaled by what the same counter reads for a plain 256 MiB relu map (a
read-once, write-once elementwise kernel of known size).

`kernels` reports every configuration the same way: GB/s against the 8 TB/s
HBM peak for bandwidth kernels, TFLOP/s against the dtype's MFMA peak for
GEMMs, ms / us end to end for the three programs. `cpu_baseline` times the C
oracle (the restated reference C lane, gcc -O2 -ffp-contract=off -fopenmp)
on the headline workload on this host; `kernels[*].cpu_ms` gives the same
oracle's time on a bounded sample of the other configurations.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
PEAK_TFLOPS = {"f32": 157.3, "f64": 78.6, "bf16": 2500.0}
METRIC = "per-kernel GB/s & GFLOP/s (% roofline); transformer-block fwd ms at 1 GPU"
SOFTMAX_ROWS, SOFTMAX_N = 16384, 1024
COPY_ELEMS = 64 * 1024 * 1024  # f32 relu map used to calibrate the HBM counters


def host_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except Exception:
        return os.cpu_count() or 1


def time_launches(C, H, launch, steps: int, warmup: int) -> float:
    """Average ms per launch of `launch(i)` over `steps` launches, HIP events
    on the library stream."""
    stream = C.lib().chelis_hip_stream()
    for i in range(warmup):
        launch(i)
    C.synchronize()
    start, end = H.Event(), H.Event()
    start.record(stream)
    for i in range(steps):
        launch(i)
    end.record(stream)
    end.synchronize()
    return start.elapsed_ms(end) / steps


def softmax_inputs():
    return (np.random.default_rng(10).standard_normal((SOFTMAX_ROWS, SOFTMAX_N)) * 2).astype(np.float32)


def bench_softmax_f32(C, H, steps, warmup):
    nbytes = SOFTMAX_ROWS * SOFTMAX_N * 4 * 2
    x = softmax_inputs()
    pairs = [(C.to_device(x), C.empty(x.shape, np.float32)) for _ in range(5)]
    ms = time_launches(C, H, lambda i: C.softmax(pairs[i % 5][0], pairs[i % 5][1]), steps, warmup)
    return {"ms": ms, "bytes": nbytes, "gbps": nbytes / (ms * 1e-3) / 1e9}, x


def bench_softmax_f64(C, H, steps, warmup):
    nbytes = 4096 * 4096 * 8 * 2
    x = np.random.default_rng(11).standard_normal((4096, 4096))
    pairs = [(C.to_device(x), C.empty(x.shape, np.float64)) for _ in range(3)]
    ms = time_launches(C, H, lambda i: C.softmax(pairs[i % 3][0], pairs[i % 3][1]), steps, warmup)
    return {"ms": ms, "bytes": nbytes, "gbps": nbytes / (ms * 1e-3) / 1e9}, x


def bench_gemm(C, H, M, N, K, dtype, seeds, steps, warmup, reps=1):
    """C = A.B with A, B ~ U(-1, 1); `reps` operand sets rotate when the
    working set would otherwise sit in the 256 MB Infinity Cache."""
    a = np.random.default_rng(seeds[0]).uniform(-1, 1, (M, K)).astype(np.float32 if dtype == "bf16" else dtype)
    b = np.random.default_rng(seeds[1]).uniform(-1, 1, (K, N) if N > 1 else (K,)).astype(a.dtype)
    if dtype == "bf16":
        # bf16 operands as bit patterns: the upper halves, rounded to nearest even
        a, b = [((x.view(np.uint32) + 0x7FFF + ((x.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
                for x in (a, b)]
        dtype = np.uint16
    sets = [(C.to_device(a), C.to_device(b)) for _ in range(reps)]
    outs = [C.matmul(da, db) for da, db in sets]
    ms = time_launches(C, H, lambda i: C.matmul(sets[i % reps][0], sets[i % reps][1], outs[i % reps]), steps, warmup)
    isz = np.dtype(dtype).itemsize
    nbytes = (M * K + K * N + M * N) * isz
    flops = 2 * M * N * K
    return {"ms": ms, "bytes": nbytes, "flops": flops, "gbps": nbytes / (ms * 1e-3) / 1e9,
            "tflops": flops / (ms * 1e-3) / 1e12}, (a, b)


def gemm_line(r, dt, bound):
    return {"ms": round(r["ms"], 5), "TFLOP/s": round(r["tflops"], 2), "GB/s": round(r["gbps"], 1),
            "frac_mfma": round(r["tflops"] / PEAK_TFLOPS[dt], 4), "frac_hbm": round(r["gbps"] / HBM_PEAK_GBPS, 4),
            "bound": bound}


def linreg_data():
    X = np.random.default_rng(1).standard_normal((8192, 32))
    w = np.random.default_rng(2).standard_normal(32)
    y = X @ w + np.random.default_rng(3).normal(0, 0.01, 8192)
    return X, w, y


def transformer_data(B=8, S=512, D=1024, F=4096):
    x = np.random.default_rng(30).standard_normal((B, S, D)).astype(np.float32)
    p = {}
    seeds = iter(range(31, 37))
    for name, shape in (("wq", (D, D)), ("wk", (D, D)), ("wv", (D, D)), ("wo", (D, D)), ("w1", (D, F)),
                        ("w2", (F, D))):
        p[name] = (np.random.default_rng(next(seeds)).standard_normal(shape) * 0.02).astype(np.float32)
    for name, n in (("bq", D), ("bk", D), ("bv", D), ("bo", D), ("b1", F), ("b2", D), ("ln1_b", D), ("ln2_b", D)):
        p[name] = np.zeros(n, np.float32)
    p["ln1_g"] = np.ones(D, np.float32)
    p["ln2_g"] = np.ones(D, np.float32)
    return x, p


PARAM_ORDER = ("ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "ln2_g", "ln2_b", "w1", "b1", "w2",
               "b2")


def mlp_data(B=1024, I=784, Hd=512, O=10):
    x = np.random.default_rng(40).uniform(0, 1, (B, I)).astype(np.float32)
    labels = np.random.default_rng(41).integers(0, O, B)
    onehot = np.eye(O, dtype=np.float32)[labels]
    w1 = (np.random.default_rng(42).standard_normal((I, Hd)) * np.sqrt(2 / I)).astype(np.float32)
    w2 = (np.random.default_rng(43).standard_normal((Hd, O)) * np.sqrt(2 / Hd)).astype(np.float32)
    return x, onehot, w1, np.zeros(Hd, np.float32), w2, np.zeros(O, np.float32)


TRANSFORMER_FLOPS = 111_669_149_696  # QKV + scores + PV + out + FFN, 2 flops per MAC
MLP_FLOPS = 1_675_624_448
LINREG_BYTES = 2_163_208


def bench_programs(C, H, steps, warmup):
    out = {}
    X, w, y = linreg_data()
    ins = [C.to_device(a) for a in (X, w, y)]
    outs = [C.empty((32,), np.float64), C.empty((), np.float64)]
    ms = time_launches(C, H, lambda i: C.program("linreg_step", ins, outs), steps, warmup)
    out["linreg_step_f64_8192x32"] = {"us": round(ms * 1e3, 2), "GB/s": round(LINREG_BYTES / (ms * 1e-3) / 1e9, 1),
                                      "frac_hbm": round(LINREG_BYTES / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                                      "bound": "launch latency (2 MB working set)"}
    x, p = transformer_data()
    tins = [C.to_device(x)] + [C.to_device(p[k]) for k in PARAM_ORDER]
    ty = C.empty(x.shape, np.float32)
    tsteps = max(3, steps // 5)
    ms = time_launches(C, H, lambda i: C.program("transformer_block", tins, [ty]), tsteps, 2)
    out["transformer_block_f32_b8_s512_d1024"] = {
        "ms": round(ms, 4), "TFLOP/s": round(TRANSFORMER_FLOPS / (ms * 1e-3) / 1e12, 2),
        "frac_mfma": round(TRANSFORMER_FLOPS / (ms * 1e-3) / 1e12 / PEAK_TFLOPS["f32"], 4)}
    del tins, ty
    args = mlp_data()
    mins = [C.to_device(a) for a in args] + [C.key_tensor(44)]
    mouts = [C.empty((), np.float32), C.empty(args[2].shape, np.float32), C.empty(args[3].shape, np.float32),
             C.empty(args[4].shape, np.float32), C.empty(args[5].shape, np.float32)]
    ms = time_launches(C, H, lambda i: C.program("mlp_train_step", mins, mouts), steps, warmup)
    out["mlp_train_step_f32_1024x784x512x10"] = {
        "us": round(ms * 1e3, 2), "TFLOP/s": round(MLP_FLOPS / (ms * 1e-3) / 1e12, 3),
        "bound": "launch latency (21 small launches)"}
    return out, (X, w, y), (x, p), args


# ---------------------------------------------------------------- bandwidth families
def bench_bandwidth(C, H, steps, warmup):
    """The memory-bound region families at HBM-sized shapes (the config
    programs hold them only at launch-bound sizes): GB/s of algorithmic bytes
    (every operand read once, every result written once) against the 8 TB/s
    peak. Three buffer sets of 256 MiB rotate, so the 256 MB Infinity Cache
    cannot hold the working set."""
    out = {}
    rng = np.random.default_rng(50)
    R, N = 16384, 4096
    x = rng.standard_normal((R, N)).astype(np.float32)
    nb = x.nbytes
    X = [C.to_device(x) for _ in range(3)]
    G = [C.to_device(x) for _ in range(3)]
    Y = [C.empty(x.shape, np.float32) for _ in range(3)]

    def line(name, launch, nbytes, bound="hbm"):
        ms = time_launches(C, H, launch, steps, warmup)
        gbps = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 2), "GB/s": round(gbps, 1), "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4),
                     "bytes": nbytes, "bound": bound}

    line("relu_f32_16384x4096", lambda i: C.relu(X[i % 3], Y[i % 3]), 2 * nb)
    line("relu_adjoint_f32_16384x4096", lambda i: C.relu_adjoint(X[i % 3], G[i % 3], Y[i % 3]), 3 * nb)
    line("dropout_f32_16384x4096", lambda i: C.dropout(44, X[i % 3], 0.1, Y[i % 3]), 2 * nb,
         "VALU (splitmix64 64-bit multiplies per element)")
    line("gelu_f32_16384x4096", lambda i: C.gelu(X[i % 3], Y[i % 3]), 2 * nb,
         "VALU (correctly rounded exp and erfc leaves)")
    sq = C.fused_chain([("sub", 0, 1), ("mul", ("s", 0), ("s", 0))])
    line("fused_chain_sqdiff_f32_16384x4096", lambda i: C.fused_elementwise(sq, [X[i % 3], G[i % 3]], Y[i % 3]),
         3 * nb)
    S1 = [C.empty((R,), np.float32) for _ in range(3)]
    line("reduce_sum_rows_f32_16384x4096", lambda i: C.reduce("sum", X[i % 3], 1, S1[i % 3]), nb + R * 4)
    line("reduce_max_rows_f32_16384x4096", lambda i: C.reduce("max", X[i % 3], 1, S1[i % 3]), nb + R * 4)
    line("reduce_sum_sqdiff_rows_f32_16384x4096",
         lambda i: C.reduce("sum", [X[i % 3], G[i % 3]], 1, S1[i % 3], chain=sq), 2 * nb + R * 4)
    S0 = [C.empty((N,), np.float32) for _ in range(3)]
    line("reduce_sum_cols_f32_16384x4096", lambda i: C.reduce("sum", X[i % 3], 0, S0[i % 3]), nb + N * 4)
    del X, G, Y
    b = rng.random((R, N)) < 0.9
    B = [C.to_device(b) for _ in range(3)]
    I1 = [C.empty((R,), np.int64) for _ in range(3)]
    line("count_bool_rows_16384x4096", lambda i: C.count(B[i % 3], 1, I1[i % 3]), b.nbytes + R * 8,
         "host round trip (the call returns the error code synchronously)")
    del B
    xs = rng.standard_normal((65536, 1024)).astype(np.float32)
    XS = [C.to_device(xs) for _ in range(3)]
    YS = [C.empty(xs.shape, np.float32) for _ in range(3)]
    gam, bet = C.to_device(np.ones(1024, np.float32)), C.to_device(np.zeros(1024, np.float32))
    line("layer_norm_f32_65536x1024", lambda i: C.layer_norm(XS[i % 3], gam, bet, 1e-5, YS[i % 3]), 2 * xs.nbytes)
    line("softmax_f32_65536x1024", lambda i: C.softmax(XS[i % 3], YS[i % 3]), 2 * xs.nbytes)
    sm = C.softmax(XS[0])
    line("softmax_adjoint_f32_65536x1024", lambda i: C.softmax_adjoint(sm, XS[(i + 1) % 3], YS[i % 3]),
         3 * xs.nbytes)
    return out


# ---------------------------------------------------------------- traffic
def traffic_child():
    """Runs under rocprofv3 --pmc: 10 headline softmax launches and 10
    launches of the relu map used as the calibration copy."""
    import chelis_amd as C

    x = softmax_inputs()
    pairs = [(C.to_device(x), C.empty(x.shape, np.float32)) for _ in range(5)]
    src = C.to_device(np.abs(np.random.default_rng(5).standard_normal(COPY_ELEMS)).astype(np.float32))
    dst = C.empty((COPY_ELEMS,), np.float32)
    for i in range(10):
        C.softmax(pairs[i % 5][0], pairs[i % 5][1])
    for _ in range(10):
        C.relu(src, dst)
    C.synchronize()


def _counter_rows(outdir):
    files = glob.glob(os.path.join(outdir, "**", "*counter_collection*.csv"), recursive=True)
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def measure_traffic(timeout_s=120):
    """HBM bytes per softmax launch from FETCH_SIZE and WRITE_SIZE, each
    scaled by the relu calibration map; None when rocprofv3 is unavailable."""
    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(prof):
        return None, "rocprofv3 not found"
    per = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        outdir = tempfile.mkdtemp(prefix="chelis_pmc_")
        try:
            cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", outdir, "-o", "pmc", "--",
                   sys.executable, os.path.abspath(__file__), "--traffic-child"]
            r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout_s)
            rows = _counter_rows(outdir)
            if not rows:
                return None, f"rocprofv3 --pmc {counter} produced no counter rows (rc {r.returncode})"
            vals = {"softmax": [], "relu": []}
            for row in rows:
                name = row.get("Kernel_Name", "")
                if row.get("Counter_Name", counter) != counter:
                    continue
                v = float(row.get("Counter_Value", "nan"))
                if "softmax_kernel" in name:
                    vals["softmax"].append(v)
                elif "unary_kernel" in name:
                    vals["relu"].append(v)
            if not vals["softmax"] or not vals["relu"]:
                return None, f"{counter}: kernels not found in the counter rows"
            per[counter] = {k: float(np.median(v)) for k, v in vals.items()}
        finally:
            shutil.rmtree(outdir, ignore_errors=True)
    copy_bytes = COPY_ELEMS * 4
    f_scale = copy_bytes / per["FETCH_SIZE"]["relu"]
    w_scale = copy_bytes / per["WRITE_SIZE"]["relu"]
    fetch = per["FETCH_SIZE"]["softmax"] * f_scale
    write = per["WRITE_SIZE"]["softmax"] * w_scale
    detail = {"fetch_bytes": round(fetch), "write_bytes": round(write),
              "raw_kib": {"fetch_softmax": per["FETCH_SIZE"]["softmax"], "write_softmax": per["WRITE_SIZE"]["softmax"],
                          "fetch_copy": per["FETCH_SIZE"]["relu"], "write_copy": per["WRITE_SIZE"]["relu"]},
              "scale": {"fetch": round(f_scale, 3), "write": round(w_scale, 3)},
              "calibration": f"relu map of {copy_bytes} B read + {copy_bytes} B written"}
    return fetch + write, detail


# ---------------------------------------------------------------- CPU baselines
def _time_cpu(fn, budget_s, max_runs=20):
    fn()
    runs, t0 = 0, time.perf_counter()
    while True:
        fn()
        runs += 1
        el = time.perf_counter() - t0
        if el > budget_s or runs >= max_runs:
            return el / runs, runs


def cpu_baselines(x_softmax, kernels, linreg, transformer, mlp, gemm_inputs):
    from oracle import oracle as O

    O.build()
    cores = host_cores()
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    threads = int(os.environ["OMP_NUM_THREADS"])
    per, runs = _time_cpu(lambda: O.softmax_rows(x_softmax), 10.0)
    head = {"value": round(x_softmax.nbytes * 2 / per / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the full config 2a tensor [16384,1024] f32, {runs} runs of the oracle softmax "
                      f"(gcc -O2 -ffp-contract=off -fopenmp, CORE-MATH expf), {per * 1e3:.1f} ms per run"}
    X, w, y = linreg
    t, _ = _time_cpu(lambda: O.linreg_step(X, w, y), 2.0)
    kernels["linreg_step_f64_8192x32"]["cpu_ms"] = round(t * 1e3, 3)
    a, b = gemm_inputs["f32"]
    t, _ = _time_cpu(lambda: O.matmul(np.ascontiguousarray(a[:128]), b), 3.0, 3)
    kernels["gemm_f32_4096^3"]["cpu_ms"] = round(t * 1e3 * 32, 1)
    a, b = gemm_inputs["f64"]
    t, _ = _time_cpu(lambda: O.matmul(np.ascontiguousarray(a[:128]), b), 3.0, 3)
    kernels["gemm_f64_4096^3"]["cpu_ms"] = round(t * 1e3 * 32, 1)
    a, b = gemm_inputs["skinny"]
    t, _ = _time_cpu(lambda: O.matmul(np.ascontiguousarray(a[:1024]), b), 3.0, 5)
    kernels["skinny_f64_8192x64x4096"]["cpu_ms"] = round(t * 1e3 * 8, 2)
    a, b = gemm_inputs["gemv"]
    t, _ = _time_cpu(lambda: O.matmul(a, b.reshape(-1, 1)), 3.0, 5)
    kernels["gemv_f64_8192x8192"]["cpu_ms"] = round(t * 1e3, 2)
    xs, p = transformer
    t, _ = _time_cpu(lambda: O.transformer_block(np.ascontiguousarray(xs[:1]), p, 16), 5.0, 2)
    kernels["transformer_block_f32_b8_s512_d1024"]["cpu_ms"] = round(t * 1e3 * 8, 1)
    t, _ = _time_cpu(lambda: O.mlp_train_step(*mlp, 44, np.float32(0.1), np.float32(0.01)), 3.0, 5)
    kernels["mlp_train_step_f32_1024x784x512x10"]["cpu_ms"] = round(t * 1e3, 2)
    kernels["_cpu_note"] = (f"C oracle on {threads} host threads; GEMM 4096^3 timed on 128 rows x32, skinny on "
                            f"1024 rows x8, transformer on batch 1 x8; others full size")
    x64 = kernels.pop("_softmax_f64_input", None)
    if x64 is not None:
        t, _ = _time_cpu(lambda: O.softmax_rows(x64), 5.0, 5)
        kernels["softmax_f64_4096x4096"]["cpu_ms"] = round(t * 1e3, 2)
    return head


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 --pmc traffic runs")
    ap.add_argument("--only-headline", action="store_true")
    ap.add_argument("--traffic-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args(argv)
    if args.traffic_child:
        traffic_child()
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "how the path would shard is described in DESIGN.md, not run.", file=sys.stderr)
        return 2

    import chelis_amd as C
    from chelis_amd import hiprt as H

    C.lib()
    head, x = bench_softmax_f32(C, H, args.steps, args.warmup)
    kernels = {"softmax_f32_16384x1024": {"ms": round(head["ms"], 5), "GB/s": round(head["gbps"], 1),
                                          "frac_hbm": round(head["gbps"] / HBM_PEAK_GBPS, 4)}}
    extra = None
    if not args.only_headline:
        s64, x64 = bench_softmax_f64(C, H, max(5, args.steps // 2), args.warmup)
        kernels["softmax_f64_4096x4096"] = {"ms": round(s64["ms"], 5), "GB/s": round(s64["gbps"], 1),
                                            "frac_hbm": round(s64["gbps"] / HBM_PEAK_GBPS, 4)}
        gs = max(3, args.steps // 5)
        # as many untimed launches as the other measurements get, so the
        # timed GEMMs run at the clocks a sustained load settles at
        gw = max(2, args.warmup)
        gin = {}
        r, gin["f32"] = bench_gemm(C, H, 4096, 4096, 4096, np.float32, (20, 21), gs, gw)
        kernels["gemm_f32_4096^3"] = gemm_line(r, "f32", "mfma")
        r, gin["f64"] = bench_gemm(C, H, 4096, 4096, 4096, np.float64, (22, 23), gs, gw)
        kernels["gemm_f64_4096^3"] = gemm_line(r, "f64", "mfma")
        r, gin["skinny"] = bench_gemm(C, H, 8192, 64, 4096, np.float64, (24, 25), gs, gw, reps=2)
        kernels["skinny_f64_8192x64x4096"] = gemm_line(r, "f64", "valu canonical tree (bit-exact)")
        r, gin["gemv"] = bench_gemm(C, H, 8192, 1, 8192, np.float64, (26, 27), gs, gw, reps=2)
        kernels["gemv_f64_8192x8192"] = gemm_line(r, "f64", "hbm")
        # bf16 (np.uint16 bit patterns) with the binary32 accumulator
        r, _ = bench_gemm(C, H, 4096, 4096, 4096, "bf16", (28, 29), gs, gw)
        kernels["gemm_bf16_4096^3"] = gemm_line(r, "bf16", "mfma")
        progs, lin, tr, mlp = bench_programs(C, H, max(5, args.steps // 2), args.warmup)
        kernels.update(progs)
        kernels.update(bench_bandwidth(C, H, max(5, args.steps // 2), args.warmup))
        extra = (x64, lin, tr, mlp, gin)
    traffic, tdetail = (None, "skipped") if args.no_traffic else measure_traffic()
    cpu = None
    if not args.no_cpu:
        if extra is not None:
            x64, lin, tr, mlp, gin = extra
            kernels["_softmax_f64_input"] = x64
            cpu = cpu_baselines(x, kernels, lin, tr, mlp, gin)
        else:
            from oracle import oracle as O

            O.build()
            os.environ.setdefault("OMP_NUM_THREADS", str(host_cores()))
            per, runs = _time_cpu(lambda: O.softmax_rows(x), 10.0)
            cpu = {"value": round(x.nbytes * 2 / per / 1e9, 3), "unit": "GB/s",
                   "cores": int(os.environ["OMP_NUM_THREADS"]), "kind": "port",
                   "sample": f"the full config 2a tensor, {runs} runs of the oracle softmax, {per * 1e3:.1f} ms/run"}
    line = {
        "metric": METRIC,
        "value": round(head["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: N(0, sigma=2) logits from numpy seed 10, resident in HBM, 5 rotating buffer pairs",
        "config": {"workload": "config 2a: fused row softmax f32 [16384,1024] (max, sub, exp, tree sum, div)",
                   "rows": SOFTMAX_ROWS, "row_len": SOFTMAX_N, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(head["gbps"], 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(head["gbps"] / HBM_PEAK_GBPS, 4),
                     "traffic": None if traffic is None else int(round(traffic)),
                     "algorithmic_bytes": head["bytes"],
                     "traffic_detail": tdetail},
        "cpu_baseline": cpu,
        "kernels": kernels,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
