"""Benchmark of cleave's tensor hot path on one MI355X.

Headline: f32 GEMM C = A B, M = N = K = 4096,
row-major, N(0,1) inputs generated on the device.  One step = one
cleave_hip_matmul_f32 call; inputs are resident in HBM before timing starts.

Prints ONE JSON line on stdout:
  value        aggregate GFLOP/s of the timed steps (2*M*N*K per step, wall clock
               between two stream synchronisations)
  roofline     the GEMM kernel's achieved TFLOP/s from HIP events recorded on the
               library stream around the timed launches, vs 157.3 TFLOP/s FP32 MFMA
  cpu_baseline the oracle's reference-faithful i-j-k loop, one core, on a row band
               of the same product, extrapolated to GFLOP/s
  secondary    the other BASELINE configs (f32 256^3, bf16 8192^3, batched bf16,
               f32 A B^T / A^T B, MLP steps/s, escape-count map, u64 count sum), the
               config-2 product on Tensor<f64> (vs 78.6 TFLOP/s FP64 MFMA), the
               MLP step through the reverse-mode tape, a matrix-vector product, and
               the maps, reductions, row-broadcast bias and general broadcasting, each with its own
               HIP-event roofline figure and (unless --no-cpu) a single-core CPU
               baseline from the restated loops on a bounded sample
  vendor_same_device
               (--vendor only) torch.matmul / torch.bmm on the GEMM shapes, timed the
               same way in a child process on the same device (with --gemm: on
               those specs, beside each spec's own figures)
Progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_FP32_MFMA = 157.3  # TFLOP/s, MI355X dense FP32 matrix
PEAK_BF16_MFMA = 2516.6  # TFLOP/s, MI355X dense BF16 matrix
PEAK_FP64_MFMA = 78.6  # TFLOP/s, MI355X dense FP64 matrix
MANDEL_VALU_PER_ITER = 8  # 7 arithmetic (2p + ci as one exact fma) + the escape compare, per iteration
PEAK_FP32_VALU_NOFMA = 78.6  # T op/s: MI355X FP32 vector peak 157.3 TFLOP/s counts an FMA as 2; one non-FMA op per lane-cycle is half
PEAK_HBM = 8000.0  # GB/s
HEADLINE_WARM_S = 0.4  # seconds of sustained load before the headline's timed steps


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def timed(ca, fn, steps, warmup, warm_s=0.0):
    """Run fn `warmup` times (and further until `warm_s` seconds have passed),
    then time `steps` calls: wall clock between two stream syncs, and HIP
    events on the library stream.  MI355X clocks settle only after ~0.1-0.3 s
    of sustained matrix-core load, so short warm-ups under-report."""
    for _ in range(warmup):
        fn()
    ca.sync()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < warm_s:
        for _ in range(4):
            fn()
        ca.sync()
    t = ca.Timer()
    w0 = time.perf_counter()
    t.start()
    for _ in range(steps):
        fn()
    ev_ms = t.stop()
    ca.sync()
    wall = time.perf_counter() - w0
    return wall, ev_ms / steps


def vendor_yardstick(steps):
    """torch.matmul / torch.bmm (hipBLASLt or rocBLAS underneath) on the bench's
    GEMM shapes and data distributions, timed the same way on the same device.
    bf16 matrix-core throughput is power-limited and differs from chip to chip,
    so a vendor figure from the same box is the fair reference point.  The
    vendor bf16 products write bf16 C (half the bytes of this library's f32 C).
    Runs in a process of its own: torch brings its own HIP runtime, which sees
    no device once this library's runtime holds it in the same process."""
    import torch

    torch.backends.cuda.matmul.allow_tf32 = False
    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    out = {}

    def run(name, fn, flop, warm_s):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < warm_s:
            for _ in range(4):
                fn()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        out[name] = {"kernel_ms": round(ms, 4), "TFLOP/s": round(flop / (ms * 1e-3) / 1e12, 1)}
        log(f"vendor {name}: {out[name]['TFLOP/s']} TFLOP/s")

    n = 4096
    a = torch.randn(n, n, device=dev, generator=g)
    b = torch.randn(n, n, device=dev, generator=g)
    c = torch.empty(n, n, device=dev)
    run("gemm_f32_nn_4096", lambda: torch.matmul(a, b, out=c), 2.0 * n ** 3, 0.3)
    del a, b, c
    m = 8192
    ab = (torch.randn(m, m, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    bb = (torch.randn(m, m, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    cb = torch.empty(m, m, device=dev, dtype=torch.bfloat16)
    run("gemm_bf16_8192", lambda: torch.matmul(ab, bb, out=cb), 2.0 * m ** 3, 0.4)
    del ab, bb, cb
    bs, k = 64, 512
    x = (torch.randn(bs, k, k, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    y = (torch.randn(bs, k, k, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    z = torch.empty(bs, k, k, device=dev, dtype=torch.bfloat16)
    run("gemm_bf16_batched_64x512", lambda: torch.bmm(x, y, out=z), 2.0 * bs * k ** 3, 0.3)
    del x, y, z
    torch.cuda.synchronize()
    return out


def vendor_shapes(specs, steps):
    """torch.matmul / torch.bmm on the --gemm specs, timed like gemm_shapes
    (0.3 s warm-up, then HIP events), in the --vendor child process.  bf16
    products are timed as torch returns them (bf16 C, half the bytes this
    library writes) and, where this torch build has it, with f32 C
    (out_dtype=torch.float32: the same bytes as here).  2-D products take the
    spec's layout as transposed views; batched bf16 products are timed with
    contiguous operands in every layout (torch.bmm on a transposed bf16 view
    is avoided on these boxes)."""
    import torch

    torch.backends.cuda.matmul.allow_tf32 = False
    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    out = {}

    def clock(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 0.3:
            for _ in range(4):
                fn()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    for spec in specs:
        dt, dims, lay = spec.split(":")
        d = [int(x) for x in dims.split("x")]
        bs, (m, n, k) = (d[0], d[1:]) if len(d) == 4 else (1, d)
        batched = len(d) == 4
        ta, tb = lay[0] == "t", lay[1] == "t"
        tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f64": torch.float64}[dt]
        lead = (bs,) if batched else ()
        if batched:
            a = torch.randn(lead + (m, k), device=dev, generator=g).to(tdt)
            b = torch.randn(lead + (k, n), device=dev, generator=g).to(tdt)
            opa, opb = a, b
        else:
            a = torch.randn((k, m) if ta else (m, k), device=dev, generator=g).to(tdt)
            b = torch.randn((n, k) if tb else (k, n), device=dev, generator=g).to(tdt)
            opa, opb = (a.t() if ta else a), (b.t() if tb else b)
        mm = torch.bmm if batched else torch.mm
        c = torch.empty(lead + (m, n), device=dev, dtype=tdt)
        ms = clock(lambda: mm(opa, opb, out=c))
        rec = {"torch_ms": round(ms, 5)}
        if dt == "bf16":
            try:
                mm(opa, opb, out_dtype=torch.float32)
                rec["torch_f32_out_ms"] = round(clock(lambda: mm(opa, opb, out_dtype=torch.float32)), 5)
            except (RuntimeError, TypeError) as e:
                rec["torch_f32_out_ms"] = None
                rec["torch_f32_out_error"] = str(e).splitlines()[0][:160]
        out[spec] = rec
        log(f"vendor {spec}: {ms * 1e3:.1f} us")
        del a, b, c, opa, opb
        torch.cuda.synchronize()
    return out


def read_traffic(name):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if any."""
    p = ROOT / "profiles" / f"{name}_traffic.md"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def cpu_info():
    model = platform.processor() or ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count()


def cpu_baseline_gemm(A, B, n, budget_s):
    """Reference-faithful loop (oracle/oracle.c or_matmul_f32_rows), one core."""
    from oracle import oracle as orc

    t0 = time.perf_counter()
    orc.matmul_rows(A, B, n, n, n, 0, 1)
    one = time.perf_counter() - t0
    rows = max(1, min(n, int(budget_s / max(one, 1e-6))))
    t0 = time.perf_counter()
    orc.matmul_rows(A, B, n, n, n, 1, 1 + rows)
    dt = time.perf_counter() - t0
    gflops = 2.0 * rows * n * n / dt / 1e9
    model, ncpu = cpu_info()
    return {
        "value": round(gflops, 4),
        "unit": "GFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"rows 1..{rows} of the 4096^3 NN product through the restated "
                   f"k-ascending loop (gcc -O2 -ffp-contract=off), {dt:.1f} s, extrapolated "
                   f"linearly in M; host: {model}, {ncpu} logical CPUs"),
    }


def _cpu_entry(value, unit, sample):
    model, ncpu = cpu_info()
    return {"value": value, "unit": unit, "cores": 1, "kind": "port",
            "sample": f"{sample}; host: {model}, {ncpu} logical CPUs"}


def _timed_cpu(fn):
    t0 = time.perf_counter()
    r = fn()
    return time.perf_counter() - t0, r


def cpu_rows(run_rows, total_rows, budget_s):
    """Time a 1-row probe, then as many further rows as fit in budget_s; returns
    (rows timed, seconds).  run_rows(r0, r1) computes rows [r0, r1)."""
    one, _ = _timed_cpu(lambda: run_rows(0, 1))
    rows = max(1, min(total_rows - 1, int(budget_s / max(one, 1e-6))))
    dt, _ = _timed_cpu(lambda: run_rows(1, 1 + rows))
    return rows, dt


def cpu_secondary(orc, name, budget_s, **kw):
    """Single-core restated loop (oracle/) on a bounded sample of a secondary
    workload, extrapolated to the full workload's unit."""
    import numpy as np
    if name == "gemm_f32_256":
        A, B, n = kw["A"], kw["B"], kw["n"]
        reps, dt = 0, 0.0
        while dt < min(budget_s, 1.0) or reps < 3:  # the whole product, repeated
            t, _ = _timed_cpu(lambda: orc.matmul(A, B))
            dt += t
            reps += 1
        return _cpu_entry(round(2.0 * n ** 3 * reps / dt / 1e9, 4), "GFLOP/s",
                          f"the whole {n}^3 product through the restated k-ascending loop, {reps} times, "
                          f"{dt:.2f} s")
    if name in ("gemm_f32_nt_4096", "gemm_f32_tn_4096"):
        A, B, n, ta, tb = kw["A"], kw["B"], kw["n"], kw["ta"], kw["tb"]
        rows, dt = cpu_rows(lambda r0, r1: orc.matmul_rows(A, B, n, n, n, r0, r1, ta, tb), n, budget_s)
        return _cpu_entry(round(2.0 * rows * n * n / dt / 1e9, 4), "GFLOP/s",
                          f"rows 1..{rows} of the {n}^3 product, restated k-ascending loop, {dt:.1f} s")
    if name == "gemm_f64_4096":
        A, B, n = kw["A"], kw["B"], kw["n"]
        rows, dt = cpu_rows(lambda r0, r1: orc.matmul_f64_rows(A, B, n, n, n, r0, r1), n, budget_s)
        return _cpu_entry(round(2.0 * rows * n * n / dt / 1e9, 4), "GFLOP/s",
                          f"rows 1..{rows} of the {n}^3 f64 product, restated k-ascending loop, {dt:.1f} s")
    if name == "gemm_bf16_8192":
        A, B, m = kw["A"], kw["B"], kw["m"]
        rows, dt = cpu_rows(lambda r0, r1: orc.matmul_bf16_rows(A, B, m, m, m, r0, r1), m, budget_s)
        return _cpu_entry(round(2.0 * rows * m * m / dt / 1e9, 4), "GFLOP/s",
                          f"rows 1..{rows} of the {m}^3 product on upcast bf16, restated f32 loop, {dt:.1f} s")
    if name == "gemm_bf16_batched_64x512":
        A, B, bs, k = kw["A"], kw["B"], kw["bs"], kw["k"]
        rows, dt = cpu_rows(lambda r0, r1: orc.matmul_bf16_rows(A, B, k, k, k, r0, r1), k, budget_s)
        return _cpu_entry(round(2.0 * rows * k * k / dt / 1e9, 4), "GFLOP/s",
                          f"rows 1..{rows} of product 0 of {bs}, restated f32 loop on upcast bf16, {dt:.1f} s")
    if name == "matvec_f32_65536x4096":
        A, x, m, k = kw["A"], kw["x"], kw["m"], kw["k"]
        rows, dt = cpu_rows(lambda r0, r1: orc.matmul_rows(A, x, m, 1, k, r0, r1, False, False), m, budget_s)
        return _cpu_entry(round(rows * k * 4 / dt / 1e9, 4), "GB/s",
                          f"rows 1..{rows} of the {m} x {k} matrix against the vector, restated k-ascending "
                          f"loop, {dt:.2f} s (matrix bytes per second)")
    if name == "mlp_step_65536x1024x4096":
        X, y, W1, W2, B_ = kw["X"], kw["y"], kw["W1"], kw["W2"], kw["B"]
        # a step costs f (the SGD update, batch-independent) + rows * r; two
        # batch sizes give both, and the full step is f + B * r
        t2, _ = _timed_cpu(lambda: orc.mlp_step(X[:2], y[:2], W1, W2, 0.01))
        bs = int(max(4, min(X.shape[0], 1024, 2 * budget_s / max(t2, 1e-6))))
        dt, _ = _timed_cpu(lambda: orc.mlp_step(X[:bs], y[:bs], W1, W2, 0.01))
        r = max((dt - t2) / (bs - 2), 1e-12)
        f = max(t2 - 2 * r, 0.0)
        full = f + B_ * r
        return _cpu_entry(round(1.0 / full, 6), "steps/s",
                          f"steps on batch rows 0..1 ({t2:.2f} s) and 0..{bs - 1} ({dt:.1f} s) of {B_} "
                          f"(forward, backward, SGD), fitted as fixed + per-row cost: {full:.0f} s per full step")
    if name == "mandelbrot_16384_1000":
        g, d, total = kw["g"], kw["d"], kw["total"]
        mid, band = g // 2, 2
        while True:  # widen a centred band of rows until it costs at least budget_s / 4
            dt, out = _timed_cpu(lambda: orc.mandelbrot(g, g, -2.0, -1.5, d, d, 1000, rows=(mid - band, mid + band)))
            if dt > budget_s / 4 or 2 * band >= g // 4:
                break
            band *= 2
        it = float(out[mid - band:mid + band].astype(np.uint64).sum())
        rate = it / dt
        return _cpu_entry(round(rate, 1), "pixel-iter/s",
                          f"rows {mid - band}..{mid + band - 1} (the set's widest band), {dt:.1f} s; "
                          f"the full grid's {total} counted iterations would take {total / rate:.0f} s")
    arr_n = kw.get("n", 1 << 24)
    rng = np.random.default_rng(7)
    if name == "sum_u32_u64_16384sq":
        v = rng.integers(0, 1000, arr_n, dtype=np.uint32)
        dt, _ = _timed_cpu(lambda: orc.sum_u64(v))
        return _cpu_entry(round(arr_n * 4 / dt / 1e9, 3), "GB/s", f"{arr_n} u32 counts summed into u64, {dt * 1e3:.0f} ms")
    v = rng.standard_normal(arr_n).astype(np.float32)
    if name == "sigmoid_map_268M":
        dt, _ = _timed_cpu(lambda: orc.sigmoid(v))
        return _cpu_entry(round(arr_n * 8 / dt / 1e9, 3), "GB/s", f"{arr_n} f32, 1/(1+expf(-x)), {dt * 1e3:.0f} ms")
    if name == "add_map_268M":
        w = rng.standard_normal(arr_n).astype(np.float32)
        dt, _ = _timed_cpu(lambda: orc.add(v, w))
        return _cpu_entry(round(arr_n * 12 / dt / 1e9, 3), "GB/s", f"{arr_n} f32 pairs, {dt * 1e3:.0f} ms")
    if name == "sum_f32_268M":
        dt, _ = _timed_cpu(lambda: orc.sum_f32(v))
        return _cpu_entry(round(arr_n * 4 / dt / 1e9, 3), "GB/s", f"{arr_n} f32, left fold, {dt * 1e3:.0f} ms")
    if name in ("add_row_bias_65536x4096", "sum_rows_65536x4096"):
        cols = 4096
        m = v.reshape(-1, cols)
        if name == "add_row_bias_65536x4096":
            bias = rng.standard_normal(cols).astype(np.float32)
            dt, _ = _timed_cpu(lambda: orc.add_row_bias(m, bias))
            return _cpu_entry(round(arr_n * 8 / dt / 1e9, 3), "GB/s", f"{m.shape[0]} x {cols} f32 plus a row bias, {dt * 1e3:.0f} ms")
        dt, _ = _timed_cpu(lambda: orc.sum_rows(m))
        return _cpu_entry(round(arr_n * 4 / dt / 1e9, 3), "GB/s", f"{m.shape[0]} x {cols} f32 summed down the columns, {dt * 1e3:.0f} ms")
    if name in ("mul_bcast_65536x4096_by_65536x1", "sum_to_shape_65536x4096_to_65536x1"):
        cols = 4096
        m = v.reshape(-1, cols)
        if name == "mul_bcast_65536x4096_by_65536x1":
            sc = rng.standard_normal((m.shape[0], 1)).astype(np.float32)
            dt, _ = _timed_cpu(lambda: orc.bcast("mul", m, sc))
            return _cpu_entry(round(arr_n * 8 / dt / 1e9, 3), "GB/s",
                              f"{m.shape[0]} x {cols} f32 times a {m.shape[0]} x 1 column, broadcast, {dt * 1e3:.0f} ms")
        dt, _ = _timed_cpu(lambda: orc.sum_to_shape(m, (m.shape[0], 1)))
        return _cpu_entry(round(arr_n * 4 / dt / 1e9, 3), "GB/s",
                          f"{m.shape[0]} x {cols} f32 summed along each row, {dt * 1e3:.0f} ms")
    if name == "max_argmax_f32_268M":
        dt, _ = _timed_cpu(lambda: (orc.max_of(v), orc.argmax(v)))
        return _cpu_entry(round(arr_n * 4 / dt / 1e9, 3), "GB/s",
                          f"{arr_n} f32, max_of then argmax (two passes, as two reference calls), {dt * 1e3:.0f} ms")
    raise KeyError(name)


def host_boundary(steps):
    """Rates of the `_host` entry points (cleave's extern boundary: pageable
    host arrays staged through HBM, results copied back, stream synchronised)
    at the BASELINE shapes, wall clock per call.  PCIe-inclusive figures for
    the record; the headline `value` never includes a host transfer."""
    import numpy as np

    from cleave_amd import host

    out = {}

    def run(name, fn, work, unit, reps):
        fn()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        dt = (time.perf_counter() - t0) / reps
        out[name] = {"ms_per_call": round(dt * 1e3, 3), unit: round(work / dt / 1e9, 2)}
        log(f"host boundary {name}: {dt * 1e3:.2f} ms per call")

    rng = np.random.default_rng(5)
    n = 4096
    A = rng.standard_normal((n, n), dtype=np.float32)
    B = rng.standard_normal((n, n), dtype=np.float32)
    run("matmul_f32_host_4096", lambda: host.matmul(A, B), 2.0 * n ** 3, "GFLOP/s", max(3, steps // 4))
    n1 = 256
    A1, B1 = A[:n1, :n1].copy(), B[:n1, :n1].copy()
    run("matmul_f32_host_256", lambda: host.matmul(A1, B1), 2.0 * n1 ** 3, "GFLOP/s", 50)
    v = rng.standard_normal(1 << 28, dtype=np.float32)
    run("sum_f32_host_268M", lambda: host.sum(v), 4.0 * v.size, "GB/s_of_input", max(3, steps // 4))
    del v
    g = 16384
    run("escape_counts_host_16384", lambda: host.escape_counts(g, g, -2.0, -1.5, 3.0 / g, 3.0 / g, 1000),
        float(g * g), "Gpixel/s", 3)
    return out


def gemm_bf16_layouts(ca, layouts, steps):
    """The bf16 8192^3 product of the bench, in each of the given layouts
    ("nn", "nt", "tn", "tt": op(A) op(B)), timed with HIP events after a 0.5 s
    clock-settling warm-up.  For comparing kernels and collecting counters."""
    m = 8192
    a32 = ca.fill_normal(ca.empty((m, m)), seed=201, std=0.02)
    ab = ca.to_bf16(a32)
    ca.fill_normal(a32, seed=202, std=0.02)
    bb = ca.to_bf16(a32)
    del a32
    c = ca.empty((m, m))
    out = {}
    for lay in layouts:
        ta, tb = lay[0] == "t", lay[1] == "t"
        _, ev = timed(ca, lambda: ca.matmul(ab, bb, trans_a=ta, trans_b=tb, out=c), steps, 3, 0.5)
        out[lay] = {"kernel_ms": round(ev, 4), "TFLOP/s": round(2.0 * m ** 3 / (ev * 1e-3) / 1e12, 1),
                    "frac_bf16_mfma": round(2.0 * m ** 3 / (ev * 1e-3) / 1e12 / PEAK_BF16_MFMA, 4)}
        log(f"gemm bf16 8192^3 {lay}: {ev:.4f} ms")
    return out


def copy_same_bytes(ca, nbytes, steps):
    """Kernel time of the library's streaming map (neg: 4 bytes read and 4
    written per element) moving nbytes / 2 each way: the floor a kernel that
    moves the same compulsory bytes meets at this size on this box."""
    n = nbytes // 8
    x = ca.fill_normal(ca.empty(n), seed=7)
    y = ca.empty(n)
    _, ev = timed(ca, lambda: ca.neg(x, out=y), steps, 3, 0.3)
    del x, y
    return ev


def gemm_bf16_batched_layouts(ca, layouts, steps):
    """The batched bf16 64 x 512^3 product of the bench, in each of the given
    layouts, timed like gemm_bf16_layouts; also as a fraction of HBM for the
    compulsory bytes (bf16 A and B read once, f32 C written once)."""
    bs, k = 64, 512
    t32 = ca.fill_normal(ca.empty((bs, k, k)), seed=301, std=0.02)
    xb = ca.to_bf16(t32)
    ca.fill_normal(t32, seed=302, std=0.02)
    yb = ca.to_bf16(t32)
    del t32
    zb = ca.empty((bs, k, k))
    hbm = bs * k * k * (2 + 2 + 4)
    out = {}
    for lay in layouts:
        ta, tb = lay[0] == "t", lay[1] == "t"
        _, ev = timed(ca, lambda: ca.matmul_batched(xb, yb, trans_a=ta, trans_b=tb, out=zb), steps * 4, 3, 0.3)
        out[lay] = {"kernel_ms": round(ev, 5), "frac_hbm": round(hbm / (ev * 1e-3) / 1e9 / PEAK_HBM, 4),
                    "frac_bf16_mfma": round(2.0 * bs * k ** 3 / (ev * 1e-3) / 1e12 / PEAK_BF16_MFMA, 4)}
        log(f"gemm bf16 batched 64 x 512^3 {lay}: {ev * 1e3:.2f} us")
    cp = copy_same_bytes(ca, hbm, steps * 4)
    out["copy_same_bytes"] = {"kernel_ms": round(cp, 5), "frac_hbm": round(hbm / (cp * 1e-3) / 1e9 / PEAK_HBM, 4)}
    log(f"streaming copy of the same {hbm >> 20} MiB: {cp * 1e3:.2f} us")
    return out


def gemm_shapes(ca, specs, steps):
    """One product per spec "dtype:MxNxK:layout", or a batch of them as
    "dtype:BxMxNxK:layout" (dtype f32, bf16 or f64, layout nn/nt/tn/tt for op(A)
    op(B)), timed with HIP events after a 0.3 s warm-up.  Reports TFLOP/s and
    the compulsory HBM bytes (A and B read once, f32 C written once) as a
    fraction of peak.  For comparing kernels and for kernel traces of one
    shape at a time."""
    import numpy as np

    out = {}
    for spec in specs:
        dt, dims, lay = spec.split(":")
        d = [int(x) for x in dims.split("x")]
        bs, (m, n, k) = (d[0], d[1:]) if len(d) == 4 else (1, d)
        lead = (bs,) if len(d) == 4 else ()
        ta, tb = lay[0] == "t", lay[1] == "t"
        if dt == "f64":
            rng = np.random.default_rng(11)
            a = ca.from_numpy(rng.standard_normal(lead + ((k, m) if ta else (m, k))))
            b = ca.from_numpy(rng.standard_normal(lead + ((n, k) if tb else (k, n))))
        else:
            a = ca.fill_normal(ca.empty(lead + ((k, m) if ta else (m, k))), seed=11)
            b = ca.fill_normal(ca.empty(lead + ((n, k) if tb else (k, n))), seed=12)
        if dt == "bf16":
            a, b = ca.to_bf16(a), ca.to_bf16(b)
        elif dt not in ("f32", "f64"):
            raise ValueError(f"unknown dtype in {spec!r}")
        c = ca.empty(lead + (m, n), "f64" if dt == "f64" else "f32")
        esz = {"bf16": 2, "f32": 4, "f64": 8}[dt]
        hbm = bs * ((m * k + k * n) * esz + m * n * (8 if dt == "f64" else 4))
        mm = ca.matmul_batched if lead else ca.matmul
        _, ev = timed(ca, lambda: mm(a, b, trans_a=ta, trans_b=tb, out=c), steps, 3, 0.3)
        out[spec] = {"kernel_ms": round(ev, 5), "TFLOP/s": round(2.0 * bs * m * n * k / (ev * 1e-3) / 1e12, 2),
                     "frac_hbm": round(hbm / (ev * 1e-3) / 1e9 / PEAK_HBM, 4)}
        log(f"gemm {spec}: {ev * 1e3:.1f} us")
        del a, b, c
    return out


COPY_ELEMS = 1 << 26  # 256 MiB of f32 read, 256 MiB written per launch


def calibrate_copy(ca, steps):
    """A plain streaming copy of known size (neg map: 4 bytes read and 4 bytes
    written per element).  Its FETCH_SIZE / WRITE_SIZE per dispatch, divided by
    the 268435456 bytes it must move each way, is the scale factor applied to
    the same counters read for the GEMM."""
    x = ca.fill_normal(ca.empty(COPY_ELEMS), seed=7)
    y = ca.empty(COPY_ELEMS)
    wall, ev = timed(ca, lambda: ca.neg(x, out=y), steps, 1)
    gbs = 2 * 4 * COPY_ELEMS / (ev * 1e-3) / 1e9
    print(json.dumps({"calibration": "copy", "bytes_each_way": 4 * COPY_ELEMS,
                      "kernel_ms": round(ev, 4), "GB/s": round(gbs, 1)}), flush=True)


def mlp_lines(ca, steps, secondary, want_cpu, cb, orc):
    """the fused MLP step and the same step through the
    reverse-mode tape, into `secondary`."""
    import numpy as np

    # MLP step (config 4)
    B_, D_, H_ = 65536, 1024, 4096
    x = ca.fill_normal(ca.empty((B_, D_)), seed=401)
    yv = ca.fill_bernoulli(ca.empty(B_), seed=402)
    lim1 = float(np.sqrt(6.0 / (D_ + H_)))
    lim2 = float(np.sqrt(6.0 / (H_ + 1)))
    w1 = ca.fill_uniform(ca.empty((D_, H_)), seed=403, lo=-lim1, hi=lim1)
    w2 = ca.fill_uniform(ca.empty(H_), seed=404, lo=-lim2, hi=lim2)
    loss = ca.empty(1)
    mlp_steps = max(5, steps // 5)
    wall_s, ev = timed(ca, lambda: ca.mlp_step(x, yv, w1, w2, 0.01, loss=loss), mlp_steps, 2, 0.3)
    gemm_fl = 2.0 * B_ * D_ * H_ * 2 + 4.0 * B_ * H_
    secondary["mlp_step_65536x1024x4096"] = {
        "steps_per_s": round(mlp_steps / wall_s, 3), "ms_per_step": round(ev, 3),
        "gemm_TFLOP/s": round(gemm_fl / (ev * 1e-3) / 1e12, 2),
        "loss_after": float(loss.numpy()[0])}
    log(f"mlp step: {mlp_steps / wall_s:.2f} steps/s ({ev:.2f} ms)")
    if want_cpu:
        secondary["mlp_step_65536x1024x4096"]["cpu_baseline"] = cpu_secondary(
            orc, "mlp_step_65536x1024x4096", cb, X=x.numpy(), y=yv.numpy(), W1=w1.numpy(), W2=w2.numpy(), B=B_)
    # The same step written as a program of the library's operators and
    # differentiated by the reverse-mode tape (cleave_amd.autograd).  The tape
    # runs the hidden layer sigmoid(X W1) w2 and its reverse rule as the fused
    # step's kernels; the output sigmoid, the error, the mean, their rules and
    # the two SGD updates are separate launches.
    from cleave_amd import autograd as ad
    fused_ms = ev
    X_, Y_ = ad.const(x), ad.const(yv.view((B_, 1)))
    w2c = w2.view((H_, 1))

    def tape_step():
        W1, W2 = ad.param(w1), ad.param(w2c)
        e = ad.sigmoid(ad.sigmoid(X_ @ W1) @ W2) - Y_
        ad.backward(ad.mean(e * e))
        ca.sgd_update(w1, W1.grad, 0.01)
        ca.sgd_update(w2c, W2.grad, 0.01)

    wall_s, ev = timed(ca, tape_step, mlp_steps, 2, 0.3)
    secondary["mlp_step_tape_65536x1024x4096"] = {
        "steps_per_s": round(mlp_steps / wall_s, 3), "ms_per_step": round(ev, 3),
        "gemm_TFLOP/s": round(gemm_fl / (ev * 1e-3) / 1e12, 2),
        "fused_over_tape": round(fused_ms / ev, 3),
        "note": "reverse-mode derive() over a tape (cleave_amd.autograd), its hidden layer on the fused "
                "kernels; the CPU baseline is mlp_step_65536x1024x4096's, the same step"}
    log(f"mlp step through the tape: {mlp_steps / wall_s:.2f} steps/s ({ev:.2f} ms)")
    del X_, Y_, w2c
    del x, yv, w1, w2


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work (headline)")
    ap.add_argument("--cpu-budget-secondary", type=float, default=2.0,
                    help="seconds of CPU baseline work per secondary workload")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--vendor", action="store_true",
                    help="also time torch.matmul (hipBLASLt) on the GEMM shapes, same device")
    ap.add_argument("--vendor-only", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--gemm-bf16", metavar="LAYOUTS", default=None,
                    help="only time the bf16 8192^3 product in the comma-separated layouts (nn,nt,tn,tt)")
    ap.add_argument("--gemm-bf16-batched", metavar="LAYOUTS", default=None,
                    help="only time the batched bf16 64 x 512^3 product in the given layouts")
    ap.add_argument("--gemm", metavar="SPECS", default=None,
                    help="only time the comma-separated products dtype:MxNxK:layout or batches dtype:BxMxNxK:layout "
                         "(e.g. f32:2048x2048x2048:nn); with --vendor, torch on the same specs too")
    ap.add_argument("--host-boundary", action="store_true",
                    help="only time the _host entry points (host arrays across the C ABI, PCIe included)")
    ap.add_argument("--mlp", action="store_true", help="only time the MLP step, fused and through the tape")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run the copy kernel used to scale rocprofv3 FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); multi-GPU runs are "
              "out of scope for this build", file=sys.stderr)
        sys.exit(2)
    if args.vendor_only:
        if args.gemm:
            print(json.dumps(vendor_shapes(args.gemm.split(","), args.steps)), flush=True)
        else:
            print(json.dumps(vendor_yardstick(max(20, args.steps // 2))), flush=True)
        return

    import numpy as np

    import cleave_amd as ca

    if not ca.device_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    ca.init()
    steps, warmup = args.steps, args.warmup
    if args.calibrate_copy:
        calibrate_copy(ca, steps)
        return
    if args.gemm_bf16:
        print(json.dumps({"gemm_bf16_8192": gemm_bf16_layouts(ca, args.gemm_bf16.split(","), steps),
                          "library": str(ca._lib.LIB_PATH)}), flush=True)
        return
    if args.gemm_bf16_batched:
        print(json.dumps({"gemm_bf16_batched_64x512": gemm_bf16_batched_layouts(
            ca, args.gemm_bf16_batched.split(","), steps), "library": str(ca._lib.LIB_PATH)}), flush=True)
        return
    if args.gemm:
        res = {"gemm": gemm_shapes(ca, args.gemm.split(","), steps), "library": str(ca._lib.LIB_PATH)}
        if args.vendor:
            # torch on the same specs in a child process (see vendor_yardstick);
            # speed ratios are torch's time over this library's
            proc = subprocess.run([sys.executable, os.path.abspath(__file__), "--vendor-only", "--gemm", args.gemm,
                                   "--steps", str(steps)], stdout=subprocess.PIPE)
            if proc.returncode != 0:
                raise RuntimeError(f"vendor child failed with status {proc.returncode}")
            ven = json.loads(proc.stdout.decode().strip().splitlines()[-1])
            for spec, v in ven.items():
                row = res["gemm"][spec]
                row.update(v)
                row["speed_vs_torch"] = round(v["torch_ms"] / row["kernel_ms"], 4)
                if v.get("torch_f32_out_ms"):
                    row["speed_vs_torch_f32_out"] = round(v["torch_f32_out_ms"] / row["kernel_ms"], 4)
        print(json.dumps(res), flush=True)
        return
    if args.host_boundary:
        print(json.dumps({"host_boundary": host_boundary(steps)}), flush=True)
        return
    if args.mlp:
        out = {}
        mlp_lines(ca, steps, out, False, 0.0, None)
        print(json.dumps({"mlp": out}), flush=True)
        return

    # ---- headline: f32 4096^3 NN --------------------------------------------
    n = 4096
    a = ca.fill_normal(ca.empty((n, n)), seed=101)
    b = ca.fill_normal(ca.empty((n, n)), seed=102)
    c = ca.empty((n, n))
    flop = 2.0 * n * n * n
    # MI355X clocks settle after 0.1-0.3 s of sustained matrix-core load: the
    # warm-up is `warmup` steps and then at least HEADLINE_WARM_S seconds.
    log(f"gemm f32 {n}^3 NN: {warmup} warmup steps + {HEADLINE_WARM_S} s clock settle + {steps} timed steps")
    wall, ev_ms = timed(ca, lambda: ca.matmul(a, b, out=c), steps, warmup, HEADLINE_WARM_S)
    value = flop * steps / wall / 1e9
    achieved = flop / (ev_ms * 1e-3) / 1e12
    log(f"  {value:.1f} GFLOP/s wall, kernel {ev_ms:.3f} ms = {achieved:.1f} TFLOP/s")
    traffic = read_traffic("gemm_f32_nn_4096")

    result = {
        "metric": "GEMM GFLOP/s + % MFMA peak (f32 4096^3, bf16 8192^3); MLP train steps/s",
        "value": round(value, 1),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "warmup_s": HEADLINE_WARM_S,
        "ms_per_step": round(wall / steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (N(0,1) from seed, generated on the device)",
        "config": {"workload": "gemm_f32_nn_4096 (BASELINE configs[1], A B)", "M": n, "N": n, "K": n,
                   "layout": "row-major", "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP32_MFMA,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA, 4),
                     "traffic": traffic},
    }

    secondary = {}
    want_cpu = not args.no_cpu
    if want_cpu:
        from oracle import oracle as orc
        A_host, B_host = a.numpy(), b.numpy()
    cb = args.cpu_budget_secondary
    if not args.no_secondary:
        sec_steps = max(20, steps // 2)
        # config 1: f32 256^3, A and B the first and second 256^2 draws of the
        # seed-0 uniform[-1,1) stream (one 2 x 256^2 fill, split in two)
        n1 = 256
        ab1 = ca.fill_uniform(ca.empty(2 * n1 * n1), seed=0)
        a1, b1 = ab1.sub(0, (n1, n1)), ab1.sub(n1 * n1, (n1, n1))
        c1 = ca.empty((n1, n1))
        fl1 = 2.0 * n1 ** 3
        wall_s, ev = timed(ca, lambda: ca.matmul(a1, b1, out=c1), 200, 20, 0.1)
        secondary["gemm_f32_256"] = {"GFLOP/s": round(fl1 * 200 / wall_s / 1e9, 1), "kernel_ms": round(ev, 5),
                                     "kernel_GFLOP/s": round(fl1 / (ev * 1e-3) / 1e9, 1),
                                     "frac_fp32_mfma": round(fl1 / (ev * 1e-3) / 1e12 / PEAK_FP32_MFMA, 4),
                                     "note": "latency-bound: one 256^3 product is 64 tiles of 32 x 32, one per "
                                             "workgroup, K split over its 4 waves (32 fp32 MFMAs each after "
                                             "one wait for all their loads); wall GFLOP/s includes the host "
                                             "call per step"}
        log(f"gemm_f32_256: {fl1 / (ev * 1e-3) / 1e9:.0f} GFLOP/s kernel")
        if want_cpu:
            secondary["gemm_f32_256"]["cpu_baseline"] = cpu_secondary(orc, "gemm_f32_256", cb,
                                                                      A=a1.numpy(), B=b1.numpy(), n=n1)
        del a1, b1, ab1, c1
        # f32 A B^T and A^T B (reverse-mode halves of the product rule)
        for name, ta, tb in [("gemm_f32_nt_4096", False, True), ("gemm_f32_tn_4096", True, False)]:
            wall_s, ev = timed(ca, lambda: ca.matmul(a, b, trans_a=ta, trans_b=tb, out=c), sec_steps, 2, 0.3)
            ach = flop / (ev * 1e-3) / 1e12
            secondary[name] = {"GFLOP/s": round(flop * sec_steps / wall_s / 1e9, 1),
                               "kernel_ms": round(ev, 4), "frac_fp32_mfma": round(ach / PEAK_FP32_MFMA, 4)}
            log(f"{name}: {ach:.1f} TFLOP/s")
            if want_cpu:
                secondary[name]["cpu_baseline"] = cpu_secondary(orc, name, cb, A=A_host, B=B_host, n=n, ta=ta, tb=tb)
        del c
        # Tensor<f64>: the config-2 product in f64 on the f64 matrix cores
        rng64 = np.random.default_rng(103)
        a64 = ca.from_numpy(rng64.standard_normal((n, n)))
        b64 = ca.from_numpy(rng64.standard_normal((n, n)))
        c64 = ca.empty((n, n), "f64")
        wall_s, ev = timed(ca, lambda: ca.matmul(a64, b64, out=c64), max(10, sec_steps // 2), 2, 0.3)
        ach = flop / (ev * 1e-3) / 1e12
        secondary["gemm_f64_4096"] = {"GFLOP/s": round(flop * max(10, sec_steps // 2) / wall_s / 1e9, 1),
                                      "kernel_ms": round(ev, 4), "frac_fp64_mfma": round(ach / PEAK_FP64_MFMA, 4)}
        log(f"gemm_f64_4096: {ach:.1f} TFLOP/s")
        if want_cpu:
            secondary["gemm_f64_4096"]["cpu_baseline"] = cpu_secondary(orc, "gemm_f64_4096", cb, A=a64.numpy(),
                                                                       B=b64.numpy(), n=n)
        del a64, b64, c64
        # bf16 8192^3
        m = 8192
        a32 = ca.fill_normal(ca.empty((m, m)), seed=201, std=0.02)
        ab = ca.to_bf16(a32)
        ca.fill_normal(a32, seed=202, std=0.02)
        bb = ca.to_bf16(a32)
        del a32
        cmat = ca.empty((m, m))
        fl = 2.0 * m ** 3
        wall_s, ev = timed(ca, lambda: ca.matmul(ab, bb, out=cmat), sec_steps, 2, 0.4)
        ach = fl / (ev * 1e-3) / 1e12
        secondary["gemm_bf16_8192"] = {"GFLOP/s": round(fl * sec_steps / wall_s / 1e9, 1), "kernel_ms": round(ev, 4),
                                       "frac_bf16_mfma": round(ach / PEAK_BF16_MFMA, 4)}
        log(f"gemm_bf16_8192: {ach:.1f} TFLOP/s")
        if want_cpu:
            secondary["gemm_bf16_8192"]["cpu_baseline"] = cpu_secondary(
                orc, "gemm_bf16_8192", cb, A=ab.numpy(), B=bb.numpy(), m=m)
        del ab, bb, cmat
        # batched bf16 64 x 512^3
        bs, k = 64, 512
        t32 = ca.fill_normal(ca.empty((bs, k, k)), seed=301, std=0.02)
        xb = ca.to_bf16(t32)
        ca.fill_normal(t32, seed=302, std=0.02)
        yb = ca.to_bf16(t32)
        del t32
        zb = ca.empty((bs, k, k))
        fl = 2.0 * bs * k ** 3
        wall_s, ev = timed(ca, lambda: ca.matmul_batched(xb, yb, out=zb), sec_steps * 4, 2, 0.3)
        ach = fl / (ev * 1e-3) / 1e12
        # compulsory HBM bytes: bf16 A and B read once, f32 C written once
        hbm = bs * k * k * (2 + 2 + 4)
        secondary["gemm_bf16_batched_64x512"] = {"GFLOP/s": round(fl * sec_steps * 4 / wall_s / 1e9, 1),
                                                 "kernel_ms": round(ev, 4),
                                                 "frac_bf16_mfma": round(ach / PEAK_BF16_MFMA, 4),
                                                 "hbm_GB/s": round(hbm / (ev * 1e-3) / 1e9, 1),
                                                 "frac_hbm": round(hbm / (ev * 1e-3) / 1e9 / PEAK_HBM, 4)}
        # the same bytes moved by the library's streaming map, same run
        cp = copy_same_bytes(ca, hbm, sec_steps * 4)
        secondary["gemm_bf16_batched_64x512"].update(
            {"copy_same_bytes_ms": round(cp, 5), "frac_of_copy": round(cp / ev, 4),
             "note": "the compulsory bytes (bf16 A, B read; f32 C written: 64 MiB each way) moved by "
                     "the library's streaming map in one launch take copy_same_bytes_ms; frac_of_copy "
                     "= that time / the product's"})
        log(f"gemm_bf16_batched_64x512: {ach:.1f} TFLOP/s; a streaming copy of the same bytes {cp * 1e3:.2f} us")
        if want_cpu:
            secondary["gemm_bf16_batched_64x512"]["cpu_baseline"] = cpu_secondary(
                orc, "gemm_bf16_batched_64x512", cb, A=xb.numpy()[0], B=yb.numpy()[0], bs=bs, k=k)
        del xb, yb, zb
        mlp_lines(ca, steps, secondary, want_cpu, cb, orc if want_cpu else None)
        # a matrix-vector product (a2 at N = 1: the reference's matmul by a
        # column vector, gemv.hip), HBM-bound on the matrix
        mv_m, mv_k = 65536, 4096
        mva = ca.fill_normal(ca.empty((mv_m, mv_k)), seed=405)
        mvx = ca.fill_normal(ca.empty((mv_k, 1)), seed=406)
        mvy = ca.empty((mv_m, 1))
        wall_s, ev = timed(ca, lambda: ca.matmul(mva, mvx, out=mvy), sec_steps, 2, 0.2)
        mv_bytes = (mv_m * mv_k + mv_k + mv_m) * 4
        secondary["matvec_f32_65536x4096"] = {
            "ms": round(ev, 4), "GB/s": round(mv_bytes / (ev * 1e-3) / 1e9, 1),
            "frac_hbm": round(mv_bytes / (ev * 1e-3) / 1e9 / PEAK_HBM, 4),
            "note": "one wave-slice per row, 16-byte loads, shuffle-tree sums (gemv.hip)"}
        log(f"matvec: {mv_bytes / (ev * 1e-3) / 1e9:.0f} GB/s")
        if want_cpu:
            secondary["matvec_f32_65536x4096"]["cpu_baseline"] = cpu_secondary(
                orc, "matvec_f32_65536x4096", cb, A=mva.numpy(), x=mvx.numpy(), m=mv_m, k=mv_k)
        del mva, mvx, mvy
        # escape-count map + u64 sum (config 3)
        g = 16384
        d = np.float32(3.0 / g)
        cnt = ca.empty((g, g), "u32")
        wall_s, ev = timed(ca, lambda: ca.escape_counts(g, g, -2.0, -1.5, d, d, 1000, out=cnt), 10, 2, 0.2)
        # sum of counts = iterations executed by escaped pixels minus one each,
        # max_iter for pixels that never escape: a lower bound of the executed work
        total = ca.sum_u64(cnt)
        # The reference's iteration is 11 FLOP; the kernel executes it in
        # MANDEL_VALU_PER_ITER VALU instructions (two products are reused,
        # zr*zi + zi*zr is p + p, and (p + p) + ci is one fma: all exact), so the
        # ceiling is the VALU issue rate over that count.
        rate = total / (ev * 1e-3)
        secondary["mandelbrot_16384_1000"] = {
            "ms": round(ev, 3), "pixel_iter_per_s": round(rate, 1),
            "TFLOP/s_11_per_iter": round(11.0 * rate / 1e12, 2),
            "valu_per_iter": MANDEL_VALU_PER_ITER,
            "frac_valu_issue": round(MANDEL_VALU_PER_ITER * rate / 1e12 / PEAK_FP32_VALU_NOFMA, 4),
            "sum_of_counts": int(total)}
        log(f"mandelbrot: {ev:.2f} ms, sum {total}")
        if want_cpu:
            secondary["mandelbrot_16384_1000"]["cpu_baseline"] = cpu_secondary(
                orc, "mandelbrot_16384_1000", cb, g=g, d=d, total=int(total))
        out_dev = ca.empty(1, "u64")
        wall_s, ev = timed(ca, lambda: ca.reduce_sum_u64(cnt, out_dev), 40, 5, 0.2)
        gbs = g * g * 4 / (ev * 1e-3) / 1e9
        secondary["sum_u32_u64_16384sq"] = {"ms": round(ev, 4), "GB/s": round(gbs, 1),
                                           "frac_hbm": round(gbs / PEAK_HBM, 4)}
        log(f"u64 sum: {gbs:.0f} GB/s")
        if want_cpu:
            secondary["sum_u32_u64_16384sq"]["cpu_baseline"] = cpu_secondary(orc, "sum_u32_u64_16384sq", cb)
        del cnt
        # sigmoid map over an H-sized tensor (65536 x 4096 f32)
        hn = 65536 * 4096
        hx = ca.fill_normal(ca.empty(hn), seed=501)
        hy = ca.empty(hn)
        wall_s, ev = timed(ca, lambda: ca.sigmoid(hx, out=hy), 30, 5, 0.2)
        gbs = hn * 8 / (ev * 1e-3) / 1e9
        secondary["sigmoid_map_268M"] = {"ms": round(ev, 4), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM, 4)}
        log(f"sigmoid map: {gbs:.0f} GB/s")
        if want_cpu:
            secondary["sigmoid_map_268M"]["cpu_baseline"] = cpu_secondary(orc, "sigmoid_map_268M", cb)
        # binary Ring map (two reads, one write per element)
        hz = ca.fill_normal(ca.empty(hn), seed=502)
        wall_s, ev = timed(ca, lambda: ca.add(hx, hz, out=hy), 30, 5, 0.2)
        gbs = hn * 12 / (ev * 1e-3) / 1e9
        secondary["add_map_268M"] = {"ms": round(ev, 4), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM, 4)}
        log(f"add map: {gbs:.0f} GB/s")
        if want_cpu:
            secondary["add_map_268M"]["cpu_baseline"] = cpu_secondary(orc, "add_map_268M", cb)
        del hz
        # bias shared by every row of the hidden layer, and its reverse rule
        hb = ca.fill_normal(ca.empty(4096), seed=503)
        hx2, hy2 = hx.view((65536, 4096)), hy.view((65536, 4096))
        wall_s, ev = timed(ca, lambda: ca.add_row_bias(hx2, hb, out=hy2), 30, 5, 0.2)
        gbs = hn * 8 / (ev * 1e-3) / 1e9
        secondary["add_row_bias_65536x4096"] = {"ms": round(ev, 4), "GB/s": round(gbs, 1),
                                                "frac_hbm": round(gbs / PEAK_HBM, 4)}
        log(f"add row bias: {gbs:.0f} GB/s")
        if want_cpu:
            secondary["add_row_bias_65536x4096"]["cpu_baseline"] = cpu_secondary(orc, "add_row_bias_65536x4096", cb)
        sr = ca.empty(4096)
        wall_s, ev = timed(ca, lambda: ca.sum_rows(hx2, out=sr), 30, 5, 0.2)
        gbs = hn * 4 / (ev * 1e-3) / 1e9
        secondary["sum_rows_65536x4096"] = {"ms": round(ev, 4), "GB/s": round(gbs, 1),
                                            "frac_hbm": round(gbs / PEAK_HBM, 4)}
        log(f"sum rows: {gbs:.0f} GB/s")
        if want_cpu:
            secondary["sum_rows_65536x4096"]["cpu_baseline"] = cpu_secondary(orc, "sum_rows_65536x4096", cb)
        # general broadcasting: a per-row scale (65536 x 1 stretched along the
        # columns) and its reverse rule, the sums along each row
        hs = ca.fill_normal(ca.empty((65536, 1)), seed=504)
        wall_s, ev = timed(ca, lambda: ca.mul(hx2, hs, out=hy2), 30, 5, 0.2)
        gbs = (hn * 8 + 65536 * 4) / (ev * 1e-3) / 1e9
        secondary["mul_bcast_65536x4096_by_65536x1"] = {"ms": round(ev, 4), "GB/s": round(gbs, 1),
                                                        "frac_hbm": round(gbs / PEAK_HBM, 4)}
        log(f"mul broadcast: {gbs:.0f} GB/s")
        if want_cpu:
            secondary["mul_bcast_65536x4096_by_65536x1"]["cpu_baseline"] = cpu_secondary(
                orc, "mul_bcast_65536x4096_by_65536x1", cb)
        wall_s, ev = timed(ca, lambda: ca.sum_to_shape(hx2, (65536, 1), out=hs), 30, 5, 0.2)
        gbs = (hn * 4 + 65536 * 4) / (ev * 1e-3) / 1e9
        secondary["sum_to_shape_65536x4096_to_65536x1"] = {"ms": round(ev, 4), "GB/s": round(gbs, 1),
                                                           "frac_hbm": round(gbs / PEAK_HBM, 4)}
        log(f"sum to shape (rows): {gbs:.0f} GB/s")
        if want_cpu:
            secondary["sum_to_shape_65536x4096_to_65536x1"]["cpu_baseline"] = cpu_secondary(
                orc, "sum_to_shape_65536x4096_to_65536x1", cb)
        del hs
        # f32 Sum and Max/argmax reductions (one read per element)
        sdev = ca.empty(1)
        wall_s, ev = timed(ca, lambda: ca.reduce_sum(hx, sdev), 30, 5, 0.2)
        gbs = hn * 4 / (ev * 1e-3) / 1e9
        secondary["sum_f32_268M"] = {"ms": round(ev, 4), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM, 4)}
        log(f"sum f32: {gbs:.0f} GB/s")
        if want_cpu:
            secondary["sum_f32_268M"]["cpu_baseline"] = cpu_secondary(orc, "sum_f32_268M", cb)
        mdev, idev = ca.empty(1), ca.empty(1, "i64")
        wall_s, ev = timed(ca, lambda: ca.reduce_max(hx, mdev, idev), 30, 5, 0.2)
        gbs = hn * 4 / (ev * 1e-3) / 1e9
        secondary["max_argmax_f32_268M"] = {"ms": round(ev, 4), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM, 4)}
        log(f"max/argmax f32: {gbs:.0f} GB/s")
        if want_cpu:
            secondary["max_argmax_f32_268M"]["cpu_baseline"] = cpu_secondary(orc, "max_argmax_f32_268M", cb)
        del hx, hy
    if secondary:
        result["secondary"] = secondary
    if args.vendor:
        # a child process (not an exec): see vendor_yardstick
        proc = subprocess.run([sys.executable, os.path.abspath(__file__), "--vendor-only", "--steps", str(steps)],
                              stdout=subprocess.PIPE, timeout=600)
        if proc.returncode != 0:
            raise RuntimeError(f"vendor yardstick child failed with status {proc.returncode}")
        result["vendor_same_device"] = json.loads(proc.stdout.decode().strip().splitlines()[-1])

    if not args.no_cpu:
        log(f"cpu baseline: ~{args.cpu_budget:.0f} s of the restated loop on one core")
        result["cpu_baseline"] = cpu_baseline_gemm(A_host, B_host, n, args.cpu_budget)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
