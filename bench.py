"""Benchmark of the SushiBLAS GEMM hot path on one MI355X.

Headline (BASELINE.json metric, configs[1]): fp32 GEMM, row-major, no
transpose, M = N = K = 8192, alpha = 1.5, beta = 0.5; A, B ~ U[-1, 1) and
C ~ N(0, 1) from the Philox4x32-10 generator (seed 20261203), generated in
HBM before timing.  A "step" is one sbx_sgemm call (include/sbx.h) over that
problem; `value` = 2*M*N*K / (average step time), in TFLOP/s.

Printed as one JSON line.  Besides the contract fields it carries:
  roofline      -- the dominant kernel against the fp32 MFMA peak
  cpu_baseline  -- the reference's CPU path stand-in (MKL's CPU sgemm via
                   torch; the reference's oneMKL SYCL path cannot be built
                   here), with the CPU oracle (oracle/, a port) nested, both
                   timed on a bounded sample of rows of the same problem, on
                   this host's cores
  parity        -- normwise error of the GPU result vs the oracle
                   (accumulating in double) over the whole matrix, on
                   identical input bits; each BASELINE GEMM config under
                   `also` carries its own cpu_baseline and parity too
  vendor        -- the same headline GEMM through torch.addmm (hipBLASLt)
                   on the same device inputs, for context (and `vendor_ms`
                   beside each GEMM config under `also`)
  also          -- the other BASELINE configs timed the same way (fp64 8192^3,
                   the ragged 4095x3001x2047 transposes, tall-skinny, 512^3), the
                   fused GEMM+ReLU epilogue against GEMM followed by ReLU, GEMV
                   (HBM GB/s), SYRK (TFLOP/s over the triangle), and the C++
                   Engine/TaskGraph path on the reference's framework-sim
                   patterns (microseconds per batch, one lane vs four)

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-also]
                       [--cpu-seconds S] [--no-cpu] [--no-vendor] [--probe]
       python bench.py --only <also key>     (one secondary workload, for profiling)
       python bench.py --calibrate-copy      (1 GiB copy, the PMC byte reference)
       python bench.py --probe --k-sweep     (512 x 512 x K on the small-problem kernel)

--probe runs everything on the probe build of the library, whose GEMM kernels
stamp the shader clock counter and a constant-rate counter per workgroup: the
GEMM configs then also report, for the dispatches of their timed loop, the
clock, the span and the MFMA busy fraction (no profiler, no serialisation).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GEMM TFLOP/s on 1 MI355X (fp32 8192³, fp64 8192³); % of MFMA peak"
PEAK = {"f32": 157.3, "f64": 78.6}  # dense MFMA TFLOP/s, MI355X
HBM_PEAK_GBS = 8000.0
SEED = 20261201


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-also", action="store_true", help="skip the secondary configs")
    ap.add_argument("--no-vendor", action="store_true",
                    help="skip timing the vendor library (torch.addmm) beside the GEMM configs")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target CPU time of the cpu_baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--only", default=None,
                    help="run one secondary workload (a key of the `also` object) and print "
                         "it alone: one workload per run for rocprofv3 counter passes")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (torch copy_) a few "
                         "times: the known-size reference for rocprofv3 FETCH_SIZE/WRITE_SIZE")
    ap.add_argument("--probe", action="store_true",
                    help="run on the probe build (lib/libsbx_probe.so): the GEMM configs "
                         "also report the clock, loop span and MFMA busy of every timed "
                         "dispatch from per-workgroup clock stamps (no serialisation)")
    ap.add_argument("--regret", type=int, default=None, metavar="SEED",
                    help="time the kernel-selection pick against every candidate plan on the "
                         "seeded shape list (regret_shapes) and report the regret")
    ap.add_argument("--regret-count", type=int, default=60,
                    help="shapes in the --regret list")
    ap.add_argument("--regret-syrk", type=int, default=0,
                    help="SYRK shapes in the --regret list (regret_syrk_shapes)")
    ap.add_argument("--regret-full", action="store_true",
                    help="keep every plan's measured and predicted time in the --regret rows")
    ap.add_argument("--hbm-rates", action="store_true",
                    help="time torch's copy and sum over 1 GiB: the HBM rates of the vendor's "
                         "own streaming kernels on this box")
    ap.add_argument("--abba", type=int, default=None, metavar="ROUNDS",
                    help="interleaved timing of the tall-skinny call (configs[3]) against "
                         "torch.addmm on the same buffers: ROUNDS rounds of four "
                         "measurements in ABBA order, then the mirror")
    ap.add_argument("--k-sweep", action="store_true",
                    help="with --probe: time 512 x 512 x K, K = 64 ... 2048, on both forms "
                         "of the small-problem kernel (by name) and fit time = intercept + "
                         "slope * K per form")
    return ap.parse_args()


def calibrate_copy():
    """1 GiB read + 1 GiB write per dispatch of torch's copy kernel."""
    import torch
    n = 1 << 28  # float32 elements = 1 GiB
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": n * 4, "dispatches": 3}), flush=True)


def hbm_rates():
    """The HBM rates the vendor's own streaming kernels reach on this box,
    timed like the workloads over 1 GiB of fp32: torch's copy (read +
    write) and torch.sum (read only) -- practical ceilings beside the 8 TB/s
    datasheet figure, for the HBM-bound rows (GEMV)."""
    import torch
    n = 1 << 28
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    acc = torch.empty((), dtype=torch.float32, device="cuda")
    copy_ms = time_launches(lambda: dst.copy_(src), 20, 3, min_warm_s=0.25)
    sum_ms = time_launches(lambda: torch.sum(src, dim=(0,), out=acc), 20, 3, min_warm_s=0.25)
    return {"bytes": n * 4, "copy_ms": round(copy_ms, 4),
            "copy_gbs": round(2 * n * 4 / (copy_ms * 1e-3) / 1e9, 1),
            "sum_ms": round(sum_ms, 4), "sum_read_gbs": round(n * 4 / (sum_ms * 1e-3) / 1e9, 1)}


PROBE = False  # --probe: record per-workgroup clock stamps of the timed dispatches
PROBE_BLOCKS = 4096  # workgroups per dispatch whose stamps are kept


PROBE_POINTS = 4  # stamp points per workgroup (SBX_PROBE_POINTS)


def probe_summary(t, ndisp, flops, dtype, call_ms, khz, cus):
    """Clock, loop span and MFMA busy of the timed dispatches, from the probe
    build's per-workgroup stamps (see sushiblas_amd/csrc/sbx_probe.h).

    t: the stamp ring as uint64, ring x PROBE_BLOCKS x PROBE_POINTS x 2
    (core cycles, real-time ticks at `khz`); unused entries are 0.  Per
    dispatch: clock = median over workgroups of core cycles / real time
    between the first and last stamp; span = last workgroup's last stamp -
    first workgroup's entry; MFMA busy = flops / (MFMA flop per cycle of the
    chip x clock x span).  `mfma_busy_of_call` uses the event-timed call time
    instead of the span (it includes the epilogue and launch gaps)."""
    import numpy as np
    if khz <= 0 or ndisp <= 0:
        return None
    per_clk = (256 if dtype == "f32" else 128) * cus  # dense MFMA flop per cycle, MI355X
    t = np.asarray(t).reshape(-1, PROBE_BLOCKS, PROBE_POINTS, 2).astype(np.float64)
    rows = []
    for d in range(min(ndisp, t.shape[0])):
        x = t[d]
        live = x[:, 0, 1] > 0
        if not live.any():
            continue
        x = x[live]
        last = 3 if (x[:, 3, 1] > 0).all() else 1  # small-problem kernel: 4 points
        cyc = x[:, last, 0] - x[:, 0, 0]
        rt = (x[:, last, 1] - x[:, 0, 1]) / (khz * 1e3)  # seconds
        ok = rt > 0
        clock = float(np.median(cyc[ok] / rt[ok])) / 1e9
        span = (x[:, last, 1].max() - x[:, 0, 1].min()) / (khz * 1e3)
        rows.append((clock, span * 1e6, float(np.median(cyc)), x))
    if not rows:
        return None
    clocks = np.array([r[0] for r in rows])
    spans = np.array([r[1] for r in rows])
    c_med, s_med = float(np.median(clocks)), float(np.median(spans))
    out = {"dispatches": len(rows), "clock_ghz": round(c_med, 3),
           "clock_ghz_min": round(float(clocks.min()), 3),
           "clock_ghz_max": round(float(clocks.max()), 3),
           "span_us": round(s_med, 2), "wg_cycles": round(float(np.median([r[2] for r in rows]))),
           "mfma_busy_span": round(flops / (per_clk * c_med * 1e9 * s_med * 1e-6), 4),
           "mfma_busy_of_call": round(flops / (per_clk * c_med * 1e9 * call_ms * 1e-3), 4)}
    x = rows[len(rows) // 2][3]
    if (x[:, 3, 1] > 0).all():  # small-problem kernel: where a workgroup's time goes
        us = lambda a, b: float(np.median(x[:, b, 1] - x[:, a, 1])) / (khz * 1e3) * 1e6
        out["wg_us"] = {"issue_first_loads": round(us(0, 1), 3), "to_mfma_done": round(us(1, 2), 3),
                        "reduce_and_store": round(us(2, 3), 3)}
        out["launch_spread_us"] = round(float(x[:, 0, 1].max() - x[:, 0, 1].min()) /
                                        (khz * 1e3) * 1e6, 3)
    return out


def time_launches(fn, steps, warmup, min_warm_s=0.0, probe=None):
    """Average device time per call of fn() over `steps` back-to-back calls,
    measured with HIP events on the stream the kernels run on.  With --probe
    and a dict `probe` = {"flops": F, "dtype": "f32"|"f64"}, the timed
    dispatches' stamps are recorded and probe["out"] gets probe_summary().

    `warmup` untimed calls come first; with min_warm_s > 0, more untimed calls
    follow until that much time has been spent warming up.  A GPU that sat
    idle during host-side setup takes tens of milliseconds to reach its
    working clock: the tall-skinny GEMM (0.3 ms a call) measured 380 us over
    its first 25 calls and 307-313 us after that, on one box."""
    import time
    import torch
    t0 = time.perf_counter()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < min_warm_s:
        for _ in range(max(1, warmup)):
            fn()
        torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    stamps = None
    if PROBE and probe is not None:
        import sushiblas_amd as sbx
        stamps = torch.zeros(steps * PROBE_BLOCKS * PROBE_POINTS * 2, dtype=torch.int64,
                             device="cuda")
        torch.cuda.synchronize()
        sbx.probe_set(stamps, PROBE_BLOCKS, steps)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    if stamps is not None:
        import numpy as np
        import sushiblas_amd as sbx
        ndisp = sbx.probe_dispatches()
        sbx.probe_set(None, 0, 0)
        probe["out"] = probe_summary(stamps.cpu().numpy().view(np.uint64), ndisp, probe["flops"],
                                     probe["dtype"], ms, sbx.probe_wall_clock_khz(),
                                     torch.cuda.get_device_properties(0).multi_processor_count)
        del stamps
    return ms  # ms


def read_traffic(workload):
    """HBM bytes per launch for `workload` ("headline" or a key of `also`)
    from the committed rocprofv3 PMC summary (profiles/hbm_traffic.md: two
    runs, FETCH_SIZE and WRITE_SIZE, each scaled by the same counter's reading
    for a plain 1 GiB copy), or None if it was not measured."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.md")
    if not os.path.exists(path):
        return None
    col = None
    for line in open(path):
        if not line.startswith("|"):
            continue
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if col is None and "traffic bytes" in cells:
            col = cells.index("traffic bytes")
        elif col is not None and len(cells) > col and cells[0] == workload:
            try:
                return int(cells[col].replace(",", ""))
            except ValueError:
                return None
    return None


VENDOR = True  # time torch (the vendor BLAS) beside each GEMM config; --no-vendor clears it


def cpu_model():
    """The host CPU's model name (from /proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _host_view(X, trans, rows, cols, ld):
    """op(X) (rows x cols) of a flat row-major buffer with leading dimension
    ld, as a 2-D numpy view: the stored matrix itself when not transposed,
    else the transpose of the stored cols x rows matrix.  The buffer must
    hold whole rows of ld elements (bench.py allocates exactly that)."""
    sr, sc = (cols, rows) if trans else (rows, cols)
    stored = X[:sr * ld].reshape(sr, ld)[:, :sc]
    return stored.T if trans else stored


def cpu_leg(dtype, ta, tb, m, n, k, alpha, beta, A, lda, B, ldb, C0, ldc, got, target_s):
    """CPU baseline and parity for one row-major GEMM configuration.

    cpu_baseline: the reference's CPU path is oneMKL's row_major::gemm on a
    SYCL CPU queue (src/ops/blas/level3/gemm.cpp:63), which cannot be built
    here (no SYCL compiler, no oneMKL-SYCL).  Its stand-in, the value
    reported, is the same vendor library's CPU GEMM called directly: MKL
    sgemm/dgemm through torch's CPU addmm (BLAS_INFO=mkl), on the first R rows
    of op(A) / C, R sized for about target_s seconds and capped at m, after
    one warm-up call, median of 3.  Nested under `port`: the oracle
    (oracle/sbo.c, blocked OpenMP) timed once on the same rows.
    parity: the GPU result over the WHOLE m x n matrix against the oracle
    accumulating in double on identical input bits (normwise relative
    Frobenius error), and the same for the timed port's rows."""
    import numpy as np
    import oracle
    threads = oracle.num_threads()
    fp32 = dtype == "f32"
    tol = 1e-5 if fp32 else 1e-12
    port_acc = 0 if fp32 else 1  # fp32: the port accumulates in fp32, as sgemm does
    g = _host_view(got, False, m, n, ldc)

    def run_rows(rows, acc):
        Cs = np.array(C0[:rows * ldc], copy=True)  # the oracle writes C in place
        t = time.perf_counter()
        oracle.gemm(0, ta, tb, rows, n, k, alpha, A, lda, B, ldb, beta, Cs, ldc, acc)
        return Cs, time.perf_counter() - t

    # sample size from a 64-row probe of the port (the slower of the two)
    r0 = min(m, 64)
    _, dt0 = run_rows(r0, port_acc)
    rate = 2.0 * r0 * n * k / max(dt0, 1e-6)
    rows = int(min(m, max(r0, (rate * target_s) / (2.0 * n * k) // 64 * 64)))
    what = (f"first {rows} of {m} rows of the same {m}x{n}x{k} {dtype} GEMM "
            f"(tA={ta}, tB={tb})")
    base = {"value": None, "unit": "TFLOP/s", "cores": threads, "kind": "reference",
            "sample": what, "cpu": cpu_model()}
    try:
        import torch
        torch.set_num_threads(threads)
        tA = torch.from_numpy(np.ascontiguousarray(_host_view(A, ta, m, k, lda)[:rows]))
        tB = torch.from_numpy(np.ascontiguousarray(_host_view(B, tb, k, n, ldb)))
        tC = torch.from_numpy(np.ascontiguousarray(_host_view(C0, False, rows, n, ldc)))
        torch.addmm(tC, tA, tB, beta=beta, alpha=alpha)  # warm-up (thread pool, packing)
        times = []
        for _ in range(3):
            t = time.perf_counter()
            out = torch.addmm(tC, tA, tB, beta=beta, alpha=alpha)
            times.append(time.perf_counter() - t)
        dt_mkl = sorted(times)[1]
        base["value"] = round(2.0 * rows * n * k / dt_mkl / 1e12, 4)
        base["stand_in"] = (f"MKL {'sgemm' if fp32 else 'dgemm'} via torch.addmm on the CPU "
                            f"(BLAS_INFO=mkl), median of 3 after a warm-up, {dt_mkl:.3f} s: the "
                            f"vendor library of the reference's CPU path (oneMKL row_major::gemm "
                            f"on a SYCL CPU queue, src/ops/blas/level3/gemm.cpp:63), which "
                            f"cannot be built here")
        base["normwise_vs_gpu"] = oracle.rel_fro_err(out.numpy(),
                                                     np.ascontiguousarray(g[:rows]))
    except Exception as e:  # the port below still gives a number
        base["stand_in_error"] = str(e)[:200]
    Cp, dt = run_rows(rows, port_acc)
    port = {"value": round(2.0 * rows * n * k / dt / 1e12, 4), "unit": "TFLOP/s",
            "cores": threads, "kind": "port",
            "sample": f"{what}; oracle/sbo.c blocked OpenMP "
                      f"{'sgemm, fp32' if fp32 else 'dgemm, fp64'} accumulation, one run, "
                      f"{dt:.2f} s"}
    base["port"] = port
    if base["value"] is None:  # MKL unavailable: the port is the baseline
        base.update({k2: port[k2] for k2 in ("value", "kind", "sample")})
    # parity over the whole matrix against the double-accumulating oracle
    if not fp32 and rows == m:
        Cd = Cp  # the fp64 port already accumulates in double
    else:
        Cd, _ = run_rows(m, 1)
    truth = np.ascontiguousarray(_host_view(Cd, False, m, n, ldc))
    g = np.ascontiguousarray(g)
    err_truth = oracle.rel_fro_err(g, truth)
    err_port = oracle.rel_fro_err(np.ascontiguousarray(g[:rows]),
                                  np.ascontiguousarray(_host_view(Cp, False, rows, n, ldc)))
    parity = {"rows": m, "normwise_vs_oracle_f64acc": err_truth,
              "port_rows": rows, "normwise_vs_port": err_port, "tolerance": tol,
              "ok": bool(err_truth <= tol)}
    return base, parity


def vendor_headline(A, B, C, m, n, k, alpha, beta, steps, warmup):
    """The same headline GEMM through torch.addmm (the vendor BLAS, hipBLASLt
    on ROCm), fp32 with TF32 off, on the same device inputs, into a separate
    output, timed the same way: context for the headline, not part of it."""
    import torch
    try:
        torch.backends.cuda.matmul.allow_tf32 = False
        A2, B2, C2 = A.view(m, k), B.view(k, n), C.view(m, n)
        out = torch.empty_like(C2)

        def step():
            torch.addmm(C2, A2, B2, beta=beta, alpha=alpha, out=out)

        ms = time_launches(step, steps, warmup, min_warm_s=0.25)
        del out
        torch.cuda.empty_cache()
        return {"what": "torch.addmm (vendor BLAS) on the same inputs, fp32, TF32 off",
                "ms": round(ms, 4), "tflops": round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 3)}
    except Exception as e:  # context only; never fails the bench
        return {"error": str(e)[:200]}


def run_config(dtype, layout, ta, tb, m, n, k, alpha, beta, seed, steps, warmup, dist="uniform",
               cpu_s=None):
    """Allocate, fill and time one GEMM configuration; returns a dict.  With
    cpu_s (row-major only), the result of one call on the initial C is
    checked against the oracle over the whole matrix (`parity`) and the CPU
    path is timed on a sample of about cpu_s seconds (`cpu_baseline`)."""
    import torch
    import sushiblas_amd as sbx
    tdt = torch.float32 if dtype == "f32" else torch.float64
    sdt = sbx.F32 if dtype == "f32" else sbx.F64
    sa = (k, m) if ta else (m, k)
    sb = (n, k) if tb else (k, n)
    lda = sa[1] if layout == 0 else sa[0]
    ldb = sb[1] if layout == 0 else sb[0]
    ldc = n if layout == 0 else m
    A = torch.empty(m * k, dtype=tdt, device="cuda")
    B = torch.empty(k * n, dtype=tdt, device="cuda")
    C = torch.empty(m * n, dtype=tdt, device="cuda")
    if dist == "tall_skinny":
        sbx.fill_normal(A, seed, 0)
        sbx.fill_normal(B, seed, 1, 1.0 / k ** 0.5)
        C.zero_()
    else:
        sbx.fill_uniform(A, seed, 0)
        sbx.fill_uniform(B, seed, 1)
        if dist == "normal_c":
            sbx.fill_normal(C, seed, 2)
        else:
            sbx.fill_uniform(C, seed, 2)
    name = sbx.gemm_select(sdt, layout, ta, tb, m, n, k, lda, ldb, ldc)

    def step():
        sbx.gemm_ex(sdt, layout, ta, tb, m, n, k, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0)

    host = None
    if cpu_s is not None and layout == 0:
        torch.cuda.synchronize()
        host = (A.cpu().numpy(), B.cpu().numpy(), C.cpu().numpy())
        step()
        torch.cuda.synchronize()
        host = host + (C.cpu().numpy(),)
    flops = 2.0 * m * n * k
    probe = {"flops": flops, "dtype": dtype}
    ms = time_launches(step, steps, warmup, min_warm_s=0.25, probe=probe)
    tflops = flops / (ms * 1e-3) / 1e12
    nbytes = (m * k + k * n + m * n * (2 if beta != 0 else 1)) * A.element_size()
    out = {"kernel": name, "ms": round(ms, 4), "tflops": round(tflops, 3),
           "pct_peak": round(100 * tflops / PEAK[dtype], 2),
           "hbm_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    if probe.get("out"):
        out["probe"] = probe["out"]
    if VENDOR and layout == 0:
        # the same problem through torch (the vendor BLAS) on the same
        # device buffers, into a separate output, timed the same way
        try:
            opa = A.view(*sa).t() if ta else A.view(*sa)
            opb = B.view(*sb).t() if tb else B.view(*sb)
            c2, o2 = C.view(m, n), torch.empty(m, n, dtype=tdt, device="cuda")
            torch.backends.cuda.matmul.allow_tf32 = False
            vms = time_launches(lambda: torch.addmm(c2, opa, opb, beta=beta, alpha=alpha, out=o2),
                                steps, warmup, min_warm_s=0.25)
            out["vendor_ms"] = round(vms, 4)
            del o2
        except Exception as e:  # context only
            out["vendor_ms"] = None
            out["vendor_error"] = str(e)[:200]
    del A, B, C
    torch.cuda.empty_cache()
    if host is not None:
        out["cpu_baseline"], out["parity"] = cpu_leg(dtype, ta, tb, m, n, k, alpha, beta,
                                                     host[0], lda, host[1], ldb, host[2], ldc,
                                                     host[3], cpu_s)
    return out


def run_fused_config(m, n, k, seed, steps, warmup):
    """GEMM+ReLU as one fused launch (sbx_gemm_fused) against the unfused pair
    (sbx_gemm_ex, then sbx_relu over C): the caller pattern of the reference's
    integration tests (tests/runtime/test_framework_sim.cpp:51-57)."""
    import torch
    import sushiblas_amd as sbx
    A = torch.empty(m * k, dtype=torch.float32, device="cuda")
    B = torch.empty(k * n, dtype=torch.float32, device="cuda")
    C = torch.empty(m * n, dtype=torch.float32, device="cuda")
    sbx.fill_uniform(A, seed, 0)
    sbx.fill_uniform(B, seed, 1)
    C.zero_()

    def fused():
        sbx.gemm_fused(sbx.F32, 0, 0, 0, m, n, k, 1.0, A, k, 0, B, n, 0, 0.0, C, n, 0)

    def unfused():
        sbx.gemm_ex(sbx.F32, 0, 0, 0, m, n, k, 1.0, A, k, 0, B, n, 0, 0.0, C, n, 0)
        sbx.relu(C)

    ms_f = time_launches(fused, steps, warmup, min_warm_s=0.25)
    ms_u = time_launches(unfused, steps, warmup, min_warm_s=0.25)
    flops = 2.0 * m * n * k
    out = {"kernel": sbx.gemm_select(sbx.F32, 0, 0, 0, m, n, k, k, n, n) + "+relu",
           "ms": round(ms_f, 4), "tflops": round(flops / (ms_f * 1e-3) / 1e12, 3),
           "pct_peak": round(100 * flops / (ms_f * 1e-3) / 1e12 / PEAK["f32"], 2),
           "ms_unfused": round(ms_u, 4), "speedup_vs_unfused": round(ms_u / ms_f, 3)}
    del A, B, C
    torch.cuda.empty_cache()
    return out


def run_gemv_config(dtype, trans, m, n, seed, steps, warmup):
    """Row-major GEMV y = A x (or A^T x), beta = 0: HBM bound, so reported as
    GB/s of algorithmic traffic (A once, x once, y written) against 8 TB/s."""
    import torch
    import sushiblas_amd as sbx
    tdt = torch.float32 if dtype == "f32" else torch.float64
    sdt = sbx.F32 if dtype == "f32" else sbx.F64
    A = torch.empty(m * n, dtype=tdt, device="cuda")
    xlen, ylen = (m, n) if trans else (n, m)
    x = torch.empty(xlen, dtype=tdt, device="cuda")
    y = torch.zeros(ylen, dtype=tdt, device="cuda")
    sbx.fill_uniform(A, seed, 0)
    sbx.fill_uniform(x, seed, 1)

    def step():
        sbx.gemv(sdt, 0, trans, m, n, 1.0, A, n, x, 1, 0.0, y, 1)

    ms = time_launches(step, steps, warmup, min_warm_s=0.25)
    nbytes = (m * n + xlen + ylen) * A.element_size()
    gbs = nbytes / (ms * 1e-3) / 1e9
    out = {"kernel": "gemv_cols" if trans else "gemv_rows", "ms": round(ms, 4),
           "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
           "bytes": nbytes}
    del A, x, y
    torch.cuda.empty_cache()
    return out


def run_syrk_config(dtype, n, k, seed, steps, warmup):
    """Row-major SYRK, lower triangle of C = A A^T (A n x k), beta = 0;
    flops counted as n(n+1)k (the triangle including its diagonal)."""
    import torch
    import sushiblas_amd as sbx
    tdt = torch.float32 if dtype == "f32" else torch.float64
    sdt = sbx.F32 if dtype == "f32" else sbx.F64
    A = torch.empty(n * k, dtype=tdt, device="cuda")
    C = torch.zeros(n * n, dtype=tdt, device="cuda")
    sbx.fill_uniform(A, seed, 0)

    def step():
        sbx.syrk(sdt, 0, 0, 0, n, k, 1.0, A, k, 0, 0.0, C, n, 0)

    ms = time_launches(step, steps, warmup, min_warm_s=0.25)
    flops = float(n) * (n + 1) * k
    tflops = flops / (ms * 1e-3) / 1e12
    out = {"kernel": sbx.syrk_select(sdt, 0, 0, 0, n, k, k, n) + " (triangle tiles)",
           "ms": round(ms, 4), "tflops": round(tflops, 3),
           "pct_peak": round(100 * tflops / PEAK[dtype], 2)}
    del A, C
    torch.cuda.empty_cache()
    return out


def engine_patterns():
    """The C++ Engine path (Level3::gemm / NonLinearOps::relu recorded into the
    TaskGraph, then Engine::execute()) on the reference's integration patterns,
    timed by sushiblas_amd/lib/sushiblas_engine_bench: one lane vs all lanes."""
    import subprocess
    exe = os.path.join(ROOT, "sushiblas_amd", "lib", "sushiblas_engine_bench")
    res = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                         timeout=300)
    if res.returncode != 0:
        raise RuntimeError("sushiblas_engine_bench failed:\n" + res.stdout[-2000:])
    out = {}
    for line in res.stdout.splitlines():
        if line.startswith("{"):
            r = json.loads(line)
            e = out.setdefault(r["pattern"], {"tasks": r["tasks"]})
            e[f"us_per_batch_lanes{r['lanes']}"] = r["us_per_batch"]
    return out


def secondary_workloads(steps_arg, cpu_s=None):
    """The `also` workloads in run order, as key -> thunk.  cpu_s: CPU sample
    seconds for each BASELINE GEMM config's cpu_baseline / parity (None: skip)."""
    steps = max(3, min(steps_arg, 10))
    w = {}
    w["fp64_8192_cfg5"] = lambda: run_config("f64", 0, 0, 0, 8192, 8192, 8192, 1.0, 0.0,
                                             SEED + 5, steps, 2, cpu_s=cpu_s)
    for ta, tb in [(0, 0), (0, 1), (1, 0), (1, 1)]:
        w[f"fp32_ragged_cfg3_t{ta}{tb}"] = (lambda ta=ta, tb=tb: run_config(
            "f32", 0, ta, tb, 4095, 3001, 2047, 1.0, 1.0, SEED + 3, steps, 2, cpu_s=cpu_s))

    def tall_skinny():
        ts = run_config("f32", 0, 0, 0, 65536, 64, 4096, 1.0, 0.0, SEED + 4, steps, 2,
                        dist="tall_skinny", cpu_s=cpu_s)
        ts["hbm_frac"] = round(ts["hbm_gbs"] / HBM_PEAK_GBS, 4)
        return ts
    w["fp32_tall_skinny_cfg4"] = tall_skinny
    w["fp32_512_cfg1"] = lambda: run_config("f32", 0, 0, 0, 512, 512, 512, 1.0, 0.0, SEED + 1,
                                            steps * 5, 5, cpu_s=cpu_s)
    w["fp32_gemm_relu_layer_512x1024x1024"] = lambda: run_fused_config(
        512, 1024, 1024, SEED + 6, steps * 5, 5)
    w["fp32_gemm_relu_8192x8192x256"] = lambda: run_fused_config(8192, 8192, 256, SEED + 7,
                                                                 steps * 2, 3)
    w["fp32_gemv_16384x16384_n"] = lambda: run_gemv_config("f32", 0, 16384, 16384, SEED + 8,
                                                           steps * 2, 3)
    w["fp32_gemv_16384x16384_t"] = lambda: run_gemv_config("f32", 1, 16384, 16384, SEED + 8,
                                                           steps * 2, 3)
    w["fp64_gemv_16384x8192_n"] = lambda: run_gemv_config("f64", 0, 16384, 8192, SEED + 8,
                                                          steps * 2, 3)
    w["fp32_syrk_8192x8192"] = lambda: run_syrk_config("f32", 8192, 8192, SEED + 9, steps, 2)
    w["fp64_syrk_8192x8192"] = lambda: run_syrk_config("f64", 8192, 8192, SEED + 9, steps, 2)
    w["engine_task_graph"] = engine_patterns
    return w


def abba_tall_skinny(rounds, steps):
    """This build's tall-skinny call and torch.addmm
    (the vendor BLAS, TF32 off) on the same buffers, timed alternately in
    one process: `rounds` rounds of four measurements of `steps`
    back-to-back calls, in ABBA order (this build, vendor, vendor, this
    build) and its mirror on alternate rounds, each after 50 ms of its own
    warm-up, so that neither call always follows the other.  A single
    sequential pair, as in the `also` line, can put either ahead when the
    two are within the clock's run-to-run spread."""
    import statistics
    import torch
    import sushiblas_amd as sbx
    m, n, k = 65536, 64, 4096
    A = torch.empty(m * k, device="cuda")
    B = torch.empty(k * n, device="cuda")
    C = torch.zeros(m * n, device="cuda")
    sbx.fill_normal(A, SEED + 4, 0)
    sbx.fill_normal(B, SEED + 4, 1, 1.0 / k ** 0.5)
    A2, B2, C2 = A.view(m, k), B.view(k, n), C.view(m, n)
    out = torch.empty(m, n, device="cuda")
    torch.backends.cuda.matmul.allow_tf32 = False
    calls = {"sbx": lambda: sbx.gemm_ex(sbx.F32, 0, 0, 0, m, n, k, 1.0, A, k, 0, B, n, 0, 0.0,
                                        C, n, 0),
             "vendor": lambda: torch.addmm(C2, A2, B2, beta=0.0, alpha=1.0, out=out)}
    for fn in calls.values():
        time_launches(fn, steps, 5, min_warm_s=0.5)
    seq, res = [], {key: [] for key in calls}
    for r in range(rounds):
        order = ("sbx", "vendor", "vendor", "sbx") if r % 2 == 0 else ("vendor", "sbx", "sbx",
                                                                        "vendor")
        for key in order:
            us = time_launches(calls[key], steps, 3, min_warm_s=0.05) * 1e3
            res[key].append(us)
            seq.append([key, round(us, 1)])
    return {"workload": "fp32 65536x64x4096 (configs[3]): this build and torch.addmm, "
                        "interleaved ABBA", "steps_per_measurement": steps,
            "median_us": {key: round(statistics.median(v), 1) for key, v in res.items()},
            "min_us": {key: round(min(v), 1) for key, v in res.items()},
            "max_us": {key: round(max(v), 1) for key, v in res.items()},
            "sequence_us": seq}


def k_sweep(steps):
    """512 x 512 x K (fp32, row-major, no transpose, alpha = 1, beta = 0) on
    both forms of the small-problem kernel, run by name (sbx_gemm_ex_plan:
    K cut over 8 waves and over 4), with the probe build's stamps:
    event-timed call time, the dispatch's span and the workgroups' phases;
    time = intercept + slope * K fitted over each form's rows.  Each row
    also names the library's own pick for that K."""
    import numpy as np
    import torch
    import sushiblas_amd as sbx
    m = n = 512
    rows = []
    for k in (64, 128, 192, 256, 384, 512, 640, 768, 1024, 1280, 1536, 2048):
        A = torch.empty(m * k, dtype=torch.float32, device="cuda")
        B = torch.empty(k * n, dtype=torch.float32, device="cuda")
        C = torch.zeros(m * n, dtype=torch.float32, device="cuda")
        sbx.fill_uniform(A, SEED + 1, 0)
        sbx.fill_uniform(B, SEED + 1, 1)
        pick = sbx.gemm_select(sbx.F32, 0, 0, 0, m, n, k, k, n, n)
        for name in ("mfma_f32_32x32_ksplit8", "mfma_f32_32x32_ksplit4"):

            def step():
                sbx.gemm_ex_plan(sbx.F32, 0, 0, 0, m, n, k, 1.0, A, k, 0, B, n, 0, 0.0, C, n, 0,
                                 1, name)

            probe = {"flops": 2.0 * m * n * k, "dtype": "f32"}
            ms = time_launches(step, steps, 5, min_warm_s=0.25, probe=probe)
            rows.append({"k": k, "kernel": name, "pick": pick, "us": round(ms * 1e3, 3),
                         "probe": probe.get("out")})
        del A, B, C
    fits = {}
    for form, name in (("8wave", "mfma_f32_32x32_ksplit8"), ("4wave", "mfma_f32_32x32_ksplit4")):
        pts = [r for r in rows if r["kernel"] == name and r["probe"]]
        if len(pts) < 2:
            continue
        ks = np.array([r["k"] for r in pts], dtype=np.float64)
        fit = {"k": [r["k"] for r in pts]}
        for key, ys in (("call_us", [r["us"] for r in pts]),
                        ("span_us", [r["probe"]["span_us"] for r in pts])):
            slope, icpt = np.polyfit(ks, np.array(ys), 1)
            fit[key] = {"intercept_us": round(float(icpt), 3), "us_per_k": round(float(slope), 6)}
        fits[form] = fit
    return {"workload": "fp32 512 x 512 x K sweep (small-problem kernel)", "rows": rows,
            "fit": fits,
            "mfma_floor_us_per_k": round(2.0 * m * n / (256 * torch.cuda.get_device_properties(0)
                                                        .multi_processor_count * 2.4e9) * 1e6, 6)}


def regret_shapes(seed, count):
    """A seeded list of GEMM problems for judging the kernel-selection model:
    fp32 (70 %) and fp64, both layouts, all four transposes; unbatched with
    m, n, k log-uniform in [64, 8192], or (a quarter) strided batches of 2-64
    entries with sides in [32, 1024]; resampled until 2mnk*batch lies in
    [1e8, 4e11] flop (each call about 2 us to 5 ms)."""
    import numpy as np
    rng = np.random.RandomState(seed)
    out = []
    while len(out) < count:
        dtype = "f32" if rng.rand() < 0.7 else "f64"
        layout, ta, tb = (int(x) for x in rng.randint(0, 2, 3))
        if rng.rand() < 0.25:
            batch = int(rng.choice([2, 4, 8, 16, 32, 64]))
            m, n, k = (int(np.exp(rng.uniform(np.log(32), np.log(1024)))) for _ in range(3))
        else:
            batch = 1
            m, n, k = (int(np.exp(rng.uniform(np.log(64), np.log(8192)))) for _ in range(3))
        flops = 2.0 * m * n * k * batch
        if not 1e8 <= flops <= 4e11:
            continue
        out.append((dtype, layout, ta, tb, m, n, k, batch))
    return out


def regret_syrk_shapes(seed, count):
    """A seeded list of SYRK problems (the triangle's plans): fp32 (70 %) and
    fp64, both layouts, triangles and transposes; n and k log-uniform in
    [64, 8192], resampled until n^2 k lies in [1e8, 4e11] flop."""
    import numpy as np
    rng = np.random.RandomState(seed + 7919)
    out = []
    while len(out) < count:
        dtype = "f32" if rng.rand() < 0.7 else "f64"
        layout, upper, trans = (int(x) for x in rng.randint(0, 2, 3))
        n, k = (int(np.exp(rng.uniform(np.log(64), np.log(8192)))) for _ in range(2))
        if not 1e8 <= float(n) * n * k <= 4e11:
            continue
        out.append((dtype, layout, upper, trans, n, k))
    return out


def _time_plans(call, plans):
    """Times of the pick (call(None)) and of every named plan, in ms: each the
    faster of two passes (plans in order, then reversed) of back-to-back
    calls, about 2 ms of the pick's work per timing."""
    import torch
    import sushiblas_amd as sbx
    call(None)
    torch.cuda.synchronize()
    t0 = time_launches(lambda: call(None), 3, 1)
    reps = int(max(3, min(200, 2.0 / max(t0, 1e-3))))
    names = [None] + [pn for pn, _ in plans]
    times = {}
    for order in (names, names[::-1]):
        for pn in order:
            try:
                ms = time_launches(lambda: call(pn), reps, 2)
            except sbx.SbxError:
                continue
            times[pn] = min(times.get(pn, float("inf")), ms)
    return times


def _regret_row(r, pick, plans, times, flops, full):
    best = min((t, pn) for pn, t in times.items() if pn is not None)
    r.update({"pick": pick, "pick_us": round(times[None] * 1e3, 2), "best": best[1],
              "best_us": round(best[0] * 1e3, 2), "regret": round(times[None] / best[0] - 1.0, 4),
              "plans": len(times) - 1,
              "pick_tflops": round(flops / (times[None] * 1e-3) / 1e12, 2)})
    if full:  # every plan's measured and predicted microseconds
        pred = dict(plans)
        r["times"] = {pn: [round(t * 1e3, 3), pred[pn]] for pn, t in times.items()
                      if pn is not None}
    print(json.dumps(r), file=sys.stderr, flush=True)
    return r


def _regret_summary(rows):
    import numpy as np
    if not rows:
        return None
    reg = np.array([r["regret"] for r in rows])
    return {"shapes": len(rows), "mean_regret": round(float(reg.mean()), 4),
            "median_regret": round(float(np.median(reg)), 4),
            "p90_regret": round(float(np.percentile(reg, 90)), 4),
            "max_regret": round(float(reg.max()), 4), "within_2pct": int((reg <= 0.02).sum()),
            "within_10pct": int((reg <= 0.10).sum())}


def regret(seed, count, full=False, syrk_count=0):
    """For each shape of regret_shapes(seed, count) and
    regret_syrk_shapes(seed, syrk_count): the time of the pick (sbx_gemm_ex,
    algo AUTO; sbx_{s,d}syrk_strided_batched) and of every plan the heuristics
    weigh (sbx_gemm_plans / sbx_syrk_plans, run through sbx_gemm_ex_plan /
    sbx_syrk_ex_plan); regret = pick / fastest - 1.  full: keep every plan's
    measured and predicted time in its row (for fitting the model)."""
    import torch
    import sushiblas_amd as sbx
    rows, srows = [], []
    for si, (dtype, layout, ta, tb, m, n, k, batch) in enumerate(regret_shapes(seed, count)):
        code = sbx.F32 if dtype == "f32" else sbx.F64
        tdt = torch.float32 if dtype == "f32" else torch.float64
        rows_a = m if (layout == 0) == (not ta) else k
        cols_a = k if (layout == 0) == (not ta) else m
        rows_b = k if (layout == 0) == (not tb) else n
        cols_b = n if (layout == 0) == (not tb) else k
        rows_c, cols_c = (m, n) if layout == 0 else (n, m)
        lda, ldb, ldc = cols_a, cols_b, cols_c  # packed: the stored row length
        sa, sb, sc = rows_a * lda, rows_b * ldb, rows_c * ldc
        A = torch.empty(sa * batch, dtype=tdt, device="cuda")
        B = torch.empty(sb * batch, dtype=tdt, device="cuda")
        C = torch.zeros(sc * batch, dtype=tdt, device="cuda")
        sbx.fill_uniform(A, SEED + si, 0)
        sbx.fill_uniform(B, SEED + si, 1)
        pick = sbx.gemm_select(code, layout, ta, tb, m, n, k, lda, ldb, ldc, batch=batch)
        plans = sbx.gemm_plans(code, layout, ta, tb, m, n, k, lda, ldb, ldc, batch)

        def call(plan):
            if plan is None:
                sbx.gemm_ex(code, layout, ta, tb, m, n, k, 1.0, A, lda, sa, B, ldb, sb, 0.0, C,
                            ldc, sc, batch)
            else:
                sbx.gemm_ex_plan(code, layout, ta, tb, m, n, k, 1.0, A, lda, sa, B, ldb, sb, 0.0,
                                 C, ldc, sc, batch, plan)

        times = _time_plans(call, plans)
        r = {"op": "gemm", "dtype": dtype, "layout": layout, "ta": ta, "tb": tb, "m": m, "n": n,
             "k": k, "batch": batch}
        rows.append(_regret_row(r, pick, plans, times, 2.0 * m * n * k * batch, full))
        del A, B, C
        torch.cuda.empty_cache()
    for si, (dtype, layout, upper, trans, n, k) in enumerate(regret_syrk_shapes(seed, syrk_count)):
        code = sbx.F32 if dtype == "f32" else sbx.F64
        tdt = torch.float32 if dtype == "f32" else torch.float64
        lda = (k if not trans else n) if layout == 0 else (n if not trans else k)
        A = torch.empty(n * k, dtype=tdt, device="cuda")
        C = torch.zeros(n * n, dtype=tdt, device="cuda")
        sbx.fill_uniform(A, SEED + 500 + si, 0)
        pick = sbx.syrk_select(code, layout, upper, trans, n, k, lda, n)
        plans = sbx.syrk_plans(code, layout, upper, trans, n, k, lda, n)

        def call(plan):
            if plan is None:
                sbx.syrk(code, layout, upper, trans, n, k, 1.0, A, lda, 0, 0.0, C, n, 0)
            else:
                sbx.syrk_ex_plan(code, layout, upper, trans, n, k, 1.0, A, lda, 0, 0.0, C, n, 0,
                                 1, plan)

        times = _time_plans(call, plans)
        r = {"op": "syrk", "dtype": dtype, "layout": layout, "upper": upper, "trans": trans,
             "n": n, "k": k}
        srows.append(_regret_row(r, pick, plans, times, float(n) * n * k, full))
        del A, C
        torch.cuda.empty_cache()
    worst = sorted(rows + srows, key=lambda r: -r["regret"])[:8]
    if not full:
        worst = [{key: v for key, v in r.items() if key != "times"} for r in worst]
    return {"workload": f"kernel-selection regret, regret_shapes({seed}, {count}) and "
                        f"regret_syrk_shapes({seed}, {syrk_count})",
            "gemm": _regret_summary(rows), "syrk": _regret_summary(srows),
            "worst": worst, "rows": rows + srows}


def main():
    global VENDOR, PROBE
    args = parse()
    VENDOR = not args.no_vendor
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.probe:
        import sushiblas_amd as sbx
        PROBE = True
        sbx.use_probe_library()
    if args.regret is not None:
        import sushiblas_amd as sbx
        sbx.lib()
        print(json.dumps(regret(args.regret, args.regret_count, args.regret_full,
                                args.regret_syrk)), flush=True)
        return
    if args.hbm_rates:
        print(json.dumps(hbm_rates()), flush=True)
        return
    if args.abba is not None:
        print(json.dumps(abba_tall_skinny(max(1, args.abba), args.steps)), flush=True)
        return
    if args.k_sweep:
        if not args.probe:
            print("--k-sweep needs --probe", file=sys.stderr)
            sys.exit(2)
        import sushiblas_amd as sbx
        sbx.lib()
        print(json.dumps(k_sweep(max(args.steps, 20))), flush=True)
        return
    if args.only:
        import sushiblas_amd as sbx
        sbx.lib()
        work = secondary_workloads(args.steps, None if args.no_cpu else args.cpu_seconds)
        if args.only not in work:
            print(f"unknown workload {args.only!r}; one of: {', '.join(work)}", file=sys.stderr)
            sys.exit(2)
        print(json.dumps({"workload": args.only, **work[args.only]()}), flush=True)
        return
    import numpy as np
    import torch
    import sushiblas_amd as sbx
    sbx.lib()

    m = n = k = 8192
    alpha, beta = 1.5, 0.5
    seed = SEED + 2
    A = torch.empty(m * k, dtype=torch.float32, device="cuda")
    B = torch.empty(k * n, dtype=torch.float32, device="cuda")
    C = torch.empty(m * n, dtype=torch.float32, device="cuda")
    sbx.fill_uniform(A, seed, 0)
    sbx.fill_uniform(B, seed, 1)
    sbx.fill_normal(C, seed, 2)
    torch.cuda.synchronize()
    kernel = sbx.gemm_select(sbx.F32, 0, 0, 0, m, n, k, k, n, n)

    # one call on the initial C for the parity check / CPU baseline
    need_host = not args.no_cpu
    if need_host:
        A_h = A.cpu().numpy()
        B_h = B.cpu().numpy()
        C0_h = C.cpu().numpy()
    sbx.sgemm(0, 0, 0, m, n, k, alpha, A, k, B, n, beta, C, n)
    torch.cuda.synchronize()
    if need_host:
        got_h = C.cpu().numpy()

    def step():
        sbx.sgemm(0, 0, 0, m, n, k, alpha, A, k, B, n, beta, C, n)

    flops = 2.0 * m * n * k
    probe = {"flops": flops, "dtype": "f32"}
    ms = time_launches(step, args.steps, args.warmup, probe=probe)
    value = flops / (ms * 1e-3) / 1e12
    traffic = read_traffic("headline")
    vendor = None if args.no_vendor else vendor_headline(A, B, C, m, n, k, alpha, beta,
                                                         args.steps, args.warmup)
    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: Philox4x32-10 A,B ~ U[-1,1), C ~ N(0,1), seed 20261203, in HBM",
        "config": {"workload": "fp32 GEMM C = 1.5*A*B + 0.5*C, row-major, no transpose, "
                               "M=N=K=8192 (BASELINE configs[1])",
                   "m": m, "n": n, "k": k, "alpha": alpha, "beta": beta, "kernel": kernel},
        "roofline": {"bound": "mfma", "achieved": round(value, 3), "peak": PEAK["f32"],
                     "unit": "TFLOP/s", "frac": round(value / PEAK["f32"], 4),
                     "traffic": traffic},
    }
    if vendor is not None:
        result["vendor"] = vendor
    if PROBE:
        result["library"] = "probe build (lib/libsbx_probe.so): per-workgroup clock stamps"
        result["probe"] = probe.get("out")
    if need_host:
        del A, B
        torch.cuda.empty_cache()
        base, parity = cpu_leg("f32", 0, 0, m, n, k, alpha, beta, A_h, k, B_h, n, C0_h, n,
                               got_h, args.cpu_seconds)
        result["cpu_baseline"] = base
        result["parity"] = parity
    else:
        result["cpu_baseline"] = None
    del C
    torch.cuda.empty_cache()

    if not args.no_also:
        also = {}
        for key, fn in secondary_workloads(args.steps,
                                           None if args.no_cpu else args.cpu_seconds).items():
            also[key] = fn()
            if key != "engine_task_graph":
                also[key]["traffic"] = read_traffic(key)
        result["also"] = also
    print(json.dumps(result), flush=True)
    del np


if __name__ == "__main__":
    main()
