"""Host-side parts of bench.py's contract (no GPU): the multi-GPU refusal and
the HBM-traffic figures it reads from the committed rocprofv3 summary."""
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def test_traffic_is_read_from_the_bytes_column():
    """roofline.traffic is the measured bytes per launch: FETCH_SIZE and
    WRITE_SIZE (KiB) scaled by the copy-kernel factors of the same file."""
    import bench
    text = open(os.path.join(ROOT, "profiles", "hbm_traffic.md")).read()
    m = re.search(r"FETCH_SIZE is scaled by ([0-9.]+) and WRITE_SIZE by ([0-9.]+)", text)
    ff, fw = float(m.group(1)), float(m.group(2))
    rows = {}
    for line in text.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if line.startswith("|") and len(cells) == 7 and cells[2][:1].isdigit():
            rows[cells[0]] = cells
    assert "headline" in rows
    for workload, cells in rows.items():
        got = bench.read_traffic(workload)
        fetch, write = (float(c.replace(",", "")) for c in cells[2:4])
        algorithmic = int(cells[4].replace(",", ""))
        assert isinstance(got, int)
        # the KiB columns are rounded averages: agree to 0.1 %
        assert abs(got - (fetch * ff + write * fw) * 1024) <= 1e-3 * got + 4096, workload
        assert abs(got / algorithmic - float(cells[6])) < 0.006, workload
    assert bench.read_traffic("no_such_workload") is None


def test_cpu_leg_reports_the_mkl_stand_in_with_the_port_nested():
    """cpu_baseline.value is the reference CPU path's stand-in (MKL through
    torch's CPU addmm); the oracle port is nested under `port`; parity covers
    the whole matrix.  A problem large enough to time (the rates are rounded
    to 1e-4 TFLOP/s), small enough to run in about a second."""
    import numpy as np
    import bench
    import oracle
    m, n, k = 384, 320, 256
    A = oracle.fill_uniform(m * k, np.float32, 7, 0)
    B = oracle.fill_uniform(k * n, np.float32, 7, 1)
    C = oracle.fill_uniform(m * n, np.float32, 7, 2)
    got = C.copy()
    oracle.gemm(0, 0, 0, m, n, k, 1.5, A, k, B, n, 0.5, got, n, 1)
    base, parity = bench.cpu_leg("f32", 0, 0, m, n, k, 1.5, 0.5, A, k, B, n, C, n, got, 0.01)
    assert base["kind"] == "reference" and base["value"] > 0 and "MKL" in base["stand_in"]
    assert base["normwise_vs_gpu"] <= 1e-5
    assert base["port"]["kind"] == "port" and base["port"]["value"] > 0
    assert parity["ok"] and parity["rows"] == m


def test_probe_summary_on_synthetic_stamps():
    """bench.probe_summary recovers the clock, span and MFMA busy from stamps
    of a known timeline: 256 workgroups (one per CU) of 524288 MFMA cycles
    of work each, run at 2.0 GHz with 80 % of the cycles busy, entries 0.5 us
    apart; the small-problem kernel's four points give its phase times."""
    import numpy as np
    import bench
    khz, cus, clock = 100000, 256, 2.0e9
    ring, blocks, P = 3, bench.PROBE_BLOCKS, bench.PROBE_POINTS
    t = np.zeros((ring, blocks, P, 2), np.uint64)
    work = 524288 / 0.8  # cycles per workgroup
    for d in range(2):
        for b in range(cus):
            t0 = 1_000_000 + d * 100_000 + b * 0.05e-6 * khz * 1e3  # ticks
            c0 = 7_000_000 + b * 1000
            t[d, b, 0] = (c0, t0)
            t[d, b, 1] = (c0 + work, t0 + work / clock * khz * 1e3)
    flops = 524288.0 * 256 * cus  # a whole chip of that work
    out = bench.probe_summary(t.reshape(-1), 2, flops, "f32", 0.5, khz, cus)
    assert out["dispatches"] == 2
    assert abs(out["clock_ghz"] - 2.0) < 1e-3
    span = work / clock * 1e6 + 255 * 0.05  # us
    assert abs(out["span_us"] - span) < 0.02
    assert abs(out["mfma_busy_span"] - 0.8 * (work / clock * 1e6) / span) < 1e-3
    assert out["wg_cycles"] == round(work)
    # the small-problem kernel's phases
    s = np.zeros((1, blocks, P, 2), np.uint64)
    for b in range(8):
        s[0, b] = [(100 + b, 1000), (300 + b, 1100), (900 + b, 1400), (1100 + b, 1500)]
    out = bench.probe_summary(s.reshape(-1), 1, 1.0, "f32", 0.01, khz, cus)
    assert out["wg_us"] == {"issue_first_loads": 1.0, "to_mfma_done": 3.0, "reduce_and_store": 1.0}
    assert out["clock_ghz"] == 0.2 and out["launch_spread_us"] == 0.0
