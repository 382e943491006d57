"""bench.py's counter summaries and its one-GPU guard (CPU: synthetic
rocprofv3 CSV files, nothing runs on a GPU).

The committed profiles/qgemm_ns_counters.json and the `roofline.traffic`
figure come from `bench.py --summarize-counters`; the small-M and latency
tables from `bench.py --kernel-counters`. These tests feed both known counter
values and check the arithmetic: the byte counters scaled by what they read
for the calibration copy of known size, MFMA busy over active cycles per XCD
and SIMD, L2 hit fraction, and the wait / latency / LDS ratios.
"""
import csv
import json
import os
import subprocess
import sys

import pytest

from conftest import ROOT

BENCH = os.path.join(ROOT, "bench.py")
K256 = "void sdq::(anonymous namespace)::qgemm_persist<256, 256, 2, 4, 2, 4, 1, 0, true, false>(int)"
K128 = "void sdq::(anonymous namespace)::qgemm_persist<128, 128, 2, 2, 2, 4, 2, 0, true, false>(int)"
KQ = "void sdq::(anonymous namespace)::act_quant_units_kernel<8, 8, 3, false, false>(float const*)"
KCOPY = "__amd_rocclr_copyBuffer"


def _write(d, rows):
    """rows: (kernel, counter, value, dispatch, start_ns, end_ns)."""
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "p_counter_collection.csv"), "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value",
                    "Start_Timestamp", "End_Timestamp"])
        for k, c, v, disp, t0, t1 in rows:
            w.writerow([disp, k, c, v, t0, t1])


def _bench(*args):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True,
                          timeout=120)


def test_summarize_counters_arithmetic(tmp_path):
    d = {n: str(tmp_path / n) for n in ("fetch", "write", "mfma", "tcc")}
    # the calibration copy reads 1 GiB (FETCH_SIZE reports half: x2.0) and writes 1 GiB (x1.0)
    _write(d["fetch"], [(KCOPY, "FETCH_SIZE", 524288, 9, 0, 1),
                        (K256, "FETCH_SIZE", 1_000_000, 1, 0, 1),
                        (K256, "FETCH_SIZE", 1_200_000, 2, 0, 1),
                        (KQ, "FETCH_SIZE", 160_000, 3, 0, 1)])
    _write(d["write"], [(KCOPY, "WRITE_SIZE", 1048576, 9, 0, 1),
                        (K256, "WRITE_SIZE", 1_500_000, 1, 0, 1),
                        (KQ, "WRITE_SIZE", 80_000, 3, 0, 1)])
    _write(d["mfma"], [(K256, "SQ_VALU_MFMA_BUSY_CYCLES", 6_144_000, 1, 0, 1),
                       (K256, "GRBM_GUI_ACTIVE", 80_000, 1, 0, 1),
                       (K128, "SQ_VALU_MFMA_BUSY_CYCLES", 1_024, 4, 0, 1),
                       (K128, "GRBM_GUI_ACTIVE", 80, 4, 0, 1)])
    _write(d["tcc"], [(K256, "TCC_HIT_sum", 70, 1, 0, 1), (K256, "TCC_MISS_sum", 30, 1, 0, 1)])
    meta = {"profile_pass": True, "copy_bytes": 1 << 30, "M": 27280, "K": 3072, "N": 14336,
            "library": "sdq test", "plan": [["qgemm_tile256x256", 0, 26880]], "cu_count": 256}
    with open(d["fetch"] + ".log", "w") as f:
        f.write("rocprofv3 noise\n" + json.dumps(meta) + "\n")
    out = str(tmp_path / "c.json")
    r = _bench("--summarize-counters", *d.values(), "--counters-json", out)
    assert r.returncode == 0, r.stderr
    s = json.load(open(out))
    assert s["workload"] == "27280x3072x14336" and s["library"] == "sdq test"
    assert s["calibration"]["fetch_scale"] == pytest.approx(2.0)
    assert s["calibration"]["write_scale"] == pytest.approx(1.0)
    k = s["kernels"]["qgemm_tile256x256"]
    assert k["fetch_bytes"] == 1_100_000 * 1024 * 2  # mean of the two dispatches, x2.0
    assert k["write_bytes"] == 1_500_000 * 1024
    assert k["hbm_bytes_per_launch"] == k["fetch_bytes"] + k["write_bytes"]
    # 6.144e6 busy cycles over (80000 / 8 XCDs) x 256 CUs x 4 SIMDs
    assert k["mfma_busy_frac"] == pytest.approx(0.6, abs=1e-4)
    assert k["active_cycles_per_xcd"] == 10_000
    assert k["l2_hit_frac"] == pytest.approx(0.7) and k["l2_requests"] == 100
    assert s["kernels"]["qgemm_tail128"]["mfma_busy_frac"] == pytest.approx(0.1, abs=1e-4)
    q = s["kernels"]["act_quant"]
    assert q["fetch_bytes"] == 160_000 * 2048 and q["write_bytes"] == 80_000 * 1024
    assert "copy" not in s["kernels"]


def test_summarize_counters_needs_the_pass_line(tmp_path):
    d = str(tmp_path / "fetch")
    _write(d, [(K256, "FETCH_SIZE", 1, 1, 0, 1)])
    r = _bench("--summarize-counters", d, "--counters-json", str(tmp_path / "c.json"))
    assert r.returncode != 0 and "no --profile-pass output line" in r.stderr


def test_kernel_counters_derived_ratios(tmp_path):
    d = str(tmp_path / "lat")
    _write(d, [(K256, "SQ_WAIT_INST_ANY", 440, 1, 1_000, 1_001_000),
               (K256, "SQ_WAVE_CYCLES", 1000, 1, 1_000, 1_001_000),
               (K256, "TCP_TCC_READ_REQ_LATENCY_sum", 217_000, 1, 1_000, 1_001_000),
               (K256, "TCP_TCC_READ_REQ_sum", 1000, 1, 1_000, 1_001_000),
               (K256, "SQ_LDS_BANK_CONFLICT", 0, 1, 1_000, 1_001_000),
               (K256, "SQ_INSTS_LDS", 5000, 1, 1_000, 1_001_000),
               (K256, "SQ_WAIT_INST_ANY", 460, 2, 0, 998_000),
               (K256, "SQ_WAVE_CYCLES", 1000, 2, 0, 998_000)])
    r = _bench("--kernel-counters", d)
    assert r.returncode == 0, r.stderr
    k = json.loads(r.stdout)["kernels"]["sdq::qgemm_persist<256, 256, 2, 4, 2, 4, 1, 0, true, false>"]
    assert k["wait_frac"] == pytest.approx(0.45)  # mean 450 over mean 1000
    assert k["l2_read_latency_cycles"] == pytest.approx(217.0)
    assert k["lds_conflict_cycles_per_inst"] == 0
    assert k["us_mean"] == pytest.approx(999.0)  # (1000 + 998) / 2 microseconds
    assert k["dispatches"] == 2


def test_bench_refuses_more_than_one_gpu():
    r = _bench("--gpus", "2")
    assert r.returncode == 2 and "--gpus must be 1" in r.stderr
