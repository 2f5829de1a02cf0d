"""bench.py's host-side arithmetic, without a GPU.

The pair counts set every TFLOP/s figure the bench prints, so they are held to
the oracle's closed-form count (itself pinned by brute force in
test_oracle.py). The roofline is checked against the bound it defines, the
rocprofv3 counter summary against a synthetic counter file whose figures are
known, and the bench's one-GPU rule through its command line.
"""
import csv
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from oracle import cra_oracle as O  # noqa: E402


@pytest.mark.parametrize("S", [1, 2, 3, 100, 363, 2048, 2049, 5000, 16384, 131072])
def test_pairs_fast_matches_oracle(S):
    assert bench.pairs_fast(S) == O.pair_count(O.make_plan(S))


def test_north_star_pairs_and_phases():
    """The per-head pair counts behind the headline figures (W = 363,
    relay top-2)."""
    assert bench.pairs_fast(131072) == 118047362
    assert bench.phase_pairs(131072) == {"local": 47513433, "strided": 23598209,
                                         "relay": 46935720}


@pytest.mark.parametrize("S", [100, 2048, 2049, 65536])
def test_phase_pairs_sum_to_total(S):
    assert sum(bench.phase_pairs(S).values()) == bench.pairs_fast(S)
    assert bench.row_pairs(range(S), S) == bench.pairs_fast(S)


def test_relay_phase_only_above_2048():
    assert bench.phase_pairs(2048)["relay"] == 0
    assert bench.phase_pairs(2049)["relay"] > 0


def test_roofline_bounds():
    # north star forward: MFMA-bound, F = 4 D P B H
    t, bound, F = bench.roofline_ms(1, 16, 131072, 128, 2, False)
    assert F == 4 * 128 * 118047362 * 16
    assert bound == "mfma"
    assert t == pytest.approx(F / (bench.PEAK_FP16_TFLOPS * 1e12) * 1e3)
    # training counts 14 D flop per pair
    _, _, Ft = bench.roofline_ms(1, 16, 131072, 128, 2, True)
    assert Ft == 14 * 128 * 118047362 * 16
    # a short sequence moves more bytes than it computes: HBM-bound, bytes / 8 TB/s
    t2, b2, _ = bench.roofline_ms(1, 8, 2048, 64, 2, False)
    assert b2 == "hbm"
    nbytes = 8 * (4 * 2048 * 64 * 2 + 4 * 2048)
    assert t2 == pytest.approx(nbytes / (bench.PEAK_HBM_GBS * 1e9) * 1e3)


def _write_counters(path, rows):
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "run_counter_collection.csv"), "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value",
                    "Start_Timestamp", "End_Timestamp"])
        for r in rows:
            w.writerow(r)


def test_counter_summary_known_figures(tmp_path):
    """One dispatch of the forward with counters chosen so that every derived
    column has a known value, beside the copy kernel that calibrates bytes."""
    fwd = "_ZN3cra12_GLOBAL__N_111fwd2_kernelIDF16_Li128ELi4ELi3EEEvNS_7FwdArgsE"
    copy = "__amd_rocclr_copyBuffer"
    _write_counters(str(tmp_path / "A"), [
        (1, copy, "FETCH_SIZE", 524288, 0, 1000),
        (1, copy, "WRITE_SIZE", 1048576, 0, 1000),
        (2, fwd, "SQ_INSTS_MFMA", 1000, 5000, 7000),            # 2000 ns
        (2, fwd, "SQ_VALU_MFMA_BUSY_CYCLES", 16000, 5000, 7000),
        (2, fwd, "GRBM_GUI_ACTIVE", 8 * 3000, 5000, 7000),       # 3000 cycles per XCD
        (2, fwd, "SQ_INSTS_VALU", 4000, 5000, 7000),
        (2, fwd, "SQ_INSTS_LDS", 500, 5000, 7000),
        (2, fwd, "SQ_LDS_BANK_CONFLICT", 250, 5000, 7000),
        (2, fwd, "SQ_WAVE_CYCLES", 400, 5000, 7000),
        (2, fwd, "SQ_WAIT_ANY", 100, 5000, 7000),
        (2, fwd, "FETCH_SIZE", 1000, 5000, 7000),
        (2, fwd, "WRITE_SIZE", 2000, 5000, 7000),
    ])
    out = bench.counter_summary([str(tmp_path / "A")], cus=256, xcds=8)
    line = next(l for l in out.splitlines() if l.startswith("| `fwd2_kernel<f16, 128, 4, 3>`"))
    cells = [c.strip() for c in line.strip("|").split("|")]
    # MFMA busy = 16000 / (3000 cycles x 256 CUs x 4 SIMDs)
    assert cells[2] == f"{16000 / (3000 * 1024):.1%}"
    assert cells[3] == "4.00"                      # VALU per MFMA
    assert cells[6] == "0.50"                      # LDS per MFMA
    assert cells[7] == "0.50"                      # conflict cycles per LDS instruction
    assert cells[8] == "25.0%"                     # waiting share of wave time
    assert cells[9] == "1.50"                      # 3000 cycles in 2000 ns
    assert cells[10] == f"{1000 * 1024 * 2 / 1e6:.1f}"   # FETCH_SIZE counts half the bytes read
    assert cells[11] == f"{2000 * 1024 / 1e6:.1f}"
    assert "Calibration" in out and "524288 KiB" in out


def test_mfma_busy_needed():
    # no executed overhead (one MFMA per 16384 algorithmic flops): the busy
    # share needed equals the target fraction times nominal peak over the
    # matrix cores' rate at that clock (256 CUs x 4 SIMDs x 1024 flop/cycle)
    flops = 3384.65e9
    n = flops / bench.MFMA_FLOPS
    rate = bench.CUS * 4 * bench.MFMA_FLOPS / 16  # flop per cycle
    for clock in (1.8, 2.4):
        want = 0.5 * bench.PEAK_FP16_TFLOPS * 1e12 / (rate * clock * 1e9)
        assert abs(bench.mfma_busy_needed(n, flops, clock, 0.5) - want) < 1e-12
    # twice the executed work needs twice the busy share; half the target, half
    assert abs(bench.mfma_busy_needed(2 * n, flops, 2.4, 0.5)
               - 2 * bench.mfma_busy_needed(n, flops, 2.4, 0.5)) < 1e-12
    assert abs(bench.mfma_busy_needed(n, flops, 2.4, 0.25)
               - 0.5 * bench.mfma_busy_needed(n, flops, 2.4, 0.5)) < 1e-12
    # the committed north-star counters: about 0.91 at their sustained clock
    ex = bench.executed_for("H16_D128_S131072_fp16")
    if ex:
        need = bench.mfma_busy_needed(sum(ex["mfma_per_launch"].values()), flops,
                                      ex["clock_ghz"], 0.5)
        assert 0.8 < need < 1.0, need


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""
