"""bench.py's profile helpers on synthetic rocprofv3 csv files (no GPU): the tables under
profiles/ and the roofline's traffic figure are computed by these functions."""
import csv
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _write(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)
    return str(path)


def test_trace_table_last_dispatches_only(bench, tmp_path):
    # 5 slow warm-up launches (clocks ramping) then 3 timed ones of 2 us: with last=3 only
    # the timed ones count
    rows = [(i * 100, i * 100 + 50_000, "k") for i in range(5)]
    rows += [(10_000_000 + i * 10_000, 10_000_000 + i * 10_000 + 2_000, "k") for i in range(3)]
    rows += [(20_000_000, 20_004_000, "other")]
    p = _write(tmp_path / "t.csv", ["Start_Timestamp", "End_Timestamp", "Kernel_Name"], rows)
    out = bench.trace_table(p, last=3)
    line = next(l for l in out.splitlines() if l.startswith("| `k`"))
    cells = [c.strip() for c in line.strip("|").split("|")]
    assert cells[1] == "3.0" and cells[2] == "2.00"
    assert "the last 3 of each kernel" in out


def test_trace_table_per_step_windows(bench, tmp_path):
    # three steps delimited by "ce_row" (once per step); the first window is skipped
    rows = []
    t = 0
    for step in range(4):
        for name, dur in (("ce_row", 10), ("gemm", 30), ("gemm", 50), ("norm", 5)):
            rows.append((name, t, t + dur))
            t += dur + 1          # a 1 ns gap after every kernel
    p = _write(tmp_path / "kt.csv", ["Kernel_Name", "Start_Timestamp", "End_Timestamp"], rows)
    out = bench.trace_table(p, "ce_row", skip=1)
    # windows 1 and 2 (between the 2nd/3rd and 3rd/4th ce_row): 95 ns of kernels, 99 ns span
    assert out.startswith("2 steps")
    assert "0.1 µs of kernels per step in a span of 0.1 µs, 4 dispatches per step" in out
    gemm = next(l for l in out.splitlines() if l.startswith("| `gemm`"))
    cells = [c.strip() for c in gemm.strip("|").split("|")]
    assert cells[1] == "2.0"                      # calls per step
    assert float(cells[2]) == pytest.approx(0.04)  # avg (30 + 50) / 2 ns in µs
    assert float(cells[6]) == pytest.approx(100 * 80 / 95, abs=0.1)


def test_trace_table_needs_enough_windows(bench, tmp_path):
    p = _write(tmp_path / "kt.csv", ["Kernel_Name", "Start_Timestamp", "End_Timestamp"],
               [("ce_row", 0, 1), ("x", 2, 3), ("ce_row", 4, 5)])
    with pytest.raises(SystemExit):
        bench.trace_table(p, "ce_row", skip=2)


def _pmc_rows(counter, entries):
    """entries: (dispatch id, kernel name, value) -> counter_collection rows (2 XCD rows each)."""
    rows = []
    for d, k, v in entries:
        for half in (0.25, 0.75):
            rows.append((d, k, counter, v * half, 0, 1000))
    return rows


PMC_HDR = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def test_pmc_summary_scales_by_the_copy(bench, tmp_path):
    # the copy of 1 GiB reads FETCH_SIZE = half its bytes and WRITE_SIZE = all of them (KiB)
    gib_kib = (1 << 30) / 1024
    cf = _write(tmp_path / "cf.csv", PMC_HDR, _pmc_rows("FETCH_SIZE", [(1, "copy_kernel", gib_kib / 2)]))
    cw = _write(tmp_path / "cw.csv", PMC_HDR, _pmc_rows("WRITE_SIZE", [(1, "copy_kernel", gib_kib)]))
    f = _write(tmp_path / "f.csv", PMC_HDR, _pmc_rows("FETCH_SIZE", [
        (1, "attn_bwd_dq_kernel<64>", 100.0), (2, "attn_bwd_dkv_kernel<64>", 300.0),
        (3, "attn_bwd_dq_kernel<64>", 140.0), (4, "attn_bwd_dkv_kernel<64>", 300.0)]))
    w = _write(tmp_path / "w.csv", PMC_HDR, _pmc_rows("WRITE_SIZE", [
        (1, "attn_bwd_dq_kernel<64>", 10.0), (2, "attn_bwd_dkv_kernel<64>", 20.0)]))
    res = bench.pmc_summary(f, w, cf, cw)
    assert res["scale_fetch"] == pytest.approx(2.0)
    assert res["scale_write"] == pytest.approx(1.0)
    dq = res["kernels"]["attn_bwd_dq_kernel"]
    assert dq["fetch_kib"] == pytest.approx(120.0) and dq["dispatches"] == [2, 1]
    expect = (120.0 * 2 + 10.0 + 300.0 * 2 + 20.0) * 1024
    assert res["traffic_bytes_per_launch"] == pytest.approx(expect)


def test_pmc_summary_wgrad_kernel_set(bench, tmp_path):
    # fx_linear_wgrad's launch: one whole-tile kernel and one reduce dispatch; the general
    # kernel (gemm_wgrad_kernel) is not part of it
    gib_kib = (1 << 30) / 1024
    cf = _write(tmp_path / "cf.csv", PMC_HDR, _pmc_rows("FETCH_SIZE", [(1, "copy_kernel", gib_kib / 2)]))
    cw = _write(tmp_path / "cw.csv", PMC_HDR, _pmc_rows("WRITE_SIZE", [(1, "copy_kernel", gib_kib)]))
    f = _write(tmp_path / "f.csv", PMC_HDR, _pmc_rows("FETCH_SIZE", [
        (1, "void fx::gemm_wgrad_fast_kernel<3>(fx::WgradArgs)", 1000.0),
        (2, "fx::wgrad_reduce_kernel(float const*, int, long, int)", 500.0),
        (3, "fx::gemm_wgrad_kernel(fx::WgradArgs)", 9999.0)]))
    w = _write(tmp_path / "w.csv", PMC_HDR, _pmc_rows("WRITE_SIZE", [
        (1, "void fx::gemm_wgrad_fast_kernel<3>(fx::WgradArgs)", 400.0),
        (2, "fx::wgrad_reduce_kernel(float const*, int, long, int)", 40.0)]))
    res = bench.pmc_summary(f, w, cf, cw, kernels=bench._WGRAD_TRAFFIC_KERNELS)
    assert set(res["kernels"]) == {"gemm_wgrad_fast_kernel", "wgrad_reduce_kernel"}
    assert res["traffic_bytes_per_launch"] == pytest.approx((1000.0 * 2 + 400.0 + 500.0 * 2 + 40.0) * 1024)


def test_wgrad_roofline_weighs_the_four_shapes_equally(bench):
    wg = {"a": {"shape_TMN": [10, 2, 3], "us": 1.0}, "b": {"shape_TMN": [10, 4, 5], "us": 3.0}}
    flop, us = bench.wgrad_roofline(wg)
    assert flop == pytest.approx((120.0 + 400.0) / 2) and us == pytest.approx(2.0)


def test_counter_table_mfma_busy(bench, tmp_path):
    # one dispatch: GRBM_GUI_ACTIVE summed over 8 XCDs = 8000 -> 1000 cycles per XCD;
    # MFMA busy 512,000 SIMD-cycles over 1024 SIMDs x 1000 cycles = 50 %
    rows = [(1, "k", "GRBM_GUI_ACTIVE", 8000.0, 0, 2000), (1, "k", "SQ_VALU_MFMA_BUSY_CYCLES", 512000.0, 0, 2000),
            (1, "k", "SQ_INSTS_VALU_MFMA_MOPS_BF16", 1000.0, 0, 2000)]
    p = _write(tmp_path / "c.csv", PMC_HDR, rows)
    out = bench.counter_table([p])
    line = next(l for l in out.splitlines() if l.startswith("| `k`"))
    cells = [c.strip() for c in line.strip("|").split("|")]
    assert cells[-2] == "50.0"
    # 1000 x 512 flops in 2000 ns = 256 GFLOP/s = 0.256 TFLOP/s
    assert cells[-1] == "0.3"


def test_counter_table_pipeline_ratios(bench, tmp_path):
    # GRBM_GUI_ACTIVE 8000 over 8 XCDs: 1000 cycles, so 256,000 CU cycles and 1,024,000 SIMD
    # cycles; TA busy 128,000 CU cycles = 50 %; 64,000 wave quad-cycles waiting = 25 % of the
    # SIMD cycles; 3000 cycles of latency over 10 L2 reads = 300
    rows = [(1, "k", "GRBM_GUI_ACTIVE", 8000.0, 0, 2000), (1, "k", "TA_TA_BUSY", 128000.0, 0, 2000),
            (1, "k", "SQ_WAIT_INST_ANY", 64000.0, 0, 2000), (1, "k", "TCP_TCC_READ_REQ_LATENCY", 3000.0, 0, 2000),
            (1, "k", "TCP_TCC_READ_REQ", 10.0, 0, 2000)]
    p = _write(tmp_path / "c.csv", PMC_HDR, rows)
    out = bench.counter_table([p])
    hdr = [c.strip() for c in out.splitlines()[0].strip("|").split("|")]
    line = next(l for l in out.splitlines() if l.startswith("| `k`"))
    cells = dict(zip(hdr, [c.strip() for c in line.strip("|").split("|")]))
    assert cells["TA_TA_BUSY % of CU cycles"] == "50.0"
    assert cells["SQ_WAIT_INST_ANY % of SIMD cycles"] == "25.0"
    assert cells["L2 read latency (cycles)"] == "300"
