"""CPU tests of the rocprofv3 summariser behind profiles/ (profsum.py): the
byte-counter calibration, the dispatch-order table and the FP32 MFMA counter
arithmetic, on small synthetic CSVs in rocprofv3's column layout whose
expected figures are worked out by hand here."""
import csv
import os

import pytest

import profsum

CC_COLS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
           "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
           "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
KT_COLS = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id", "Kernel_Id", "Kernel_Name",
           "Correlation_Id", "Start_Timestamp", "End_Timestamp"]
GEMM = "void ppdl::(anonymous namespace)::k_gemm_dma<64, 64, 2, false, 2, 2>(ppdl::GemmArgs, int, int)"
COPY = "__amd_rocclr_copyBuffer"


def _write(path, cols, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=cols)
        w.writeheader()
        for r in rows:
            w.writerow({c: r.get(c, 0) for c in cols})


def _counters(directory, name, records):
    """records: (dispatch, kernel, counter, [values per instance])"""
    os.makedirs(directory, exist_ok=True)
    rows = []
    for d, k, c, vals in records:
        for v in vals:
            rows.append({"Dispatch_Id": d, "Kernel_Name": k, "Counter_Name": c, "Counter_Value": v})
    _write(os.path.join(directory, name + "_counter_collection.csv"), CC_COLS, rows)


def test_short_names():
    assert profsum.short(GEMM) == "k_gemm_dma<64, 64, 2, false, 2, 2>"
    assert profsum.short(COPY) == COPY


def test_traffic_calibrated_by_the_copy(tmp_path):
    # the 1 MiB copy reads and writes 1 MiB; its FETCH_SIZE reads 512 KiB
    # (factor 2) and its WRITE_SIZE 1024 KiB (factor 1)
    f, w = str(tmp_path / "f"), str(tmp_path / "w")
    _counters(f, "a", [(1, COPY, "FETCH_SIZE", [512.0]), (2, GEMM, "FETCH_SIZE", [100.0, 50.0]),
                       (3, GEMM, "FETCH_SIZE", [200.0])])
    _counters(w, "a", [(1, COPY, "WRITE_SIZE", [1024.0]), (2, GEMM, "WRITE_SIZE", [10.0]),
                       (3, GEMM, "WRITE_SIZE", [30.0])])
    t = profsum.traffic(f, w, 1)
    assert t["calibration"]["FETCH_SIZE_factor"] == 2.0 and t["calibration"]["WRITE_SIZE_factor"] == 1.0
    k = t["kernels"]["k_gemm_dma<64, 64, 2, false, 2, 2>"]
    # instances of a dispatch add up: (150 + 200) / 2 KiB x 2, (10 + 30) / 2 KiB x 1
    assert k["dispatches"] == 2
    assert k["fetch_bytes"] == 175 * 1024 * 2
    assert k["write_bytes"] == 20 * 1024
    assert k["bytes"] == k["fetch_bytes"] + k["write_bytes"]


def test_traffic_needs_the_calibration_copy(tmp_path):
    f = str(tmp_path / "f")
    _counters(f, "a", [(2, GEMM, "FETCH_SIZE", [1.0])])
    with pytest.raises(SystemExit):
        profsum.traffic(f, f, 1)


def test_dispatch_order_table(tmp_path):
    f, w = str(tmp_path / "f"), str(tmp_path / "w")
    _counters(f, "a", [(1, COPY, "FETCH_SIZE", [1024.0]), (7, GEMM, "FETCH_SIZE", [2048.0]),
                       (5, GEMM, "FETCH_SIZE", [1024.0])])
    _counters(w, "a", [(1, COPY, "WRITE_SIZE", [1024.0]), (7, GEMM, "WRITE_SIZE", [0.0]),
                       (5, GEMM, "WRITE_SIZE", [512.0])])
    rows = profsum.dispatches(f, w, 1, 5).splitlines()[2:]
    # library dispatches only, ascending id; 1 MiB copy -> factor 1 on both
    assert len(rows) == 2
    assert rows[0].split("|")[3].strip() == "%.2f" % (1024 * 1024 / 1e6)
    assert rows[0].split("|")[4].strip() == "%.2f" % (512 * 1024 / 1e6)
    assert rows[1].split("|")[3].strip() == "%.2f" % (2048 * 1024 / 1e6)


def test_mfma_counter_arithmetic(tmp_path):
    d = str(tmp_path / "m")
    # one dispatch of 2 GFLOP: MOPS = 2e9 / 512; busy = (2e9 / 4096) MFMAs x 64
    # cycles over 1024 SIMDs; GRBM_GUI_ACTIVE summed over 8 XCDs = 8 x 100000
    mops = 2e9 / 512
    busy = 2e9 / 4096 * 64
    _counters(d, "n", [(4, GEMM, "SQ_INSTS_VALU_MFMA_MOPS_F32", [mops]), (4, GEMM, "SQ_INSTS_VALU_MFMA_XF32", [0.0]),
                       (4, GEMM, "SQ_VALU_MFMA_BUSY_CYCLES", [busy]), (4, GEMM, "GRBM_GUI_ACTIVE", [800000.0])])
    _write(os.path.join(d, "n_kernel_trace.csv"), KT_COLS,
           [{"Kind": "KERNEL_DISPATCH", "Dispatch_Id": 4, "Kernel_Name": GEMM, "Start_Timestamp": 1000,
             "End_Timestamp": 1000 + 40000}])
    _write(os.path.join(d, "n_agent_info.csv"), ["Name", "Simd_Count", "Num_Xcc"],
           [{"Name": "gfx950", "Simd_Count": 1024, "Num_Xcc": 8}])
    row = profsum.mfma(d).splitlines()[2].split("|")
    assert row[1].strip() == "`k_gemm_dma<64, 64, 2, false, 2, 2>`"
    assert float(row[3]) == pytest.approx(2.0, abs=1e-4)          # GFLOP per dispatch
    assert int(row[4]) == 0                                        # XF32 MFMA instructions
    # busy / (1024 SIMDs x 100000 cycles per XCD) = 31.25 M / 102.4 M
    assert float(row[5]) == pytest.approx(100.0 * busy / (1024 * 100000.0), abs=0.05)
    assert float(row[6]) == pytest.approx(40.0, abs=0.01)          # us per dispatch
    assert float(row[7]) == pytest.approx(50.0, abs=0.1)           # 2 GFLOP / 40 us
