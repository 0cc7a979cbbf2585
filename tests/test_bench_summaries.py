"""bench.py's rocprofv3 summaries on synthetic counter files: the derived
figures follow the counters' units (SQ_WAVE_CYCLES, SQ_BUSY_CU_CYCLES,
SQ_WAIT_ANY and SQ_ACTIVE_INST_VALU in quad-cycles; GRBM_GUI_ACTIVE summed
over 8 XCCs) and the traffic scale comes from the copy calibration."""
import csv
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

K = "void anelm::rmsnorm_row_kernel<2, 1, false, false, true>(void*, float*, float const*, void const*, long, int, long, long, long, float)"
OTHER = "void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<float> >(int, at::native::FillFunctor<float>)"
FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def _write(d, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "r_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, FIELDS)
        w.writeheader()
        for i, (k, c, v) in enumerate(rows):
            w.writerow(dict(Dispatch_Id=i, Kernel_Name=k, Counter_Name=c, Counter_Value=v))


def test_sq_summary_units(tmp_path):
    raw = dict(SQ_WAVES=1000, SQ_WAVE_CYCLES=250_000, SQ_BUSY_CU_CYCLES=10_000, SQ_WAIT_ANY=125_000,
               SQ_WAIT_INST_ANY=25_000, SQ_INSTS_VALU=300_000, SQ_ACTIVE_INST_VALU=40_960, SQ_INSTS_SALU=80_000,
               SQ_INSTS_VMEM_RD=4000, SQ_INSTS_VMEM_WR=2000, SQ_INSTS_LDS=9000, SQ_WAIT_INST_LDS=0,
               SQ_ACTIVE_INST_ANY=1, GRBM_GUI_ACTIVE=8 * 40_000, MeanOccupancyPerActiveCU=24.5, VmemLatency=812.0)
    dirs = []
    for i, counters in enumerate(bench.SQ_PASSES):
        d = str(tmp_path / f"p{i}")
        # two dispatches of the kernel (the mean is taken) and one of another kernel (ignored)
        rows = [(K, c, raw[c] * s) for c in counters for s in (0.5, 1.5)] + [(OTHER, c, 1e9) for c in counters]
        _write(d, rows)
        dirs.append(d)
    text = bench.sq_summary(dirs, workload="qwen3-8b-prefill")
    got = json.loads(text.split("sq_json: ")[1])["per_dispatch"]["rmsnorm"]
    assert got["waves"] == 1000
    assert got["waves_per_cu"] == 0.1                       # 4 * 250000 / (40000 cycles * 256 CUs)
    assert got["occ_rocprof"] == 24.5
    assert got["kernel_cycles"] == 40_000                   # GRBM_GUI_ACTIVE / 8 XCCs
    assert got["wave_cycles"] == 1000                       # 4 * 250000 / 1000
    assert got["wait"] == 0.5 and got["issue_wait"] == 0.1
    assert got["vmem_lat"] == 812
    assert got["valu_util"] == 0.004                        # 4 * 40960 / (1024 * 40000)
    assert got["vmem_rd_per_wave"] == 4.0 and got["vmem_wr_per_wave"] == 2.0
    assert list(json.loads(text.split("sq_json: ")[1])["per_dispatch"]) == ["rmsnorm"]   # the other kernel matches no op


def test_pmc_summary_scales_by_copy_calibration(tmp_path):
    d = {n: str(tmp_path / n) for n in ("f", "w", "cf", "cw")}
    _write(d["f"], [(K, "FETCH_SIZE", 1024.0)])
    _write(d["w"], [(K, "WRITE_SIZE", 2048.0)])
    # the copy of 1 GiB reads back as half its bytes in FETCH_SIZE and all of them in WRITE_SIZE
    _write(d["cf"], [("__amd_rocclr_copyBuffer", "FETCH_SIZE", (1 << 30) / 1024 / 2)])
    _write(d["cw"], [("__amd_rocclr_copyBuffer", "WRITE_SIZE", (1 << 30) / 1024)])
    text = bench.pmc_summary(d["f"], d["w"], d["cf"], d["cw"], workload="qwen3-8b-prefill")
    row = next(l for l in text.splitlines() if l.startswith("| rmsnorm |"))
    traffic = int(row.split("|")[6])
    assert traffic == 2 * 1024 * 1024 + 2048 * 1024
