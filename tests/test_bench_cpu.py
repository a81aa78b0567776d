"""bench.py's bookkeeping that needs no GPU: kernel classes of the profile
summaries, the step breakdown and the fabric-side byte count of a step."""
import csv
import os

import pytest

import bench as B


@pytest.mark.parametrize("name,cls", [
    ("Cijk_Ailk_Bljk_BBS_BH_Bias_HAS_SAV_UserArgs_MT256x256x64", "torch"),
    ("void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<float> >(int)", "torch"),
    ("void cvmm::topk_gemm_kernel<bf16, bf16, true>(cvmm::TopkGemmParams)", "dense_topk"),
    ("cvmm::topk_slot_table_kernel(int const*, int const*, long const*)", "dense_prep"),
    ("void cvmm::scale_rows_kernel<bf16, unsigned int>(void const*, int)", "dense_prep"),
    ("void cvmm::sort_scatter_cast_kernel<int, bf16>(cvmm::ScatterArgs<int>)", "sort"),
    ("void cvmm::copy_ids_count_kernel<long>(long const*, long)", "sort"),
    ("void cvmm::combine_rows_wave_kernel<bf16>(int)", "combine"),
    ("void cvmm::routed_small_kernel<4>(cvmm::GemmParams)", "gemm"),
    ("void cvmm::route_topk_hist_kernel<float, 16, 8>(float const*)", "router"),
])
def test_kernel_classes(name, cls):
    assert B.kernel_class(name) == cls


def test_breakdown_sums_to_the_phases():
    phases = {"prepare": 0.002, "fwd": 0.05, "bwd": 0.1}
    kt = {"sort": {"ms_per_step": 0.012, "avg_ms": 0.006, "launches_per_step": 2}}
    b = B.breakdown(phases, kt)
    assert b["sel"] == 0.012
    assert abs(sum(b.values()) - sum(phases.values())) < 1e-12
    assert B.breakdown(phases, {})["sel"] == 0.0


def _write_csv(path, header, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_step_fabric_bytes(tmp_path):
    """Per-dispatch FETCH + WRITE (KiB, copy-calibrated) times the trace's
    dispatches, over the steps the traced run made."""
    d = tmp_path / "wl"
    _write_csv(str(d / "trace" / "x" / "run_kernel_stats.csv"),
               ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"],
               [["kA", 10, 1000, 100, 50, 1, 1, 0], ["kB", 20, 900, 45, 45, 1, 1, 0],
                ["kC", 10, 100, 10, 5, 1, 1, 0]])
    (d / "trace.log").write_text("noise\nsteps run: 10\n")
    cc = ["Kernel_Name", "Counter_Name", "Counter_Value"]
    _write_csv(str(d / "fetch" / "x" / "run_counter_collection.csv"), cc,
               [["kA", "FETCH_SIZE", 100], ["kA", "FETCH_SIZE", 300], ["kB", "FETCH_SIZE", 10]])
    _write_csv(str(d / "write" / "x" / "run_counter_collection.csv"), cc,
               [["kA", "WRITE_SIZE", 50], ["kB", "WRITE_SIZE", 30]])
    cp = tmp_path / "copy"
    kib = B.COPY_BYTES / 1024
    _write_csv(str(cp / "FETCH_SIZE" / "x" / "run_counter_collection.csv"), cc, [["copy", "FETCH_SIZE", kib / 2]])
    _write_csv(str(cp / "WRITE_SIZE" / "x" / "run_counter_collection.csv"), cc, [["copy", "WRITE_SIZE", kib]])
    f = B.step_fabric(str(d), str(cp))
    # fetch factor 2, write factor 1; kA: (200 * 2 + 50) KiB x 10 calls, kB: (10 * 2 + 30) KiB x 20 calls
    assert f["fabric_bytes_per_step"] == int(((200 * 2 + 50) * 10 + (10 * 2 + 30) * 20) * 1024 / 10)
    assert f["steps_traced"] == 10
    assert f["covered"] == pytest.approx(1900 / 2000)


def test_committed_traffic_records_are_records():
    """Every profiles/traffic_*.json that bench.py reads holds bytes per launch
    (a class whose kernels the counters could not attribute gets no file)."""
    import glob
    import json
    files = glob.glob(os.path.join(B.ROOT, "profiles", "traffic_*.json"))
    assert files
    for f in files:
        with open(f) as fh:
            d = json.load(fh)
        assert isinstance(d, dict), f
        key = "fabric_bytes_per_step" if os.path.basename(f).startswith("traffic_step_") else "bytes_per_launch"
        assert d.get(key, 0) > 0, f


def test_missing_or_empty_traffic_reads_as_none(tmp_path, monkeypatch):
    monkeypatch.setattr(B, "ROOT", str(tmp_path))
    os.makedirs(tmp_path / "profiles")
    assert B.load_traffic("gemm_fwd", "nothing") is None
    (tmp_path / "profiles" / "traffic_gemm_fwd_empty.json").write_text("null")
    assert B.load_traffic("gemm_fwd", "empty") is None
