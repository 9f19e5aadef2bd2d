"""bench.py's host-side paths, on the CPU: the one-GPU guard and the rocprofv3 summaries (kernel trace, counter and
HBM-traffic tables) over small synthetic CSV files in rocprofv3's column layout."""
import csv
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BENCH = os.path.join(HERE, "..", "bench.py")


def run(*args):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True, timeout=120)


def write_csv(path, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def table_rows(out):
    return [[c.strip() for c in l.strip().strip("|").split("|")] for l in out.splitlines()
            if l.startswith("| ") and not l.startswith("| kernel")]


def test_more_than_one_gpu_is_refused():
    r = run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_trace_summary(tmp_path):
    name = "void mkv::(anonymous namespace)::decode_combine<9, false>(float const*, int)"
    rows = [{"Kernel_Name": name, "Grid_Size_X": "16384", "Workgroup_Size_X": "256", "Start_Timestamp": str(s),
             "End_Timestamp": str(s + d)} for s, d in ((1000, 4000), (9000, 5000), (20000, 3000))]
    rows.append({"Kernel_Name": "void mkv::(anonymous namespace)::decode_f16<false>(_Float16 const*)",
                 "Grid_Size_X": "55296", "Workgroup_Size_X": "512", "Start_Timestamp": "100",
                 "End_Timestamp": "24600"})
    # a name the trace left mangled (decode_f16<true>), and a torch kernel, which is left out
    rows.append({"Kernel_Name": "_ZN3mkv12_GLOBAL__N_110decode_f16ILb1EEEvPDF16_S2_mPKfiiifiiPfS4_S4_S4_iiii", "Grid_Size_X": "33792",
                 "Workgroup_Size_X": "512", "Start_Timestamp": "0", "End_Timestamp": "6500"})
    rows.append({"Kernel_Name": "void at::native::vectorized_elementwise_kernel<4>(int)", "Grid_Size_X": "64",
                 "Workgroup_Size_X": "64", "Start_Timestamp": "0", "End_Timestamp": "90000"})
    f = tmp_path / "run_kernel_trace.csv"
    write_csv(str(f), rows)
    r = run("--trace-summary", str(f))
    assert r.returncode == 0, r.stderr
    t = table_rows(r.stdout)
    assert len(t) == 3
    # ordered by total time: the decode (24.5 us) before the three merges (12 us in all)
    assert t[0][:4] == ["mkv::decode_f16<false>", "55296", "512", "1"] and t[0][4] == "24.50"
    assert t[1][:4] == ["mkv::decode_combine<9, false>", "16384", "256", "3"]
    assert t[1][4:] == ["4.00", "4.00", "3.00", "5.00"]  # mean, median, min, max
    assert t[2][:5] == ["mkv::decode_f16<true>", "33792", "512", "1", "6.50"]


def pmc_dir(root, counter, values):
    """values: {(kernel, grid): [per-dispatch values]}"""
    rows = [{"Kernel_Name": k, "Grid_Size": str(g), "Counter_Name": counter, "Counter_Value": str(v)}
            for (k, g), vs in values.items() for v in vs]
    write_csv(os.path.join(root, "host", "run_counter_collection.csv"), rows)
    return root


def test_pmc_summary_scales_by_the_copy_kernel(tmp_path):
    copy = ("void at::native::vectorized_elementwise_kernel<4>(int)", 16777216)
    dec = ("void mkv::(anonymous namespace)::decode_f16<false>(_Float16 const*)", 110592)
    flint = ("void mkv::flint::(anonymous namespace)::fl_dec16<0, 2>(void const*)", 49152)
    # the copy reads and writes 256 MiB: FETCH_SIZE reads half of it (scale 2), WRITE_SIZE all of it (scale 1)
    f = pmc_dir(str(tmp_path / "f"), "FETCH_SIZE", {copy: [131072.0], dec: [66000.0, 66002.0], flint: [33665.0]})
    w = pmc_dir(str(tmp_path / "w"), "WRITE_SIZE", {copy: [262144.0], dec: [7160.0, 7160.0], flint: [816.0]})
    r = run("--pmc-summary", f, w)
    assert r.returncode == 0, r.stderr
    assert "scale 2.000" in r.stdout and "scale 1.000" in r.stdout
    t = {row[0]: row for row in table_rows(r.stdout)}
    assert set(t) == {"decode_f16<false>", "fl_dec16<0, 2>"}
    d = t["decode_f16<false>"]
    assert d[1:3] == ["110592", "2"]
    read_mb = 66001.0 * 1024 * 2 / 1e6
    assert float(d[5]) == pytest.approx(read_mb, abs=0.01)
    assert float(d[6]) == pytest.approx(7160.0 * 1024 / 1e6, abs=0.01)


def test_counter_summary(tmp_path):
    dec = ("void mkv::(anonymous namespace)::decode_f16<false>(_Float16 const*)", 110592)
    rows = [{"Kernel_Name": dec[0], "Grid_Size": str(dec[1]), "Counter_Name": c, "Counter_Value": str(v)}
            for c, vs in (("SQ_INSTS_MFMA", [206976, 206976]), ("GRBM_GUI_ACTIVE", [600000, 700000])) for v in vs]
    rows.append({"Kernel_Name": "void at::native::other(int)", "Grid_Size": "64", "Counter_Name": "SQ_INSTS_MFMA",
                 "Counter_Value": "1"})
    write_csv(str(tmp_path / "c" / "host" / "run_counter_collection.csv"), rows)
    r = run("--counter-summary", str(tmp_path / "c"))
    assert r.returncode == 0, r.stderr
    lines = [l for l in r.stdout.splitlines() if l.startswith("| ")]
    assert lines[0] == "| kernel | grid | dispatches | GRBM_GUI_ACTIVE | SQ_INSTS_MFMA |"
    t = table_rows(r.stdout)
    assert len(t) == 1 and t[0][1:] == ["110592", "2", "650000", "206976"]
