"""bench.py's host-side profile summaries (no GPU): per-(kernel, grid) rows from a
rocprofv3 kernel trace, and per-(kernel, grid) counter means from --pmc collections."""
import csv

import bench


def _write(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_kernel_trace_summary_splits_kernels_by_grid(tmp_path):
    path = tmp_path / "kt_kernel_trace.csv"
    name = "void mi355x::(anonymous namespace)::prefill_kernel<0, 4, true, 8>(mi355x::(anonymous namespace)::PrefillArgs)"
    rows = [[name, 0, 400_000, 352256, 1, 1], [name, 0, 420_000, 352256, 1, 1],
            [name, 0, 30_000, 69632, 1, 1]]
    _write(path, ["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X",
                  "Grid_Size_Y", "Grid_Size_Z"], rows)
    lines = bench.summarize_kernel_trace(str(path)).splitlines()
    assert lines[1].split()[:4] == ["prefill_kernel<0,", "4,", "true,", "8>"]
    big = [ln for ln in lines if " 352256 " in ln][0].split()
    small = [ln for ln in lines if " 69632 " in ln][0].split()
    assert big[5] == "2" and float(big[6]) == 410.0      # calls, avg_us
    assert small[5] == "1" and float(small[6]) == 30.0


def test_counter_summary_means_per_kernel_and_grid(tmp_path):
    paths = []
    for i, counter in enumerate(("FETCH_SIZE", "WRITE_SIZE")):
        p = tmp_path / f"p{i}.csv"
        _write(p, ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"],
               [[1, "void mi355x::(anonymous namespace)::linear_kernel<0>(x)", 98304, counter, 10],
                [2, "void mi355x::(anonymous namespace)::linear_kernel<0>(x)", 98304, counter, 30],
                [3, "silu_mul_vec<0>(x)", 4096, counter, 7]])
        paths.append(str(p))
    text = bench.summarize_counters(paths, "linear")
    assert "linear_kernel<0>  grid 98304  dispatches 2" in text
    assert "silu" not in text
    assert [ln.split()[-1] for ln in text.splitlines()[1:]] == ["20.0", "20.0"]


def test_gap_summary_splits_stretches_at_host_pauses(tmp_path):
    path = tmp_path / "kt.csv"
    rows, t = [], 0
    for gap_ns in (1000, 500):  # two serving runs: 1 us and 0.5 us between kernels
        for i in range(1200):
            rows.append(["decode_mma_kernel<0>" if i % 10 == 0 else "other", t, t + 5000])
            t += 5000 + gap_ns
        t += 10 ** 9  # a one-second host pause
    _write(path, ["Kernel_Name", "Start_Timestamp", "End_Timestamp"], rows)
    lines = bench.summarize_gaps(str(path)).splitlines()
    first, second = lines[1].split(), lines[2].split()
    assert first[1] == second[1] == "1200" and first[2] == "120"
    assert float(first[6]) == 1.0 and float(second[6]) == 0.5
    # Idle time by the kernel it follows: in the first run 120 gaps of 1 us follow the
    # decode kernel and 1079 follow the others.
    i = lines.index("# stretch 0: idle time by the kernel it follows (top 8)")
    table = {ln.split()[0]: ln.split() for ln in lines[i + 2:i + 4]}
    assert table["other"][3] == "1079" and table["decode_mma_kernel<0>"][3] == "120"
    assert float(table["decode_mma_kernel<0>"][1]) == 0.12
