"""Host-only checks of bench.py's rocprofv3 summarisers on synthetic traces:
which dispatches count as the timed ones, and where the training step starts."""
import csv
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

NS = "gdn2::(anonymous namespace)::"


def _trace(path, rows):
    """rows: (name, duration_us) in launch order, back to back."""
    t = 1_000_000
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for name, dur in rows:
            w.writerow({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + int(dur * 1000)})
            t += int(dur * 1000) + 500


def test_timed_summary_skips_warmups_and_takes_steps(tmp_path, capsys):
    import bench

    intra = f"void {NS}chunk_intra_kernel<128, 128, false>(gdn2::ChunkParams)"
    inter = f"void {NS}chunk_inter_kernel<128, 0, 4>(gdn2::ChunkParams, int)"
    dec = f"void {NS}decode_fused_kernel<128, 128>(gdn2::DecodeParams)"
    pre = "void (anonymous namespace)::stream_copy_kernel(HIP_vector_type<float, 4u>*, long)"
    post = "void (anonymous namespace)::tail_copy_kernel(float*, float const*, long)"
    rows = [(pre, 1.0)] + [(intra, 700.0), (inter, 700.0)] * 4 + [(post, 1.0)]  # settle loop, then its marker
    for i in range(2 + 3):  # 2 warm-ups (long), then 3 timed steps
        rows += [(intra, 900.0 if i < 2 else 500.0), (inter, 900.0 if i < 2 else 600.0)]
    rows += [(pre, 1.0)] + [(intra, 1.0), (inter, 1.0)] * 2 + [(post, 1.0)]  # the layer's settle loop
    rows += [(intra, 2.0), (inter, 2.0)] * 6  # the layer's own calls: another section, not counted
    rows += [(pre, 1.0)] + [(dec, 77.0)] * 5 + [(post, 1.0)]  # decode settle loop
    rows += [(dec, 99.0)] * 8 + [(dec, 28.0)] * 4 + [(dec, 99.0)]  # 8 warm-ups, 4 timed, 1 check
    p = tmp_path / "kt.csv"
    _trace(p, rows)
    bench.timed_summary(str(p), warmup=2, steps=3, decode_steps=4)
    out = capsys.readouterr().out
    assert "| 3 | 500.0 | 500.0 | 500.0 |" in out
    assert "| 3 | 600.0 | 600.0 | 600.0 |" in out
    assert "| 4 | 28.0 | 28.0 | 28.0 |" in out


def test_train_summary_starts_at_the_input_gemm(tmp_path, capsys):
    import bench

    gemm = "Cijk_Ailk_Bljk_S_B_MT128x256x32_MI16x16x1"
    rows = [(gemm, 9300.0)]                                   # previous step's dx GEMM
    rows += [(gemm, 9280.0), (gemm, 160.0), (gemm, 158.0)]   # x W_in, f_proj_1, g_proj_1
    rows += [(f"void {NS}project_kernel(gdn2::ProjectParams)", 870.0), (gemm, 9350.0)]
    p = tmp_path / "tt.csv"
    _trace(p, rows)
    bench.train_summary(str(p))
    out = capsys.readouterr().out
    lines = [l for l in out.splitlines() if l.startswith("| ") and "start us" not in l and "---" not in l]
    assert lines[0].startswith("| 0.0 | 9280.0 |"), lines[0]
    assert len(lines) == 5


def test_stats_summary_folds_gemm_kernels(tmp_path, capsys):
    import bench

    p = tmp_path / "stats.csv"
    with open(p, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage"])
        w.writeheader()
        w.writerow({"Name": f"void {NS}chunk_inter_kernel<128, 0, 4>(gdn2::ChunkParams, int)", "Calls": 2,
                    "TotalDurationNs": 1_200_000, "AverageNs": 600_000, "Percentage": 10.0})
        for i in range(3):
            w.writerow({"Name": f"Cijk_Alik_Bljk_S_B_MT{i}", "Calls": 1, "TotalDurationNs": 3_000_000,
                        "AverageNs": 3_000_000, "Percentage": 30.0})
    bench.stats_summary(str(p))
    out = capsys.readouterr().out
    assert "| `chunk_inter_kernel<128, 0, 4>` | 2 | 600.0 | 1200.0 | 10.0 |" in out
    assert "| hipBLASLt GEMM kernels (3 names) | 3 | 3000.0 | 9000.0 | 90.0 |" in out


@pytest.mark.parametrize("xs,med", [([7.0], 7.0), ([3.0, 1.0, 2.0], 2.0), ([4.0, 1.0, 3.0, 2.0], 2.5)])
def test_median(xs, med):
    import bench

    assert bench._median(xs) == med


def test_configs_summary_counts_the_first_settled_section_of_each_shape(tmp_path, capsys):
    import bench

    intra = f"void {NS}chunk_intra_kernel<128, 128, false>(gdn2::ChunkParams)"
    inter = f"void {NS}chunk_inter_kernel<128, 0, 4>(gdn2::ChunkParams, int)"
    pre = "void (anonymous namespace)::stream_copy_kernel(HIP_vector_type<float, 4u>*, long)"
    post = "void (anonymous namespace)::tail_copy_kernel(float*, float const*, long)"
    g = 512 * 64  # 64 chunks
    rows = [(pre, 1.0, 256)] + [(intra, 70.0, g), (inter, 70.0, 256)] * 3 + [(post, 1.0, 256)]
    rows += [(intra, 90.0, g), (inter, 90.0, 256)]  # one warm-up
    rows += [(intra, 15.0, g), (inter, 55.0, 256)] * 2  # two timed steps
    rows += [(pre, 1.0, 256), (post, 1.0, 256)] + [(intra, 5.0, g), (inter, 5.0, 256)] * 3  # the layer's calls
    p = tmp_path / "kt.csv"
    t = 1_000_000
    with open(p, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X"])
        w.writeheader()
        for name, dur, grid in rows:
            w.writerow({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + int(dur * 1000),
                        "Grid_Size_X": grid})
            t += int(dur * 1000) + 500
    bench.configs_summary(str(p), warmup=1, steps=2)
    out = capsys.readouterr().out
    assert "| `chunk_intra_kernel<128, 128, false>` x 64 | `chunk_intra_kernel<128, 128, false>` | 32768 | 2 | 15.0 |" in out
    assert "| `chunk_inter_kernel<128, 0, 4>` | 256 | 2 | 55.0 |" in out
