"""The diagnostics build: host statistics (CPU) and one run per workload (GPU).

The GPU test runs the diagnostics module in a child process (it routes the
package through libgabor_hip_diag.so for the rest of its process) and checks
the backward's lane histogram against the forward's replay lists: a wave
processes a record exactly when its quadrant bit is set in the record's
replay entry, so the histogram's total must equal the number of set bits.
"""

import json
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from diff_gabor_splatting_amd import diagnostics

ROOT = Path(__file__).resolve().parents[1]


def test_log2_histogram_bins():
    values = torch.tensor([0.0, 0.5, 1.0, 1.9, 2.0, 3.9, 4.0, 1000.0])
    assert diagnostics.log2_histogram(values) == {"0": 2, "1": 2, "2": 2, "4": 1, "512": 1}


def test_launch_profile_of_known_stamps():
    # Four tiles at 1000 kHz (one tick = 1 us): two run together from 0, a
    # third starts when the first ends, a long one runs alone at the end.
    span = torch.tensor([[0, 10], [0, 4], [4, 12], [12, 40]])
    profile = diagnostics.launch_profile(span, 1000)
    assert profile["span_us"] == 40
    assert profile["peak_tiles_in_flight"] == 2
    # Fewer than one tile in flight never happens inside the span; below
    # half the peak (1) means zero tiles: none here.
    assert profile["tail_us_below_half_peak"] == 0
    assert profile["longest_tile_us"] == 28 and profile["longest_tile_began_us"] == 12
    assert profile["tile_us_sum"] == 10 + 4 + 8 + 28
    assert profile["tile_us"]["p100"] == 28


def test_launch_profile_tail_counts_time_below_half_the_peak():
    # Four tiles together for 10 us, then one alone for 30 us.
    span = torch.tensor([[0, 10], [0, 10], [0, 10], [0, 40]])
    profile = diagnostics.launch_profile(span, 1000)
    assert profile["peak_tiles_in_flight"] == 4
    assert profile["tail_us_below_half_peak"] == 30
    assert profile["ended_90pct_us"] == 10  # index int(0.9 * 3) = 2 of [10, 10, 10, 40]


def test_lane_summary():
    hist = [0] * 65
    hist[1], hist[8], hist[40], hist[64] = 3, 1, 2, 4
    summary = diagnostics.lane_summary(hist)
    assert summary["record_wave_pairs"] == 10
    assert summary["mean_taking_lanes"] == pytest.approx((3 + 8 + 80 + 256) / 10)
    assert summary["share_at_most_8"] == pytest.approx(0.4)
    assert summary["share_all_64"] == pytest.approx(0.4)


def test_replay_quadrant_bits_counts_each_tiles_entries():
    # Two tiles: the first's list starts at 0 with 2 entries, the second's at
    # 5 with 1 entry; entries past a tile's count are ignored.
    ranges = torch.tensor([[0, 4], [5, 9]], dtype=torch.int32)
    counts = torch.tensor([2, 1], dtype=torch.int32)
    lists = torch.zeros((9, 2), dtype=torch.int32)
    lists[0, 1] = (0b0001 << 28) | 3
    lists[1, 1] = (0b0110 << 28) | 1
    lists[2, 1] = (0b0111 << 28) | 2  # beyond the first tile's count
    lists[5, 1] = int(-(1 << 31)) | (0b111 << 28)  # all four quadrant bits
    assert diagnostics.replay_quadrant_bits(lists, counts, ranges) == 1 + 2 + 4


def test_product_library_refuses_diagnostics():
    from diff_gabor_splatting_amd import _native

    status = _native.lib.gs_diagnostics_set(None, None, None, 0, None)
    assert status == 1 and b"without diagnostics" in _native.lib.gs_last_error()


def test_walk_summary_counts():
    hist = [0] * 65
    hist[2], hist[64] = 3, 1
    lanes = diagnostics.lane_summary(hist)
    walk = diagnostics.walk_summary(1000, 640, lanes)
    assert walk == {"forward_pixel_record_visits": 1000, "forward_samples_evaluated": 640,
                    "backward_samples_evaluated": 256, "backward_samples_taken": 70}


def test_packing_summary_ratios():
    summary = diagnostics.packing_summary([0, 0, 200, 180, 150, 195, 198, 0])
    assert summary["wave_steps"] == 200 and summary["ratio_halves_at_best"] == 0.9
    assert summary["ratio_blocks_in_order"] == 0.99
    assert diagnostics.packing_summary([0] * 8)["ratio_halves_at_best"] is None


def test_collect_restores_the_product_library(monkeypatch):
    """collect() renders through the diagnostics library and switches the
    package back to the library it used before, also when the run fails."""
    from diff_gabor_splatting_amd import _native

    if not diagnostics.DIAGNOSTICS_LIBRARY.exists():
        pytest.skip("the diagnostics library is not built")
    before = _native.library_path()
    seen = []

    def failing_run(name, device):
        seen.append(_native.library_path())
        raise RuntimeError("planted failure")

    monkeypatch.setattr(diagnostics, "_collect", failing_run)
    with pytest.raises(RuntimeError, match="planted failure"):
        diagnostics.collect("config0", torch.device("cpu"))
    assert seen == [diagnostics.DIAGNOSTICS_LIBRARY]
    assert _native.library_path() == before
    assert _native.lib.gs_diagnostics_set(None, None, None, 0, None) == 1


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
@pytest.mark.parametrize("workload", ["harness-classic", "config1"])
def test_diagnostics_run_matches_the_replay_lists(tmp_path, workload):
    output = tmp_path / "report.json"
    print(f"diagnostics child: {workload}", flush=True)
    done = subprocess.run(
        [sys.executable, "-m", "diff_gabor_splatting_amd.diagnostics", "--workload", workload,
         "--json", str(output)],
        cwd=ROOT, capture_output=True, text=True, timeout=240,
    )
    assert done.returncode == 0, done.stdout[-2000:] + done.stderr[-4000:]
    report = json.loads(output.read_text())[workload]
    lanes = report["backward_taking_lanes"]
    assert lanes["histogram"][0] == 0
    assert lanes["record_wave_pairs"] == report["replay_quadrant_bits"] > 0
    assert 1 <= lanes["mean_taking_lanes"] <= 64
    walk = report["forward_walk"]
    assert walk["backward_samples_taken"] <= walk["backward_samples_evaluated"]
    packing = report["backward_packing"]
    assert packing["wave_steps"] == lanes["record_wave_pairs"]
    for kind in ("halves", "blocks"):
        # Packing can only save steps, and never more than the at-best bound.
        assert (packing[f"{kind}_at_best"] <= packing[f"{kind}_in_order"]
                <= packing["wave_steps"])
    assert packing["blocks_at_best"] <= packing["halves_at_best"]
    # Every in-image pixel visits at least the records it took; the lockstep
    # walk evaluates at least one sample per visit that passed the footprint
    # tests, and the tiles' lists bound the visits.
    assert 0 < walk["forward_pixel_record_visits"] <= 256 * report["intersections"]
    assert walk["forward_samples_evaluated"] > 0
    for kernel in ("render_forward", "render_backward"):
        profile = report[kernel]
        assert 0 < profile["ended_90pct_us"] <= profile["ended_99pct_us"] <= profile["span_us"]
        assert 0 < profile["longest_tile_us"] <= profile["span_us"]
        assert sum(profile["tile_us_log2_histogram"].values()) == report["tiles"]
