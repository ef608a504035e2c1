"""Host logic of bench.py, on the CPU: the decode traffic figure is reported only for the kernel
sources it was measured on."""
from __future__ import annotations

import bench


def test_traffic_reported_only_for_the_measured_kernel_sources(tmp_path, monkeypatch):
    profile = tmp_path / "traffic.md"
    monkeypatch.setattr(bench, "TRAFFIC_PROFILE", profile)
    assert bench.measured_traffic()[0] is None  # no summary
    here = bench.decode_source_hash()
    assert len(here) == 16 and int(here, 16) >= 0
    profile.write_text(f"# counters\ntraffic_bytes_per_launch: 174519573\nkernel_source_sha16: {here}\n")
    value, note = bench.measured_traffic()
    assert value == 174519573 and here in note
    # a summary taken on other sources (a stale counter) is not reported
    profile.write_text("traffic_bytes_per_launch: 174519573\nkernel_source_sha16: 0123456789abcdef\n")
    value, note = bench.measured_traffic()
    assert value is None and "not reported" in note
    profile.write_text("traffic_bytes_per_launch: 174519573\n")
    assert bench.measured_traffic()[0] is None


def test_source_hash_follows_the_kernel_sources(tmp_path, monkeypatch):
    a, b = tmp_path / "decode.hip", tmp_path / "common.h"
    a.write_text("kernel v1")
    b.write_text("helpers")
    monkeypatch.setattr(bench, "TRAFFIC_SOURCES", (a, b))
    h1 = bench.decode_source_hash()
    a.write_text("kernel v2")
    assert bench.decode_source_hash() != h1


def test_prefill_counters_reported_only_for_the_measured_kernel_sources(tmp_path, monkeypatch):
    profile = tmp_path / "prefill.md"
    monkeypatch.setattr(bench, "PREFILL_PROFILE", profile)
    assert bench.prefill_counters()[0] is None  # no summary
    here = bench.prefill_source_hash()
    profile.write_text(f"# counters\nkernel_source_sha16: {here}\nvalu_per_tile_wave: 392.7\nmfma_busy_fraction: 0.33\n")
    value, note = bench.prefill_counters()
    assert value == {"valu_per_tile_wave": 392.7, "mfma_busy_fraction": 0.33} and here in note
    profile.write_text("kernel_source_sha16: 0123456789abcdef\nvalu_per_tile_wave: 392.7\n")
    value, note = bench.prefill_counters()
    assert value is None and "not reported" in note


def test_committed_counter_summaries_match_the_committed_sources():
    """The committed summaries were taken on the committed kernel sources (so the bench line reports
    both figures): a kernel change without new counters shows up here, not as a silent stale figure."""
    assert bench.measured_traffic()[0] is not None, bench.measured_traffic()[1]
    assert bench.prefill_counters()[0] is not None, bench.prefill_counters()[1]
