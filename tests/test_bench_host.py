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
