"""bench.py's roofline.traffic figure: read from the committed counter
profile only while the kernel generator it was measured on is unchanged."""
from __future__ import annotations

import bench


def test_traffic_reported_for_the_measured_generator():
    assert bench.measured_traffic() == 201516282


def test_traffic_is_null_once_the_generator_changes(tmp_path, monkeypatch):
    edited = tmp_path / "k_fused.cpp"
    edited.write_bytes(open(bench.TRAFFIC_SOURCE, "rb").read() + b"// edit\n")
    monkeypatch.setattr(bench, "TRAFFIC_SOURCE", str(edited))
    assert bench.measured_traffic() is None


def test_traffic_is_null_without_a_hash(tmp_path, monkeypatch):
    prof = tmp_path / "p.md"
    prof.write_text("traffic_bytes_per_launch: 123\n")
    monkeypatch.setattr(bench, "TRAFFIC_PROFILE", str(prof))
    assert bench.measured_traffic() is None
