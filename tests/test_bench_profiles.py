"""The counter summaries behind bench.py's roofline.traffic (profiles/
*_traffic_*.md) were measured on the current kernel sources: each records the
SHA-256 of the sources it was measured on, and bench.py reports the figure
only while they match (CPU only; no GPU work)."""
import glob
import os
import re

import pytest

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SUMMARIES = sorted(glob.glob(os.path.join(ROOT, "profiles", "*_traffic_*.md")))


def test_every_bench_line_has_a_summary():
    names = {os.path.basename(p) for p in SUMMARIES}
    for key in ("cfg1", "cfg2", "cfg3", "cfg4", "cfg5", "cfg4_separate"):
        assert f"decode_traffic_{key}.md" in names
    assert "prefill_traffic_cfg5.md" in names


@pytest.mark.parametrize("path", SUMMARIES, ids=[os.path.basename(p) for p in SUMMARIES])
def test_traffic_summary_matches_kernel_sources(path):
    name = os.path.basename(path)
    kind, key = re.match(r"(decode|prefill)_traffic_(.+)\.md$", name).groups()
    text = open(path).read()
    recorded = re.search(r"kernel_sources_sha256:\s*([0-9a-f]+)", text)
    assert recorded, f"{name} records no kernel_sources_sha256"
    assert recorded.group(1) == bench.kernel_fingerprint(kind), (
        f"{name} was measured on other {kind} kernel sources: measure its FETCH_SIZE / WRITE_SIZE "
        f"again (the commands it lists) and record `python3 bench.py --kernel-fingerprint {kind}`")
    assert bench.profile_traffic(key, kind) > 0


def test_a_changed_source_nulls_the_figure(monkeypatch):
    """A summary whose fingerprint differs from the sources gives no figure."""
    monkeypatch.setattr(bench, "kernel_fingerprint", lambda kind: "0" * 16)
    assert bench.profile_traffic("cfg4") is None
    assert bench.profile_traffic("cfg5", "prefill") is None
