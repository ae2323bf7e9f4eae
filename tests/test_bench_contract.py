"""CPU checks of bench.py's contract: it refuses more than one GPU before
touching one, its headline buffer sets are a multiple of its stream count and
span more than twice the MALL, and the HBM-traffic figures it reports are
the ones the committed profiles hold (so the JSON line and profiles/ cannot
drift apart)."""
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"),
                        "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "single MI355X" in r.stderr
    assert r.stdout == ""


def test_headline_buffer_sets():
    n = bench.ntt_sets()
    assert n % bench.NTT_STREAMS == 0
    # each role (source, destination) rotates over more than twice the MALL
    assert n * 2 * 32 * bench.LIMB_BYTES > 2 * bench.MALL_BYTES


def _table_row(name, kernel):
    """(FETCH_SIZE KiB, WRITE_SIZE KiB, HBM bytes) of a profile table row"""
    with open(os.path.join(ROOT, "profiles", name)) as f:
        for line in f:
            if line.startswith("| `%s`" % kernel):
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                return float(cells[2]), float(cells[3]), int(cells[6])
    raise AssertionError("%s: no row for %s" % (name, kernel))


def test_bconv_traffic_matches_profile():
    fetch, write, total = _table_row("bconv_config3_traffic.md",
                                     "bconv_mfma<1, true, false>")
    assert bench.BCONV_TRAFFIC == total
    assert abs(total - (fetch * 2 + write) * 1024) < 1024


def test_hmult_traffic_matches_profile():
    """the bench's figure is the sum of the profile's eight per-launch rows
    (| # | kernel | ... | HBM bytes |), each consistent with its counters"""
    rows = []
    with open(os.path.join(ROOT, "profiles", "hmult_config4_traffic.md")) as f:
        for line in f:
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) == 8 and cells[0].isdigit():
                rows.append(cells)
    assert [int(c[0]) for c in rows] == list(range(1, 9))
    for c in rows:
        fetch, write, total = float(c[3]), float(c[4]), int(c[7])
        assert abs(total - (fetch * 2 + write) * 1024) < 1024
    assert bench.HMULT_TRAFFIC == sum(int(c[7]) for c in rows)


def test_ntt_traffic_from_profile():
    _, _, total = _table_row("ntt_fwd_config2_traffic.md",
                             "ntt_fwd_1p<0, false>")
    assert bench.traffic_from_profile() == total


def test_hmult_launch_count_matches_trace():
    """the eight launches the traffic sum counts are the kernel trace's"""
    with open(os.path.join(ROOT, "profiles",
                           "hmult_config4_kernel_trace.md")) as f:
        text = f.read().split("## Cold")[0]
    calls = {m.group(1): int(m.group(2)) for m in
             re.finditer(r"\| `([^`]+)` \| (\d+) \|", text)}
    steps = calls["modup_keyacc"]
    assert sum(calls.values()) == 8 * steps
