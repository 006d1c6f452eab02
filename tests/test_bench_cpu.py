"""bench.py's host-side pieces (no GPU): traffic records, host description, one-GPU guard."""

import os
import re
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def recorded(name):
    with open(os.path.join(ROOT, "profiles", name)) as fh:
        return int(re.search(r"^traffic_bytes_per_launch: (\d+)$", fh.read(), re.M).group(1))


def test_traffic_records_are_read_from_profiles():
    assert bench.measured_traffic("decode_stream", "c2") == recorded("decode_stream_c2_traffic.md")
    assert bench.measured_traffic("prefill", "c4") == recorded("prefill_c4_traffic.md")
    assert bench.measured_traffic("decode_stream", "c5") is None  # no record: null, not a guess


def test_traffic_records_match_their_counters():
    # FETCH_SIZE (KiB, reported at half the bytes read) x 2 + WRITE_SIZE (KiB) x 1.
    for name, kernel in [("decode_stream_c2_traffic.md", "decode_stream_kernel"),
                         ("prefill_c4_traffic.md", "prefill_kernel")]:
        with open(os.path.join(ROOT, "profiles", name)) as fh:
            text = fh.read()
        row = re.search(r"^\| " + kernel + r"<[^|]*> \| (\d+) \| (\d+) \|$", text, re.M)
        fetch, write = int(row.group(1)), int(row.group(2))
        assert recorded(name) == (2 * fetch + write) * 1024


def test_host_cpu_description():
    text = bench.host_cpu()
    assert "logical CPUs visible" in text and str(os.cpu_count()) in text


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                          text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr
