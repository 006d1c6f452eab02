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


def test_traffic_records_name_the_shipping_kernel(tmp_path):
    # A record counts only when its kernel line names the kernel this build launches.
    (tmp_path / "profiles").mkdir()
    good = tmp_path / "profiles" / "decode_stream_kernel_c2_traffic.md"
    good.write_text(f"kernel: {bench.DOMINANT_KERNEL['c2']}\ntraffic_bytes_per_launch: 123\n")
    assert bench.measured_traffic("c2", root=str(tmp_path)) == 123
    good.write_text("kernel: decode_stream_kernel<128, false, false>\ntraffic_bytes_per_launch: 123\n")
    assert bench.measured_traffic("c2", root=str(tmp_path)) is None  # an older template: stale
    assert bench.measured_traffic("c5", root=str(tmp_path)) is None  # no record: null, not a guess
    # A step the library routed to the partitioned kernel did not run the recorded kernel.
    good.write_text(f"kernel: {bench.DOMINANT_KERNEL['c2']}\ntraffic_bytes_per_launch: 123\n")
    assert bench.measured_traffic("c2", partition=2048, root=str(tmp_path)) is None
    assert bench.measured_traffic("c2g2", root=str(tmp_path)) is None
    for workload in ("c2", "c3", "c4", "c5"):
        value = bench.measured_traffic(workload)
        kernel = bench.DOMINANT_KERNEL[workload]
        path = os.path.join(ROOT, "profiles", f"{kernel.split('<')[0]}_{workload}_traffic.md")
        if value is not None:
            assert value == recorded(os.path.basename(path))


def test_traffic_records_match_their_counters():
    # FETCH_SIZE (KiB, reported at half the bytes read) x 2 + WRITE_SIZE (KiB) x 1, for the
    # kernel the record names.
    for name in sorted(os.listdir(os.path.join(ROOT, "profiles"))):
        if not name.endswith("_traffic.md"):
            continue
        with open(os.path.join(ROOT, "profiles", name)) as fh:
            text = fh.read()
        kernel = re.search(r"^kernel: (.*)$", text, re.M)
        if kernel is None:
            continue
        row = re.search(r"^\| " + re.escape(kernel.group(1)) + r" \| (\d+) \| (\d+) \|$", text, re.M)
        fetch, write = int(row.group(1)), int(row.group(2))
        assert recorded(name) == (2 * fetch + write) * 1024, name


def test_host_cpu_description():
    text = bench.host_cpu()
    assert "logical CPUs" in text and "affinity mask" in text and str(os.cpu_count()) in text


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                          text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr


def test_repaged_tables_hold_the_same_tokens():
    # bench.py --page-size: a block table re-paged to smaller pages names the
    # same slot for every token of every row, and nothing past a row's length.
    import numpy as np

    from gaudirt_amd import workloads

    rng = np.random.default_rng(0)
    lens = np.array([1, 127, 128, 129, 300, 4096])
    table = workloads.permuted_block_tables(rng, lens, 128, 64)
    for page in (128, 64, 16, 4, 2, 1):
        paged = workloads.repage_tables(table, lens, 128, page)
        for row, n in enumerate(lens):
            tokens = np.arange(n)
            want = table[row, tokens // 128] * 128 + tokens % 128
            assert np.array_equal(paged[row, tokens // page] * page + tokens % page, want), (page, row)
            assert (paged[row, (n + page - 1) // page:] == -1).all(), (page, row)
