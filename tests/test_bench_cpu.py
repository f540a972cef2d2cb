"""CPU tests of bench.py's host-side contract: the committed HBM-traffic summary it reads the
roofline's `traffic` from is arithmetically consistent, the step-time spread helper, and the
one-GPU refusal of `--gpus N` (which exits before touching a GPU)."""
import json
import os
import re
import subprocess
import sys

import numpy as np

from tests.conftest import ROOT

sys.path.insert(0, ROOT)
import bench  # noqa: E402


def _traffic_summary():
    with open(os.path.join(ROOT, "profiles", "flash_c4_hbm_traffic.md")) as f:
        return f.read()


def test_traffic_line_matches_the_counter_table():
    """traffic_bytes_per_launch = (FETCH_SIZE x read factor + WRITE_SIZE x write factor) KiB
    for every kernel of the table, with the factors of the copy calibration stated above it."""
    text = _traffic_summary()
    m = re.search(r"read bytes = FETCH_SIZE x ([0-9.]+) KiB and write bytes = WRITE_SIZE x "
                  r"([0-9.]+) KiB", text)
    assert m, "calibration factors not stated"
    fr, fw = float(m.group(1)), float(m.group(2))
    line = next(l for l in text.splitlines() if l.startswith("traffic_bytes_per_launch:"))
    table = json.loads(line.split(":", 1)[1])
    rows = re.findall(r"^\| `([^`]+)` \| (\d+) \| (\d+) \|", text, re.M)
    assert {r[0] for r in rows} == set(table)
    for name, fetch, write in rows:
        want = (int(fetch) * fr + int(write) * fw) * 1024
        assert abs(table[name] - want) <= 1024, (name, table[name], want)


def test_profiled_traffic_reads_the_dominant_kernel():
    got = bench.profiled_traffic("flash_bwd_dkdv_kernel")
    text = _traffic_summary()
    line = next(l for l in text.splitlines() if l.startswith("traffic_bytes_per_launch:"))
    table = json.loads(line.split(":", 1)[1])
    want = [v for k, v in table.items() if k.startswith("flash_bwd_dkdv_kernel<")]
    assert got == want[0] and got > 0
    assert bench.profiled_traffic("no_such_kernel") is None


def test_spread_median_and_iqr():
    per = [3.0, 1.0, 2.0, 5.0, 4.0]
    s = bench.spread(per)
    assert s["median"] == 3.0
    q1, q3 = np.percentile(per, [25, 50, 75])[[0, 2]]
    assert s["iqr"] == [round(float(q1), 4), round(float(q3), 4)]


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
