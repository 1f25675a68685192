"""CPU checks of bench.py's contract that need no GPU: more than one GPU is refused with a
message before anything touches a device, and the HBM traffic of the dominant kernel is
reported only from a PMC summary measured on the kernel sources in the tree (the summary
carries their sha256; any other sources give null and the reason)."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_traffic_only_from_the_sources_it_was_measured_on(monkeypatch):
    import bench
    with open(os.path.join(ROOT, "profiles", "traffic_gemv_cfg2_down.json")) as f:
        rec = json.load(f)
    # the summary's own figures: HBM bytes per launch between the algorithmic bytes and 1.2x
    # (every weight byte fetched once, plus the activations and a few lines of slack)
    alg = rec.get("algorithmic_bytes_per_launch", 14159138)
    assert alg <= rec["hbm_bytes_per_launch"] <= 1.2 * alg
    assert len(rec["kernel_source_sha256"]) == 64
    value, why = bench.measured_traffic()
    if rec["kernel_source_sha256"] == bench.kernel_source_hash():
        assert value == rec["hbm_bytes_per_launch"] and "matches" in why
    else:
        assert value is None and "differs" in why
    # other sources: no figure, and the reason
    monkeypatch.setattr(bench, "kernel_source_hash", lambda: "0" * 64)
    value, why = bench.measured_traffic()
    assert value is None and "differs" in why


def test_traffic_hash_covers_the_kernel_sources():
    """Every header the measured kernel's translation units include, directly or through
    other headers, is hashed (found here by a scan of its own, not bench's)."""
    import bench
    import re
    for rel in bench.TRAFFIC_SOURCES:
        assert os.path.exists(os.path.join(ROOT, rel)), rel
    csrc = os.path.join(ROOT, "spectra_amd", "csrc")
    todo, found = ["gemv_rows_plain.hip", "gemv.hip"], set()
    while todo:
        name = todo.pop()
        if name in found:
            continue
        found.add(name)
        path = os.path.join(csrc, name)
        with open(path if os.path.exists(path) else os.path.join(ROOT, "include", name)) as f:
            todo += re.findall(r'#include "([^"]+)"', f.read())
    hashed = {os.path.basename(rel) for rel in bench.TRAFFIC_SOURCES}
    assert found <= hashed, found - hashed
    assert {"gemv_rows.h", "gemv_stream.h", "gemv_kernel.h", "common.h"} <= hashed
    assert bench.kernel_source_hash() == bench.kernel_source_hash()
