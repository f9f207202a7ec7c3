"""CPU checks of bench.py's contract and of the tools that write profiles/.

* `--gpus` other than 1 is refused with exit status 2 before any GPU work;
* the trace summary keeps only the timed steps and recomputes the dominant
  family's roofline fraction from the kernels' mean durations;
* roofline.traffic comes from profiles/hbm_traffic_config<N>.txt only when
  that summary was taken at the current kernel sources;
* every committed profile that names a source digest names the current one.
"""
import csv
import glob
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def _trace_csv(path, warmup, steps, durations):
    """A kernel trace of warmup + steps steps, each launching the config-3
    kernels in order with the given durations (ns); warm-up steps run 3x
    slower, so a summary that kept them would show it."""
    rows = []
    ts = 1_000_000
    did = 1
    for step in range(warmup + steps):
        for name, ns in durations:
            d = ns * (3 if step < warmup else 1)
            rows.append({"Kernel_Name": name, "Dispatch_Id": did, "Start_Timestamp": ts,
                         "End_Timestamp": ts + d})
            ts += d + 1000
            did += 1
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Dispatch_Id", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        w.writerows(rows)


def test_trace_summary_timed_steps_and_family_fraction(tmp_path):
    durations = [(k, 1000 * (i + 1)) for i, k in enumerate(
        ["k_check_detectors_lds", "k_transpose_idx", "k_fill_tm_dma", "k_fill_commit",
         "k_transpose_keys4", "k_propagate_units", "k_propagate_scatter",
         "k_wgrad_commit_values", "k_bucket_samples", "k_wgrad_slices"])]
    path = tmp_path / "run_kernel_trace.csv"
    _trace_csv(path, 2, 3, durations)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--trace-summary", str(path),
                        "--config", "3", "--warmup", "2", "--steps", "3"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    out = r.stdout
    # the last kernel's mean is its timed duration, not the warm-up's
    m = re.search(r"^k_wgrad_slices\s+1\.00\s+(\S+)", out, re.M)
    assert m and float(m.group(1)) == pytest.approx(0.010)
    fam = {"gather_w_gradients_fc": (8 + 9 + 10) * 1e-3}
    m = re.search(r"^gather_w_gradients_fc\s+(\S+) ms", out, re.M)
    assert m and float(m.group(1)) == pytest.approx(fam["gather_w_gradients_fc"])
    ub = bench.family_unique_bytes(3)["gather_w_gradients_fc"]
    frac = ub / (fam["gather_w_gradients_fc"] * 1e-3) / 1e9 / bench.PEAK_HBM_GBS
    m = re.search(r"dominant family gather_w_gradients_fc: .* = (\S+) of", out)
    assert m and float(m.group(1)) == pytest.approx(frac, rel=1e-3)


def test_traffic_only_at_current_sources(tmp_path, monkeypatch):
    (tmp_path / "profiles").mkdir()
    f = tmp_path / "profiles" / "hbm_traffic_config3.txt"
    digest = bench.source_digest()
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    monkeypatch.setattr(bench, "source_digest", lambda: digest)
    f.write_text(f"# HBM bytes\n# sources {digest}\ngather_w_gradients_fc 8869223949\n")
    t = bench.traffic_fields("gather_w_gradients_fc", 3, 1.5)
    assert t["traffic"] == 8869223949 and not t["traffic_stale"]
    assert t["traffic_gbs"] == pytest.approx(8869223949 / 1.5e-3 / 1e9, abs=0.1)
    f.write_text("# HBM bytes\n# sources 0000000000000000\ngather_w_gradients_fc 8869223949\n")
    t = bench.traffic_fields("gather_w_gradients_fc", 3, 1.5)
    assert t["traffic"] is None and t["traffic_stale"]


def test_committed_profiles_name_the_current_sources():
    digest = bench.source_digest()
    found = 0
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.txt"))):
        with open(path) as fh:
            for line in fh:
                m = re.search(r"(?:source digest(?: of the kernels profiled)?:|# sources) ([0-9a-f]{16})", line)
                if m:
                    found += 1
                    assert m.group(1) == digest, f"{os.path.basename(path)} was taken at {m.group(1)}"
    assert found >= 10
