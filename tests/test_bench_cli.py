"""The benchmark's own contract on the CPU: one GPU only, a sequence-length override for the
operator workloads only (and a batch override), kernel labels of profiler names, and the HBM-traffic record built from
counter runs (scaled by a plain copy of known size)."""
from __future__ import annotations

import csv
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stdout + r.stderr


def test_sequence_length_only_for_operator_workloads():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--workload", "ce_qwen3b_l32768",
                        "--seqlen", "1024"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "operator workloads only" in r.stderr
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--workload", "prefill_qwen3b_l32768",
                        "--batch", "2"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 2 and "operator workloads only" in r.stderr


@pytest.mark.parametrize("name,label", [
    ("_ZN5dsalt10fwd_kernelIDF16bLi64ELi32ELi2ELb0EEEvNS_10AttnParamsE", "attn_fwd"),
    ("_ZN5dsalt13bwd_dq_kernelIDF16bLi64ELi32ELb0EEEvNS_10AttnParamsE", "bwd_dq"),
    ("_ZN5dsalt15bwd_dkdv_kernelIDF16bLi64ELb0ELb0EEEvNS_10AttnParamsE", "bwd_dkdv"),
    ("_ZN5dsalt14bwd_lmk_kernelIDF16bLi64ELi8EEEvNS_10AttnParamsE", "bwd_lmk"),
    ("_ZN5dsalt18bwd_lmk_sum_kernelIDF16bLi64EEEvNS_10AttnParamsE", "bwd_lmk_sum"),
    ("dsalt::row_plan_kernel(dsalt::AttnParams)", "row_plan"),
    ("dsalt::sel_part_kernel(dsalt::SelectParams, float const*)", "sel_part"),
    # library kernels whose names contain a label inside a longer identifier keep their name
    ("void at::native::reduce_kernel<512, 1>(float)", "void at::native::reduce_kernel<512, 1>(float)"),
    ("void at::native::vectorized_gather_kernel<16>(char*)", "void at::native::vectorized_gather_kernel<16>(char*)"),
])
def test_profiler_names_map_to_labels(name, label):
    assert bench.short_kernel_name(name) == label


def _pmc(d, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for i, (k, c, v) in enumerate(rows):
            w.writerow({"Dispatch_Id": i, "Kernel_Name": k, "Counter_Name": c, "Counter_Value": v})


def test_traffic_record_scales_by_the_copy(tmp_path, monkeypatch):
    dq = "_ZN5dsalt13bwd_dq_kernelIDF16bLi64ELi32ELb0EEEvNS_10AttnParamsE"
    cp = "void at::native::vectorized_elementwise_kernel<4>(neg)"
    out = tmp_path / "prof"
    # a 1 MiB copy reads FETCH_SIZE 512 KiB (factor 2) and writes WRITE_SIZE 1024 KiB (factor 1)
    _pmc(out / "copy_fetch", [(cp, "FETCH_SIZE", 512.0)])
    _pmc(out / "copy_write", [(cp, "WRITE_SIZE", 1024.0)])
    # two dispatches of dQ: their mean counts
    _pmc(out / "fetch", [(dq, "FETCH_SIZE", 100.0), (dq, "FETCH_SIZE", 300.0)])
    _pmc(out / "write", [(dq, "WRITE_SIZE", 50.0), (dq, "WRITE_SIZE", 50.0)])
    (tmp_path / "profiles").mkdir()
    monkeypatch.setattr(bench, "HERE", str(tmp_path))  # the record goes to tmp_path/profiles
    monkeypatch.setattr(bench, "kernel_source_sha", lambda: "unit")
    rec = bench.traffic_from(str(out), "unit_workload", copy_mib=1)
    assert rec["bwd_dq"]["fetch_bytes"] == 200 * 1024 * 2
    assert rec["bwd_dq"]["write_bytes"] == 50 * 1024
    assert rec["bwd_dq"]["bytes"] == 200 * 1024 * 2 + 50 * 1024
    assert rec["_calibration"]["fetch_factor"] == pytest.approx(2.0)
    assert any("--traffic-from" in c for c in rec["_commands"])
    with open(tmp_path / "profiles" / "traffic_unit_workload.json") as f:
        assert json.load(f)["bwd_dq"] == rec["bwd_dq"]
    assert not any("--variant" in c for c in rec["_commands"])
    # a counted run with a fixed tiling names it in the bench commands and the rewrite
    rec = bench.traffic_from(str(out), "unit_workload", copy_mib=1, variant="3")
    assert [c.endswith("--variant 3") for c in rec["_commands"]] == [True, True, False, False, True]
