"""bench.py's traffic bookkeeping on the CPU: the counter summary and the
source-digest check that keeps a figure measured on other kernel sources out
of the bench line."""

import csv
import importlib.util
import json
import os

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test",
                                                  os.path.join(REPO, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _write_counters(folder, rows):
    os.makedirs(folder, exist_ok=True)
    with open(os.path.join(folder, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name",
                                          "Counter_Value"])
        w.writeheader()
        for i, (k, c, v) in enumerate(rows):
            w.writerow({"Dispatch_Id": i, "Kernel_Name": k, "Counter_Name": c,
                        "Counter_Value": v})


def test_traffic_summary_and_digest(bench, tmp_path, monkeypatch):
    gate = "void cmk::iq2xxs_gemv_kernel<0, true, true, 1, false, false, 0>(cmk::GemvArgs)"
    down = "void cmk::iq2xxs_gemv_kernel<0, true, true, 2, false, false, 0>(cmk::GemvArgs)"
    copy = "__amd_rocclr_copyBuffer"
    # the copy reads 256 MiB: FETCH_SIZE shows half of it, WRITE_SIZE all of it
    _write_counters(tmp_path / "copy_FETCH_SIZE", [(copy, "FETCH_SIZE", 131072.0)] * 3)
    _write_counters(tmp_path / "copy_WRITE_SIZE", [(copy, "WRITE_SIZE", 262144.0)] * 3)
    _write_counters(tmp_path / "gemv_FETCH_SIZE",
                    [(gate, "FETCH_SIZE", 7000.0), (gate, "FETCH_SIZE", 7000.0),
                     (down, "FETCH_SIZE", 7600.0), ("other", "FETCH_SIZE", 1e6)])
    _write_counters(tmp_path / "gemv_WRITE_SIZE",
                    [(gate, "WRITE_SIZE", 56.0), (gate, "WRITE_SIZE", 56.0),
                     (down, "WRITE_SIZE", 16.0)])
    out = tmp_path / "traffic.json"
    bench.traffic_summary(str(tmp_path), str(out))
    t = json.load(open(out))
    assert t["fetch_size_factor"] == 2.0 and t["write_size_factor"] == 1.0
    assert t["fetch_bytes_per_launch"] == round(7200.0 * 1024 * 2)  # (7000+7000+7600)/3
    assert t["write_bytes_per_launch"] == round(128.0 / 3 * 1024)
    assert t["hbm_bytes_per_launch"] == t["fetch_bytes_per_launch"] + t["write_bytes_per_launch"]
    assert sorted(t["kernels"]) == sorted([gate, down])
    assert t["source_digest"] == bench.gemv_source_digest()

    # reported while the digest matches, null once the sources differ
    monkeypatch.setattr(bench, "TRAFFIC_FILE", str(out))
    value, note = bench.load_traffic()
    assert value == t["hbm_bytes_per_launch"] and "measured on these" in note
    t["source_digest"] = "0" * 16
    json.dump(t, open(out, "w"))
    value, note = bench.load_traffic()
    assert value is None and "not reported" in note


def test_committed_traffic_file_names_the_benched_kernel(bench):
    t = json.load(open(bench.TRAFFIC_FILE))
    assert "source_digest" in t and len(t["source_digest"]) == 16
    assert all("iq2xxs_gemv_kernel<0, true, true," in k for k in t["kernels"])
