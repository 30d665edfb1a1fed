"""bench.py's contract pieces that need no GPU: the one-GPU guard, the
counter-run arithmetic behind roofline.traffic, and the algorithmic bytes
the roofline prices."""

from __future__ import annotations

import csv
import subprocess
import sys

import pytest

from conftest import ROOT


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def _counter_csv(folder, counter, rows):
    folder.mkdir(parents=True)
    with open(folder / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for did, name, value in rows:
            # counters come split over the chip's blocks: two rows per dispatch
            w.writerow({"Dispatch_Id": did, "Kernel_Name": name, "Counter_Name": counter, "Counter_Value": value / 2})
            w.writerow({"Dispatch_Id": did, "Kernel_Name": name, "Counter_Name": counter, "Counter_Value": value / 2})


def test_traffic_scaling_from_counter_runs(tmp_path):
    import bench

    copy_bytes = bench.COPY_BYTES
    # FETCH_SIZE reads half the copy's bytes (scale 2); WRITE_SIZE all of them
    _counter_csv(tmp_path / "f", "FETCH_SIZE", [
        (1, "__amd_rocclr_copyBuffer", copy_bytes / 1024 / 2),
        (2, "void plh::k_sample_chunks<float, true>(plh::SampleArgs)", 1000.0),
        (3, "void plh::k_sample_chunks<float, true>(plh::SampleArgs)", 3000.0),
        (4, "void plh::k_sample_final<float, true>(plh::SampleArgs)", 99999.0),
    ])
    _counter_csv(tmp_path / "w", "WRITE_SIZE", [
        (1, "__amd_rocclr_copyBuffer", copy_bytes / 1024),
        (2, "void plh::k_sample_chunks<float, true>(plh::SampleArgs)", 10.0),
        (3, "void plh::k_sample_chunks<float, true>(plh::SampleArgs)", 30.0),
    ])
    out = bench.traffic_from("char65", str(tmp_path / "f"), str(tmp_path / "w"), dst=tmp_path / "t.json")
    cal = out["calibration"]
    assert cal["FETCH_SIZE"]["scale"] == pytest.approx(2.0) and cal["WRITE_SIZE"]["scale"] == pytest.approx(1.0)
    ch = out["per_kernel"]["k_sample_chunks"]["counters"]
    assert ch["FETCH_SIZE"]["kib_per_launch"] == pytest.approx(2000.0)
    assert ch["WRITE_SIZE"]["kib_per_launch"] == pytest.approx(20.0)
    chunks = 2000.0 * 1024 * 2 + 20.0 * 1024
    assert out["bytes_per_launch"] == pytest.approx(chunks)  # the headline kernel alone
    final = 99999.0 * 1024 * 2  # one launch in the probe's PROBE_STEPS steps
    # per step: each kernel's bytes per launch times its launches per step
    assert out["bytes_per_step"] == pytest.approx((2 * chunks + final) / bench.PROBE_STEPS)
    assert (tmp_path / "t.json").exists()


def test_instructions_per_token_from_counter_runs(tmp_path):
    """--valu-from: per row group, the k_sample_chunks counters averaged
    over its launches, times 64 lanes, over the tokens of one launch."""
    import bench

    B, V = 4, 1000
    dirs = []
    for g in range(2):
        folder = tmp_path / f"g{g}"
        folder.mkdir()
        with open(folder / "run_counter_collection.csv", "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
            w.writeheader()
            for did, scale in ((10, 1.0), (11, 3.0)):  # two launches: their mean is taken
                for c, v in (("SQ_INSTS_VALU", 500.0), ("SQ_INSTS_SALU", 100.0), ("SQ_INSTS_LDS", 10.0),
                             ("SQ_WAVES", 8.0)):
                    w.writerow({"Dispatch_Id": did, "Kernel_Name": "void plh::k_sample_chunks<float, true, false>()",
                                "Counter_Name": c, "Counter_Value": v * scale * (g + 1)})
            # another kernel's counters are ignored
            w.writerow({"Dispatch_Id": 12, "Kernel_Name": "void plh::k_sample_final<float, true, false>()",
                        "Counter_Name": "SQ_INSTS_VALU", "Counter_Value": 1e9})
        dirs.append(str(folder))
    out = bench.valu_from("mixed128k", dirs, dst=tmp_path / "v.json", shape=(B, V))
    g0, g1 = out["groups"]
    assert g0["launches"] == 2 and g0["rows"] == "greedy"
    assert g0["valu_per_token"] == pytest.approx(1000.0 * 64 / (B * V))
    assert g1["valu_per_token"] == pytest.approx(2000.0 * 64 / (B * V))
    assert g1["salu_per_token"] == pytest.approx(400.0 * 64 / (B * V))
    assert g0["lds_per_token"] == pytest.approx(20.0 * 64 / (B * V))
    assert (tmp_path / "v.json").exists()


def test_instructions_per_token_per_kernel(tmp_path):
    """--valu-kernels-from: every sampler kernel's counters averaged over
    its launches (template arguments dropped), per token of the batch;
    other kernels are left out."""
    import bench

    B, V = 2, 500
    with open(tmp_path / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for did, kern, v in ((1, "void plh::k_sample_chunks<float, true, true>(plh::SampleArgs)", 100.0),
                             (2, "void plh::k_nuc_window<float>(plh::SampleArgs)", 40.0),
                             (3, "void plh::k_sample_chunks<float, true, true>(plh::SampleArgs)", 300.0),
                             (4, "void at::native::elementwise_kernel<128, 4>(int)", 1e9)):
            for c in ("SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_WAVES"):
                w.writerow({"Dispatch_Id": did, "Kernel_Name": kern, "Counter_Name": c, "Counter_Value": v})
    out = bench.valu_kernels_from("zipf152k", str(tmp_path), dst=tmp_path / "k.json", shape=(B, V))
    ks = {k["kernel"]: k for k in out["kernels"]}
    assert set(ks) == {"k_sample_chunks", "k_nuc_window"}
    assert ks["k_sample_chunks"]["launches"] == 2
    assert ks["k_sample_chunks"]["valu_per_token"] == pytest.approx(200.0 * 64 / (B * V))
    assert ks["k_nuc_window"]["lds_per_token"] == pytest.approx(40.0 * 64 / (B * V))
    assert (tmp_path / "k.json").exists()


def test_chunk_timeline_from_stamps():
    """--phase-stamps: the chunk pass's timeline from its real-time stamps.
    Two CUs with two slots each run three workgroups a slot, back to back
    with a 20-count gap; the clock rate, the span, the lifetimes, the
    residency and the refill gap come out as constructed."""
    import numpy as np

    import bench

    B, C = 3, 4  # 12 chunks: 2 CUs x 2 slots x 3 in turn
    n = B * C
    ph = np.zeros((4096, 8), np.int64)
    rt = np.zeros((4096, 9), np.int64)
    hw = np.zeros((4096, 2), np.int64)
    life, gap = 100, 20
    for g in range(n):
        cu, slot, k = g % 2, (g // 2) % 2, g // 4
        t0 = k * (life + gap)
        rt[g, 0] = t0
        rt[g, 1:] = t0 + life - 5  # waves 0..6 end 5 counts early
        rt[g, 8] = t0 + life  # the last wave
        ph[g, 0], ph[g, 7] = 1000, 1000 + 22 * (life - 5)  # 2.2 GHz: 22 clocks a 10 ns count
        hw[g, 0] = cu << 8  # CU id bits 11:8 of HW_ID
        hw[g, 1] = 0
    t = bench.chunk_timeline(ph, rt, hw, B, C)
    assert t["cus"] == 2
    assert t["clock_ghz"] == pytest.approx(2.2)
    assert t["span_us"] == pytest.approx((2 * (life + gap) + life) * 0.01)
    assert t["workgroup_life_us_median"] == pytest.approx(life * 0.01)
    assert t["slot_refill_gap_us_median"] == pytest.approx(gap * 0.01)
    assert t["wave0_end_to_last_wave_end_us_median"] == pytest.approx(5 * 0.01)
    # 12 lives of 100 over 2 CUs x a span of 340
    assert t["resident_workgroups_per_cu_mean"] == pytest.approx(round(12 * life / (2 * 340), 2))


def test_algorithmic_bytes_of_the_headline_workload():
    """4V per row of fp32 logits, 4H per history id of a penalised row, 48
    per row of parameters, uniform, offset and id."""
    from pagellm_amd import workloads

    w = workloads.mixed128k()
    B, V = w["logits"].shape
    pen_ids = sum(len(c) for c, p in zip(w["contexts"], w["params"]) if p.repetition_penalty != 1.0)
    assert workloads.algorithmic_bytes(w) == 4 * B * V + 4 * pen_ids + 48 * B == 131_870_720


def test_cpu_baseline_reports_one_core_and_all_cores():
    """The CPU baseline child (no GPU) times the oracle on one pinned core and
    over a pool of single-core processes, and both agree on the ids."""
    import json
    import subprocess
    import sys

    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--cpu-baseline-child", "--workload", "char65",
                        "--cpu-rows", "16", "--cpu-reps", "1"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["cores"] == 1 and out["kind"] == "port" and out["value"] > 0
    assert out["all_cores"]["cores"] >= 1 and out["all_cores"]["value"] > 0
