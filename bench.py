"""Sampler benchmark: sampled rows/s and HBM GB/s on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload mixed128k]

A step is one batched sampling pass over one batch held in HBM (default
mixed128k: 256 rows x 128256 fp32 logits, mixed per-row parameters, see
pagellm_amd/workloads.py).  Three copies of the logits rotate across steps
(3 x 131 MB > the 256 MB Infinity Cache), so every step streams from HBM.
The K timed steps are bracketed by HIP events recorded on the stream the
kernels are launched on; `value` is rows/s over them.  A second pass of K
steps with the library's kernel timing on (HIP events around each of the
fast path's two launches, same stream) gives the average duration of the
streaming kernel, k_sample_chunks, which the roofline object prices:
algorithmic bytes per launch / that duration.  Rank 0 prints one JSON line.

The CPU baseline is the numpy oracle looping over rows like the reference
engine (llm_engine.py:238-254), one pinned core with BLAS threads pinned to
1, on a bounded sample of the same workload, in a child process that never
touches the GPU.

HBM traffic per launch (roofline.traffic) comes from two rocprofv3 counter
runs of `bench.py --pmc-probe` (FETCH_SIZE, then WRITE_SIZE), each scaled by
what the same counter reads for a device-to-device copy of known size in
the same process; `bench.py --traffic-from FETCH_DIR WRITE_DIR` turns the
two result folders into profiles/traffic_<workload>.json, which later runs
report.
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBPS = 8000.0
PEAK_FP32_MFMA_TFLOPS = 157.3
METRIC = "sampled rows/sec + HBM GB/s (% peak), batch 256 × vocab 128256 fp32"


_POOL_JOB = None  # (logits, params, uniforms, contexts) of the sample, shared with forked workers


def _pool_init(cores) -> None:
    import multiprocessing

    ident = multiprocessing.current_process()._identity
    os.sched_setaffinity(0, {cores[(ident[0] - 1) % len(cores)] if ident else cores[0]})


def _pool_rows(rows):
    import oracle

    x, params, u, ctx = _POOL_JOB
    return oracle.sample_batch(x[rows], [params[i] for i in rows], u[rows], [ctx[i] for i in rows])


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _parity_rows(w, rows, gpu_ids):
    """Oracle ids for the given rows against the GPU's, with the boundary
    gauges for every row: greedy rows must agree exactly; a sampled row may
    differ only if its uniform lies within 1e-6 of a CDF boundary or its
    top-p cut within 1e-12 of flipping (the 1e-6 boundary rule), and the
    kernels' fixed-point CDF keeps every mismatch within 1e-12 of one
    (``mismatches_outside_1e-12`` counts those that are not)."""
    import oracle
    from oracle.sampler import sample_boundary_gaps

    greedy = mism = explained = in_band = outside_tight = 0
    greedy_exact = True
    for r in rows:
        prm, x, ctx, u = w["params"][r], w["logits"][r], w["contexts"][r], w["uniforms"][r]
        ref = oracle.sample(x, prm, u, ctx)
        if prm.greedy:
            greedy += 1
            if int(gpu_ids[r]) != ref:
                greedy_exact = False
                mism += 1
            continue
        g_topp, g_draw = sample_boundary_gaps(x, prm, u, ctx)
        band = g_topp < 1e-12 or g_draw < 1e-6
        in_band += band
        if int(gpu_ids[r]) != ref:
            mism += 1
            explained += band
            outside_tight += not (g_topp < 1e-12 or g_draw < 1e-12)
    return {"rows": len(rows), "greedy_rows": greedy, "greedy_exact": greedy_exact, "mismatches": mism,
            "boundary_cases": explained, "rows_in_boundary_band": in_band,
            "unexplained_mismatches": mism - explained, "mismatches_outside_1e-12": outside_tight}


def _parity_verify(w, toks, nacc):
    import numpy as np

    import oracle
    from oracle.sampler import verify_boundary_gap

    rt, rn = oracle.verify_batch(w["p"], w["q"], w["draft"], w["accept_u"], w["resample_u"])
    mism = explained = in_band = outside_tight = 0
    for b in range(len(rn)):
        gap = verify_boundary_gap(w["p"][b], w["q"][b], [int(t) for t in w["draft"][b]], w["accept_u"][b],
                                  w["resample_u"][b])
        band = gap < 1e-6
        in_band += band
        if int(nacc[b]) != int(rn[b]) or not np.array_equal(toks[b], rt[b]):
            mism += 1
            explained += band
            outside_tight += not gap < 1e-12
    return {"rows": int(len(rn)), "accept_counts_exact": bool(np.array_equal(nacc, rn)), "mismatches": mism,
            "boundary_cases": explained, "rows_in_boundary_band": in_band, "unexplained_mismatches": mism - explained,
            "mismatches_outside_1e-12": outside_tight}


def cpu_baseline_child(workload: str, rows: int, reps: int, ids_path: str | None) -> None:
    """Runs in a fresh process that never touches the GPU, BLAS pinned to one
    thread: the oracle over the sample on one pinned core (the engine's
    single thread), then the same sample split row-wise over a pool of
    processes, one per allowed core (at most 16).  Untimed afterwards: the
    GPU ids of every configuration the parent measured (ids_path) against
    the oracle's on the same inputs and uniforms."""
    global _POOL_JOB
    cores = sorted(os.sched_getaffinity(0))
    os.sched_setaffinity(0, {cores[0]})
    import multiprocessing

    import numpy as np

    import oracle
    from pagellm_amd import workloads

    w = workloads.WORKLOADS[workload]()
    B = w["logits"].shape[0]
    sel = np.linspace(0, B - 1, min(rows, B)).astype(int)
    x = w["logits"][sel]
    params = [w["params"][i] for i in sel]
    u = w["uniforms"][sel]
    ctx = [w["contexts"][i] for i in sel]
    oracle.sample_batch(x[:2], params[:2], u[:2], ctx[:2])  # warm-up
    times = []
    ids1 = None
    for _ in range(reps):
        t0 = time.perf_counter()
        ids1 = oracle.sample_batch(x, params, u, ctx)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    # all allowed cores: rows dealt round-robin (every worker gets every
    # parameter group), forked workers share the sample copy-on-write
    n = min(len(cores), 16)
    _POOL_JOB = (x, params, u, ctx)
    parts = [np.arange(j, len(sel), n) for j in range(n)]
    ptimes = []
    with multiprocessing.get_context("fork").Pool(n, initializer=_pool_init, initargs=(cores,)) as pool:
        pool.map(_pool_rows, [p[:1] for p in parts])  # warm-up
        for _ in range(reps):
            t0 = time.perf_counter()
            res = pool.map(_pool_rows, parts)
            ptimes.append(time.perf_counter() - t0)
    ids_n = np.empty(len(sel), dtype=np.int64)
    for p, r in zip(parts, res):
        ids_n[p] = r
    if not np.array_equal(ids_n, np.asarray(ids1)):
        raise RuntimeError("the pooled CPU baseline disagrees with the one-core run")
    pmed = float(np.median(ptimes))
    parity = None
    if ids_path:
        got = np.load(ids_path, allow_pickle=False)
        parity = {}
        if workload in got.files:  # the headline: the timed rows' oracle ids against the GPU's
            gpu = got[workload]
            ref = np.asarray(ids1)
            rows_all = [int(i) for i in sel]
            parity[workload] = _parity_rows(w, rows_all, gpu)
            assert parity[workload]["mismatches"] == int(np.sum(gpu[sel] != ref))
        for name in ("char65", "zipf32k", "zipf152k"):
            if name in got.files and name != workload:
                wn = workloads.WORKLOADS[name]()
                Bn = wn["logits"].shape[0]
                rows_n = list(range(Bn)) if Bn <= 256 else list(range(0, Bn, Bn // 128))
                parity[name] = _parity_rows(wn, rows_n, got[name])
        if "spec32k_tokens" in got.files:
            parity["spec32k"] = _parity_verify(workloads.spec32k(), got["spec32k_tokens"], got["spec32k_nacc"])
    print(json.dumps({
        "value": len(sel) / med, "unit": "rows/s", "cores": 1, "kind": "port",
        "sample": f"{len(sel)} of {B} {workload} rows (evenly spaced, all parameter groups), "
                  f"median of {reps} reps of {med:.2f} s, numpy {np.__version__}, "
                  f"host cpus {os.cpu_count()} ({len(cores)} allowed), {_cpu_model()}",
        "all_cores": {"value": len(sel) / pmed, "unit": "rows/s", "cores": n,
                      "sample": f"the same rows over {n} single-core processes, median of {reps} reps "
                                f"of {pmed:.3f} s"},
        "parity": parity,
    }))


def run_cpu_baseline(workload: str, rows: int, reps: int, ids_path: str | None = None):
    env = dict(os.environ, OMP_NUM_THREADS="1", OPENBLAS_NUM_THREADS="1", MKL_NUM_THREADS="1",
               HIP_VISIBLE_DEVICES="", CUDA_VISIBLE_DEVICES="")
    cmd = [sys.executable, str(Path(__file__).resolve()), "--cpu-baseline-child", "--workload", workload,
           "--cpu-rows", str(rows), "--cpu-reps", str(reps)]
    if ids_path:
        cmd += ["--gpu-ids", ids_path]
    r = subprocess.run(cmd, capture_output=True, text=True, env=env, timeout=900)
    if r.returncode != 0:
        sys.stderr.write(r.stderr)
        return None
    return json.loads(r.stdout.strip().splitlines()[-1])


COPY_BYTES = 256 << 20


def _probe_rows(workload: str, group: int | None, B: int) -> list:
    """Rows of a counter probe: the whole batch, or (mixed128k) one of its
    four parameter groups of 64 rows, repeated to the batch size so the
    chunk kernel runs a full grid of one row mode."""
    if group is None:
        return list(range(B))
    if workload != "mixed128k" or not 0 <= group < 4:
        raise SystemExit("--probe-group applies to mixed128k's four row groups (0-3)")
    g = list(range(64 * group, 64 * group + 64))
    return (g * (B // 64 + 1))[:B]


def pmc_probe(workload: str, group: int | None = None) -> None:
    """A short run for counter collection: a copy of COPY_BYTES (the
    calibration), then a few sampler steps (all rows, or one row group)."""
    import numpy as np
    import torch

    from pagellm_amd import _native, workloads
    from pagellm_amd.sampling import _nucleus_hint, _pack_histories, _pack_params

    if workload == "spec32k":
        _pmc_probe_verify()
        return
    w = workloads.WORKLOADS[workload]()
    B, V = w["logits"].shape
    rows = _probe_rows(workload, group, B)
    params = [w["params"][i] for i in rows]
    contexts = [w["contexts"][i] for i in rows]
    dev = torch.device("cuda:0")
    ctx = _native.Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    t, k, p, r = _pack_params(params)
    hint = _nucleus_hint(t, k, p, w["logits"].shape[1])
    hist_ids, hist_off = _pack_histories(contexts, params, B, V)
    x = torch.from_numpy(np.ascontiguousarray(w["logits"][rows])).to(dev)
    d = {n: torch.from_numpy(a).to(dev) for n, a in
         dict(t=t, k=k, p=p, r=r, u=w["uniforms"][rows], ids=hist_ids, off=hist_off).items() if a is not None}
    out = torch.empty(B, dtype=torch.int32, device=dev)
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    for _ in range(PROBE_STEPS):
        ctx.sample(x.data_ptr(), _native.PLH_F32, V, B, V,
                   d["ids"].data_ptr() if "ids" in d else None, d["off"].data_ptr() if "off" in d else None,
                   d["t"].data_ptr(), d["k"].data_ptr(), d["p"].data_ptr(), d["r"].data_ptr(),
                   d["u"].data_ptr(), out.data_ptr(), None, hint)
    torch.cuda.synchronize()
    ctx.close()
    print("pmc probe done", flush=True)


PROBE_STEPS = 3


def _pmc_probe_verify() -> None:
    """The counter probe of spec32k: the calibration copy, then PROBE_STEPS
    verify calls on one set of p and q."""
    import torch

    from pagellm_amd import _native, workloads

    w = workloads.spec32k()
    B, k1, V = w["p"].shape
    k = k1 - 1
    dev = torch.device("cuda:0")
    ctx = _native.Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    d = {n: torch.from_numpy(w[n]).to(dev) for n in ("p", "q", "accept_u", "resample_u")}
    dr = torch.from_numpy(w["draft"].astype("int32")).to(dev)
    tok = torch.empty((B, k1), dtype=torch.int32, device=dev)
    nacc = torch.empty(B, dtype=torch.int32, device=dev)
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    for _ in range(PROBE_STEPS):
        ctx.verify(d["p"].data_ptr(), d["q"].data_ptr(), _native.PLH_F64, B, k, V, dr.data_ptr(),
                   d["accept_u"].data_ptr(), d["resample_u"].data_ptr(), False, tok.data_ptr(), nacc.data_ptr())
    torch.cuda.synchronize()
    ctx.close()
    print("pmc probe done", flush=True)


def _spec32k_compulsory_bytes() -> int:
    """Bytes one spec32k verify call must read (data dependent, from the
    oracle's stop positions): 16 B per accept test made, then p and q of
    the rejected position, or p_k after k acceptances (float64)."""
    import numpy as np

    from pagellm_amd import workloads

    w = workloads.spec32k()
    B, k1, V = w["p"].shape
    k = k1 - 1
    rows = np.arange(B)[:, None]
    px = w["p"][rows, np.arange(k)[None, :], w["draft"]]
    qx = w["q"][rows, np.arange(k)[None, :], w["draft"]]
    with np.errstate(divide="ignore", invalid="ignore"):
        ok = w["accept_u"] < np.minimum(1.0, px / qx)  # speculative.py:51-53
    n = np.where(ok.all(axis=1), k, np.argmin(ok, axis=1))  # the first rejection, else k
    return int(sum(16 * min(int(s) + 1, k) + (16 * V if s < k else 8 * V) for s in n))


def traffic_from(workload: str, fetch_dir: str, write_dir: str, dst: Path | None = None) -> dict:
    """HBM bytes per launch of every sampler kernel from the two counter
    runs of a --pmc-probe (PROBE_STEPS steps), their sum per step, and (for
    the headline) k_sample_chunks alone; written to
    profiles/traffic_<workload>.json (or dst)."""
    import csv

    def per_kernel(folder: str, counter: str):
        rows = {}
        for f in Path(folder).rglob("*counter_collection.csv"):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] != counter:
                    continue
                key = (r["Dispatch_Id"], r["Kernel_Name"])
                rows[key] = rows.get(key, 0.0) + float(r["Counter_Value"])
        return rows

    def short(n: str) -> str:
        n = n.split("(")[0].split("<")[0]
        return n.split("::")[-1]

    res, kernels = {}, {}
    for counter, folder in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = per_kernel(folder, counter)
        copies = [v for (_, n), v in rows.items() if "copy" in n.lower() or "elementwise" in n.lower()]
        if not copies:
            raise SystemExit(f"{counter}: no copy dispatch in {folder}")
        kib_copy = max(copies)
        factor = COPY_BYTES / (kib_copy * 1024.0)
        mine = {}
        for (_, n), v in rows.items():
            if short(n).startswith(("k_sample", "k_nuc", "k_verify")):
                mine.setdefault(short(n), []).append(v)
        if not mine:
            raise SystemExit(f"{counter}: no sampler kernel dispatch in {folder}")
        for name, vs in mine.items():
            kernels.setdefault(name, {})[counter] = {
                "launches": len(vs), "kib_per_launch": sum(vs) / len(vs),
                "bytes_per_launch": sum(vs) / len(vs) * 1024.0 * factor}
        res[counter] = {"copy_kib": kib_copy, "copy_bytes": COPY_BYTES, "scale": factor}
    per_kernel_out = {}
    step = 0.0
    for name, c in sorted(kernels.items()):
        b = sum(c[k]["bytes_per_launch"] for k in c)
        per_step = b * c["FETCH_SIZE"]["launches"] / PROBE_STEPS if "FETCH_SIZE" in c else b
        per_kernel_out[name] = {"bytes_per_launch": b, "launches_per_step": c.get("FETCH_SIZE", {}).get("launches", 0)
                                / PROBE_STEPS, "counters": c}
        step += per_step
    from pagellm_amd import workloads
    if workload == "spec32k":
        alg = _spec32k_compulsory_bytes()
    else:
        alg = workloads.algorithmic_bytes(workloads.WORKLOADS[workload]())
    out = {"workload": workload, "probe_steps": PROBE_STEPS, "bytes_per_step": step,
           "algorithmic_bytes": alg, "traffic_over_algorithmic": step / alg, "per_kernel": per_kernel_out,
           "calibration": res}
    if "k_sample_chunks" in per_kernel_out:  # the headline's dominant kernel
        out["kernel"] = "k_sample_chunks"
        out["bytes_per_launch"] = per_kernel_out["k_sample_chunks"]["bytes_per_launch"]
    dst = dst if dst is not None else ROOT / "profiles" / f"traffic_{workload}.json"
    dst.write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out))
    return out


PHASES = {0: "start", 1: "wave parts", 2: "normaliser", 3: "row buckets", 4: "cut-bucket entries loaded",
          10: "mass selection start", 14: "level bins counted", 15: "level barrier passed",
          11: "level pick", 12: "rank list", 13: "ranked",
          5: "cut selected", 6: "per-chunk kept sums", 7: "draw bins", 8: "draw bin scattered", 9: "end"}


CHUNK_PHASES = {1: "register maxima", 2: "chunk range", 3: "threshold", 4: "counted", 5: "placed",
                6: "buckets written", 7: "end (wave 0)"}


def chunk_timeline(ph, rt, hw, B: int, C: int) -> dict:
    """k_sample_chunks' stamps of one step (ph [g, 8] shader clock, rt [g, 9]
    real-time clock: start, then each wave's end, hw [g, 2] HW_ID and XCC_ID):
    the clock rate, the kernel's span, the workgroups' lifetimes, how many
    were resident per CU on average and over time, and the gap between a
    workgroup's last wave ending and the next workgroup starting in the CU
    slot it freed."""
    import numpy as np

    n = B * C
    ph, rt, hw = ph[:n], rt[:n], hw[:n]
    start, wend = rt[:, 0], rt[:, 1:]
    end = wend.max(axis=1)
    life = end - start
    ghz = float(np.median((ph[:, 7] - ph[:, 0]) / np.maximum(wend[:, 0] - start, 1))) / 10.0
    cu = ((hw[:, 1] & 0xF) * 8 + ((hw[:, 0] >> 13) & 7)) * 32 + ((hw[:, 0] >> 12) & 1) * 16 + ((hw[:, 0] >> 8) & 0xF)
    t0, span = start.min(), end.max() - start.min()
    cus = np.unique(cu)
    bins = 10
    edges = t0 + span * (np.arange(bins) + 0.5) / bins
    occ = [float(((start[None, :] <= e) & (end[None, :] > e)).sum()) / len(cus) for e in edges]
    gaps = []
    for c in cus:
        idx = np.where(cu == c)[0]
        idx = idx[np.argsort(start[idx])]
        held = []
        for j in idx:
            held.sort()
            if len(held) >= 2:
                gaps.append(start[j] - held.pop(0))
            held.append(end[j])
    us = 0.01  # real-time clock: 100 MHz
    return {"clock_ghz": round(ghz, 3), "cus": int(len(cus)), "span_us": round(float(span) * us, 2),
            "workgroup_life_us_median": round(float(np.median(life)) * us, 2),
            "resident_workgroups_per_cu_mean": round(float(life.sum()) / (len(cus) * float(span)), 2),
            "resident_workgroups_per_cu_over_time": [round(v, 2) for v in occ],
            "slot_refill_gap_us_median": round(float(np.median(gaps)) * us, 3) if gaps else None,
            "wave0_end_to_last_wave_end_us_median": round(float(np.median(end - wend[:, 0])) * us, 3)}


def phase_stamps(steps: int = 6) -> dict:
    """k_sample_final's and k_sample_chunks' phase clock stamps on
    mixed128k, from the profiling build (python -m pagellm_amd.build
    --phase-stamps): per row group, the median over rows (chunks) and steps
    (the first step dropped) of the shader clock ticks from the workgroup's
    start to each phase it reaches; for the chunk kernel also its timeline
    (chunk_timeline) per step."""
    import ctypes

    import numpy as np
    import torch

    from pagellm_amd import _native, workloads
    from pagellm_amd.sampling import _pack_histories, _pack_params

    _native.LIB_PATH = ROOT / "pagellm_amd" / "_stamps" / "libpagellm_hip.so"
    if not _native.LIB_PATH.exists():
        raise SystemExit("build the profiling library first: python -m pagellm_amd.build --phase-stamps")
    w = workloads.mixed128k()
    B, V = w["logits"].shape
    dev = torch.device("cuda:0")
    ctx = _native.Context(0)
    t, k, p, r = _pack_params(w["params"])
    hist_ids, hist_off = _pack_histories(w["contexts"], w["params"], B, V)
    x = torch.from_numpy(w["logits"]).to(dev)
    d = {n: torch.from_numpy(a).to(dev) for n, a in
         dict(t=t, k=k, p=p, r=r, u=w["uniforms"], ids=hist_ids, off=hist_off).items()}
    out = torch.empty(B, dtype=torch.int32, device=dev)
    runs, cruns, fruns = [], [], []
    C = (V + 16383) // 16384  # 64 KB chunks of float32
    for _ in range(steps):
        ctx.sample(x.data_ptr(), _native.PLH_F32, V, B, V, d["ids"].data_ptr(), d["off"].data_ptr(),
                   d["t"].data_ptr(), d["k"].data_ptr(), d["p"].data_ptr(), d["r"].data_ptr(),
                   d["u"].data_ptr(), out.data_ptr(), None, 0)
        torch.cuda.synchronize()
        buf = (ctypes.c_ulonglong * (256 * 16))()
        if ctx.lib.plh_phase_stamps(buf) != 0:
            raise SystemExit("plh_phase_stamps failed")
        runs.append(np.frombuffer(buf, dtype=np.uint64).reshape(256, 16).astype(np.int64))
        cph, crt, chw = (ctypes.c_ulonglong * (4096 * 8))(), (ctypes.c_ulonglong * (4096 * 9))(), (ctypes.c_uint * (4096 * 2))()
        if ctx.lib.plh_chunk_stamps(cph, crt, chw) != 0:
            raise SystemExit("plh_chunk_stamps failed")
        cruns.append((np.frombuffer(cph, dtype=np.uint64).reshape(4096, 8).astype(np.int64),
                      np.frombuffer(crt, dtype=np.uint64).reshape(4096, 9).astype(np.int64),
                      np.frombuffer(chw, dtype=np.uint32).reshape(4096, 2).astype(np.int64)))
        frt = (ctypes.c_ulonglong * (256 * 2))()
        if ctx.lib.plh_final_rt(frt) != 0:
            raise SystemExit("plh_final_rt failed")
        fruns.append(np.frombuffer(frt, dtype=np.uint64).reshape(256, 2).astype(np.int64))
    ctx.close()
    a = np.stack(runs[1:])
    res = {"workload": "mixed128k", "unit": "shader clock ticks from the workgroup's start", "groups": {},
           "chunk_groups": {}, "chunk_timeline": [chunk_timeline(*r, B, C) for r in cruns[1:]],
           "final_timeline": []}
    for (cp_, crt_, _), frt_ in zip(cruns[1:], fruns[1:]):
        chunk_end = crt_[:B * C, 1:].max()
        f0, f1 = frt_[:B, 0], frt_[:B, 1]
        life = f1 - f0
        res["final_timeline"].append({
            "gap_us_chunk_last_wave_to_first_merge_start": round(float(f0.min() - chunk_end) * 0.01, 2),
            "span_us": round(float(f1.max() - f0.min()) * 0.01, 2),
            "start_spread_us": round(float(f0.max() - f0.min()) * 0.01, 2),
            "life_us_median_per_group": [round(float(np.median(life[64 * g:64 * g + 64])) * 0.01, 2) for g in range(4)]})
    cph = np.stack([r[0][:B * C] for r in cruns[1:]])
    for g in range(4):
        blk = cph[:, 64 * g * C:64 * (g + 1) * C, :]
        rel = blk - blk[:, :, 0:1]
        ph = {}
        for kk, name in CHUNK_PHASES.items():
            v = rel[:, :, kk].reshape(-1)
            v = v[(v > 0) & (v < 10 ** 7)]
            if len(v):
                ph[name] = int(np.median(v))
        res["chunk_groups"][f"group {g}"] = ph
    names = ["greedy", "top_k 50", "top_p 0.9", "top_k 40 + top_p 0.95 + T 0.6 + penalty 1.1"]
    for g in range(4):
        blk = a[:, 64 * g:64 * g + 64, :]
        rel = blk - blk[:, :, 0:1]
        ph = {}
        for kk in PHASES:
            if kk == 0:
                continue
            v = rel[:, :, kk].reshape(-1)
            v = v[(v > 0) & (v < 10 ** 7)]  # phases a row does not reach keep a stale or zero stamp
            if len(v):
                ph[PHASES[kk]] = int(np.median(v))
        res["groups"][f"group {g}: {names[g]}"] = dict(sorted(ph.items(), key=lambda kv: kv[1]))
    return res


VALU_COUNTERS = ("SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_WAVES")


def valu_from(workload: str, dirs: list, dst: Path | None = None, shape: tuple | None = None) -> dict:
    """Instructions per token of k_sample_chunks for each mixed128k row
    group, from one rocprofv3 counter run per group (`--pmc SQ_INSTS_VALU
    SQ_INSTS_SALU SQ_INSTS_LDS SQ_WAVES -- python3 bench.py --pmc-probe
    --probe-group G`, G = 0..3 in the order given): wave instructions x 64
    lanes / tokens per launch, written to profiles/valu_<workload>.json."""
    import csv

    if shape is None:
        from pagellm_amd import workloads
        shape = workloads.WORKLOADS[workload]()["logits"].shape
    B, V = shape
    names = ["greedy", "top_k 50", "top_p 0.9", "top_k 40 + top_p 0.95 + T 0.6 + penalty 1.1"]
    groups = []
    for gi, folder in enumerate(dirs):
        per = {}
        for f in Path(folder).rglob("*counter_collection.csv"):
            for r in csv.DictReader(open(f)):
                if "k_sample_chunks" not in r["Kernel_Name"] or r["Counter_Name"] not in VALU_COUNTERS:
                    continue
                per.setdefault(r["Dispatch_Id"], {}).setdefault(r["Counter_Name"], 0.0)
                per[r["Dispatch_Id"]][r["Counter_Name"]] += float(r["Counter_Value"])
        if not per:
            raise SystemExit(f"no k_sample_chunks counters in {folder}")
        launches = list(per.values())
        mean = {c: sum(x.get(c, 0.0) for x in launches) / len(launches) for c in VALU_COUNTERS}
        tokens = B * V
        groups.append({"group": gi, "rows": names[gi] if gi < len(names) else str(gi), "launches": len(launches),
                       "per_launch": mean,
                       "valu_per_token": mean["SQ_INSTS_VALU"] * 64 / tokens,
                       "salu_per_token": mean["SQ_INSTS_SALU"] * 64 / tokens,
                       "lds_per_token": mean["SQ_INSTS_LDS"] * 64 / tokens})
    out = {"workload": workload, "kernel": "k_sample_chunks", "tokens_per_launch": B * V,
           "note": "wave instructions x 64 lanes / tokens; each group's 64 rows repeated to 256",
           "groups": groups}
    dst = dst if dst is not None else ROOT / "profiles" / f"valu_{workload}.json"
    dst.write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out))
    return out


def valu_kernels_from(workload: str, folder: str, dst: Path | None = None, shape: tuple | None = None) -> dict:
    """Instructions per token of every sampler kernel of one counter run of
    the whole batch (`--pmc SQ_INSTS_VALU SQ_INSTS_SALU SQ_INSTS_LDS
    SQ_WAVES -- python3 bench.py --pmc-probe --workload W`): per kernel
    (template arguments dropped), the counters averaged over its launches,
    wave instructions x 64 lanes / the batch's tokens, written to
    profiles/valu_kernels_<workload>.json."""
    import csv

    if shape is None:
        from pagellm_amd import workloads
        shape = workloads.WORKLOADS[workload]()["logits"].shape
    B, V = shape
    per = {}
    for f in Path(folder).rglob("*counter_collection.csv"):
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] not in VALU_COUNTERS:
                continue
            name = r["Kernel_Name"].split("(")[0].split("<")[0].replace("void ", "").replace("plh::", "")
            if not name.startswith(("k_sample", "k_nuc")):
                continue
            d = per.setdefault(name, {}).setdefault(r["Dispatch_Id"], {})
            d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    if not per:
        raise SystemExit(f"no sampler kernel counters in {folder}")
    tokens = B * V
    kernels = []
    for name, launches in sorted(per.items()):
        mean = {c: sum(x.get(c, 0.0) for x in launches.values()) / len(launches) for c in VALU_COUNTERS}
        kernels.append({"kernel": name, "launches": len(launches), "per_launch": mean,
                        "valu_per_token": mean["SQ_INSTS_VALU"] * 64 / tokens,
                        "salu_per_token": mean["SQ_INSTS_SALU"] * 64 / tokens,
                        "lds_per_token": mean["SQ_INSTS_LDS"] * 64 / tokens})
    out = {"workload": workload, "tokens_per_launch": tokens,
           "note": "wave instructions x 64 lanes / the batch's tokens, per kernel launch", "kernels": kernels}
    dst = dst if dst is not None else ROOT / "profiles" / f"valu_kernels_{workload}.json"
    dst.write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out))
    return out


MALL_BYTES = 256 << 20  # MI355X Infinity Cache
ROTATE_BYTES = 2 * MALL_BYTES  # rotating input sets span at least this much, so steps stream from HBM


def _n_sets(set_bytes: int, least: int = 2, most: int = 64) -> int:
    """Copies to rotate: enough to span ROTATE_BYTES, at most `most` (a
    config too small to fill the cache that way is latency-bound anyway and
    is labelled cache-resident)."""
    return min(most, max(least, -(-ROTATE_BYTES // max(1, set_bytes))))


def bench_config(name: str, steps: int = 20, warmup: int = 3) -> dict:
    """rows/s of one more sampling workload, inputs resident in HBM, timed
    with HIP events like the headline.  Enough copies of the logits rotate
    across steps to span twice the 256 MB Infinity Cache, so every step
    reads its logits from HBM.  Also returns the ids of the last step."""
    import torch

    from pagellm_amd import _native, workloads
    from pagellm_amd.sampling import _nucleus_hint, _pack_histories, _pack_params

    w = workloads.WORKLOADS[name]()
    B, V = w["logits"].shape
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    ctx = _native.Context(0)
    ctx.set_stream(stream.cuda_stream)
    t, k, p, r = _pack_params(w["params"])
    hint = _nucleus_hint(t, k, p, w["logits"].shape[1])
    hist_ids, hist_off = _pack_histories(w["contexts"], w["params"], B, V)
    nsets = _n_sets(w["logits"].nbytes)
    x0 = torch.from_numpy(w["logits"]).to(dev)
    xs = [x0] + [x0.clone() for _ in range(nsets - 1)]
    d = {n: torch.from_numpy(a).to(dev) for n, a in
         dict(t=t, k=k, p=p, r=r, u=w["uniforms"], ids=hist_ids, off=hist_off).items() if a is not None}
    out = torch.empty(B, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()

    def step(i):
        ctx.sample(xs[i % nsets].data_ptr(), _native.PLH_F32, V, B, V,
                   d["ids"].data_ptr() if "ids" in d else None, d["off"].data_ptr() if "off" in d else None,
                   d["t"].data_ptr(), d["k"].data_ptr(), d["p"].data_ptr(), d["r"].data_ptr(),
                   d["u"].data_ptr(), out.data_ptr(), None, hint)

    fb0 = ctx.fallback_rows()
    with torch.cuda.stream(stream):
        for i in range(warmup):
            step(i)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(steps):
            step(i)
        b.record(stream)
        torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    nbytes = workloads.algorithmic_bytes(w)
    res = {"rows_per_s": B / (ms * 1e-3), "ms_per_step": ms, "batch": B, "vocab": V,
           "algorithmic_bytes_per_step": nbytes, "hbm_gbps": nbytes / (ms * 1e-3) / 1e9,
           "rotating_input_sets": nsets, "inputs_bytes_rotated": nsets * w["logits"].nbytes,
           "inputs_cache_resident": nsets * w["logits"].nbytes < MALL_BYTES,
           "fallback_rows_per_step": (ctx.fallback_rows() - fb0) / (warmup + steps)}
    ids = out.cpu().numpy().astype("int64")
    ctx.close()
    del xs, x0
    torch.cuda.empty_cache()
    return res, ids


def bench_verify(steps: int = 50, warmup: int = 5) -> dict:
    """The speculative verify workload (64 rows, k = 4, V = 32000, float64 p
    and q resident in HBM): rows/s and the data-dependent compulsory bytes
    (per row: 16 B per accept test, then the rows the final draw reads:
    p and q of the rejected position, or p_k).  p/q copies rotate across
    steps (each set is 147 MB; together they span twice the Infinity
    Cache).  A second pass with the library's kernel timing gives the two
    launches' average durations.  Also returns the last step's outputs."""
    import torch

    from pagellm_amd import _native, workloads

    w = workloads.spec32k()
    B, k1, V = w["p"].shape
    k = k1 - 1
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    ctx = _native.Context(0)
    ctx.set_stream(stream.cuda_stream)
    nsets = _n_sets(w["p"].nbytes + w["q"].nbytes)
    p0 = torch.from_numpy(w["p"]).to(dev)
    q0 = torch.from_numpy(w["q"]).to(dev)
    ps = [p0] + [p0.clone() for _ in range(nsets - 1)]
    qs = [q0] + [q0.clone() for _ in range(nsets - 1)]
    dr = torch.from_numpy(w["draft"].astype("int32")).to(dev)
    au = torch.from_numpy(w["accept_u"]).to(dev)
    ru = torch.from_numpy(w["resample_u"]).to(dev)
    tok = torch.empty((B, k1), dtype=torch.int32, device=dev)
    nacc = torch.empty(B, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()

    def step(i):
        ctx.verify(ps[i % nsets].data_ptr(), qs[i % nsets].data_ptr(), _native.PLH_F64, B, k, V, dr.data_ptr(),
                   au.data_ptr(), ru.data_ptr(), False, tok.data_ptr(), nacc.data_ptr())

    with torch.cuda.stream(stream):
        for i in range(warmup):
            step(i)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(steps):
            step(i)
        b.record(stream)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / steps
        ctx.set_kernel_timing(True)
        ctx.kernel_times()
        for i in range(steps):
            step(i)
        parts_ms, draw_ms, calls = ctx.kernel_times()
        ctx.set_kernel_timing(False)
    n = nacc.cpu().numpy()
    nbytes = int(sum(16 * (min(int(s) + 1, k)) + (16 * V if s < k else 8 * V) for s in n))
    res = {"rows_per_s": B / (ms * 1e-3), "ms_per_step": ms, "batch": B, "k": k, "vocab": V,
           "accepted_per_row": float(n.mean()), "compulsory_bytes_per_step": nbytes,
           "hbm_gbps": nbytes / (ms * 1e-3) / 1e9, "rotating_input_sets": nsets,
           "kernel_ms": {"k_verify_parts": parts_ms / max(1, calls), "k_verify_draw": draw_ms / max(1, calls)}}
    out = (tok.cpu().numpy().astype("int64"), n.astype("int64"))
    ctx.close()
    del ps, qs, p0, q0
    torch.cuda.empty_cache()
    return res, out


def bench_head(steps: int = 20, warmup: int = 3, N: int = 256, D: int = 4096, V: int = 128256) -> dict:
    """The logits producer at the sampler's headline shape: final RMSNorm and
    lm_head (256 rows, model width 4096, 128 256-token vocabulary, float32
    weights resident in HBM, random-init) writing the logits the sampler
    reads.  Reports launches/s of the pair and the product's float32 matrix
    rate against the 157.3 TFLOP/s fp32 MFMA peak."""
    import torch

    from pagellm_amd import _native

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    h = torch.randn((N, D), device=dev, dtype=torch.float32, generator=g)
    norm = 1 + 0.1 * torch.randn(D, device=dev, dtype=torch.float32, generator=g)
    W = 0.02 * torch.randn((D, V), device=dev, dtype=torch.float32, generator=g)
    out = torch.empty((N, V), device=dev, dtype=torch.float32)
    stream = torch.cuda.Stream(device=dev)
    ctx = _native.Context(0)
    ctx.set_stream(stream.cuda_stream)
    torch.cuda.synchronize()

    def step():
        ctx.rmsnorm_lm_head(h.data_ptr(), D, N, D, norm.data_ptr(), 1e-5, W.data_ptr(), V, V, out.data_ptr(), V)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(steps):
        step()
    b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    flops = 2.0 * N * D * V
    tflops = flops / (ms * 1e-3) / 1e12
    res = {"launches_per_s": 1e3 / ms, "ms_per_step": ms, "rows": N, "width": D, "vocab": V,
           "dtype": "fp32", "flop_per_step": flops, "tflops": tflops, "mfma_fp32_frac": tflops / PEAK_FP32_MFMA_TFLOPS,
           "weight_bytes": 4 * D * V, "weight_gbps": 4.0 * D * V / (ms * 1e-3) / 1e9}
    ctx.close()
    return res


def copy_bandwidth(nbytes: int = 1 << 30, reps: int = 10) -> float:
    """GB/s of a plain device-to-device copy (bytes read + bytes written per
    second): the secondary, measured denominator beside the 8 TB/s peak."""
    import torch

    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    gbps = 2.0 * nbytes * reps / (a.elapsed_time(b) * 1e-3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return gbps


def bench_end_to_end(w, logits, steps: int = 50, warmup: int = 5) -> dict:
    """Host-inclusive time per step of the engine adapter with the logits
    already in HBM: each step uploads the per-row parameters, uniforms and
    history spans from the host, runs the sampler, appends the ids to the
    device-resident histories and downloads the ids (wall clock, one host
    thread, the download waits for the step)."""
    import numpy as np

    from pagellm_amd import _native
    from pagellm_amd.engine import BatchSampler, DeviceHistories

    B, V = w["logits"].shape
    H = max(len(c) for c in w["contexts"])
    hist = DeviceHistories(V, B, H + warmup + steps + 1, ctx=_native.Context(0))
    for b in range(B):
        hist.add(b, np.asarray(w["contexts"][b]))
    sampler = BatchSampler(hist)
    keys = list(range(B))
    u = w["uniforms"]
    for _ in range(warmup):
        sampler.sample(logits, w["params"], None, keys, uniforms=u)
    t0 = time.perf_counter()
    for _ in range(steps):
        ids = sampler.sample(logits, w["params"], None, keys, uniforms=u)
    dt = (time.perf_counter() - t0) / steps
    hist.ctx.close()
    return {"us_per_step": dt * 1e6, "rows_per_s": B / dt, "steps": steps, "ids_checked": int(ids.shape[0])}


def load_traffic(workload: str):
    f = ROOT / "profiles" / f"traffic_{workload}.json"
    if f.exists():
        try:
            return json.loads(f.read_text()).get("bytes_per_launch")
        except Exception:
            return None
    return None


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="mixed128k", choices=["mixed128k", "zipf32k", "zipf152k", "char65", "spec32k"],
                    help="spec32k: counter probes and traffic summaries only")
    ap.add_argument("--sets", type=int, default=3, help="rotating input copies")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=256)
    ap.add_argument("--cpu-reps", type=int, default=5)
    ap.add_argument("--cpu-baseline-child", action="store_true")
    ap.add_argument("--gpu-ids", help="(child) .npz of the GPU ids each configuration produced")
    ap.add_argument("--pmc-probe", action="store_true", help="short run for rocprofv3 counter passes")
    ap.add_argument("--phase-stamps", action="store_true",
                    help="k_sample_final's phase clock stamps on mixed128k (the profiling build)")
    ap.add_argument("--probe-group", type=int, help="(--pmc-probe) one mixed128k row group, 0-3, repeated")
    ap.add_argument("--valu-from", nargs="+", metavar="DIR",
                    help="counter run folders of --pmc-probe --probe-group 0..3 -> profiles/valu_<workload>.json")
    ap.add_argument("--valu-kernels-from", metavar="DIR",
                    help="counter run folder of --pmc-probe (whole batch) -> profiles/valu_kernels_<workload>.json")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the other workloads (zipf32k, zipf152k, char65, spec32k verify)")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"))
    ap.add_argument("--only", choices=["spec32k", "head128k", "zipf32k", "zipf152k", "char65"],
                    help="run one of the other configurations alone and print its JSON (for profiling)")
    args = ap.parse_args()

    if args.cpu_baseline_child:
        cpu_baseline_child(args.workload, args.cpu_rows, args.cpu_reps, args.gpu_ids)
        return
    if args.traffic_from:
        traffic_from(args.workload, *args.traffic_from)
        return
    if args.valu_from:
        valu_from(args.workload, args.valu_from)
        return
    if args.valu_kernels_from:
        valu_kernels_from(args.workload, args.valu_kernels_from)
        return
    if args.phase_stamps:
        print(json.dumps(phase_stamps(), indent=1))
        return
    if args.pmc_probe:
        pmc_probe(args.workload, args.probe_group)
        return
    if args.only:
        kw = dict(steps=min(args.steps, 50), warmup=min(args.warmup, 5))
        if args.only == "head128k":
            res = bench_head(**kw)
        elif args.only == "spec32k":
            res = bench_verify(**kw)[0]
        else:
            res = bench_config(args.only, **kw)[0]
        print(json.dumps(res), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(rows shard across GPUs with no exchange; see the sharding notes in the design document)",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from pagellm_amd import _native, workloads
    from pagellm_amd.sampling import _nucleus_hint, _pack_histories, _pack_params

    print(f"[bench] generating {args.workload}", file=sys.stderr, flush=True)
    w = workloads.WORKLOADS[args.workload]()
    B, V = w["logits"].shape
    algo_bytes = workloads.algorithmic_bytes(w)

    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    ctx = _native.Context(0)
    ctx.set_stream(stream.cuda_stream)
    torch.cuda.set_stream(stream)

    t, k, p, r = _pack_params(w["params"])
    hint = _nucleus_hint(t, k, p, w["logits"].shape[1])
    hist_ids, hist_off = _pack_histories(w["contexts"], w["params"], B, V)
    logits = [torch.from_numpy(w["logits"]).to(dev) for _ in range(args.sets)]
    d = {n: torch.from_numpy(a).to(dev) for n, a in
         dict(t=t, k=k, p=p, r=r, u=w["uniforms"], ids=hist_ids, off=hist_off).items() if a is not None}
    out = torch.empty(B, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()

    def step(i):
        x = logits[i % args.sets]
        ctx.sample(x.data_ptr(), _native.PLH_F32, V, B, V,
                   d["ids"].data_ptr() if "ids" in d else None, d["off"].data_ptr() if "off" in d else None,
                   d["t"].data_ptr(), d["k"].data_ptr(), d["p"].data_ptr(), d["r"].data_ptr(),
                   d["u"].data_ptr(), out.data_ptr(), None, hint)

    fb0 = ctx.fallback_rows()
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(args.steps):
        step(i)
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    fallback = (ctx.fallback_rows() - fb0) / max(1, args.warmup + args.steps)

    # per-kernel durations of the same steps (events between the two launches)
    ctx.set_kernel_timing(True)
    ctx.kernel_times()
    for i in range(args.steps):
        step(i)
    stream_ms, merge_ms, calls = ctx.kernel_times()
    ctx.set_kernel_timing(False)
    kernel_ms = stream_ms / max(1, calls)
    merge_avg_ms = merge_ms / max(1, calls)

    # each step bracketed on its own, for the spread across steps
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for i, (e0, e1) in enumerate(evs):
        e0.record(stream)
        step(i)
        e1.record(stream)
    torch.cuda.synchronize()
    per_step = np.array([e0.elapsed_time(e1) for e0, e1 in evs])

    ids = out.cpu().numpy()
    greedy = [i for i, pp in enumerate(w["params"]) if pp.greedy]
    if greedy and not np.array_equal(ids[greedy], np.argmax(w["logits"][greedy], axis=1)):
        print("[bench] WARNING: greedy rows disagree with numpy argmax", file=sys.stderr)

    rows_per_s = B / (ms * 1e-3)
    gbps = algo_bytes / (ms * 1e-3) / 1e9
    kernel_gbps = algo_bytes / (kernel_ms * 1e-3) / 1e9 if calls else None
    print("[bench] end to end (engine adapter, host in the loop)", file=sys.stderr, flush=True)
    e2e = bench_end_to_end(w, logits[0])
    print("[bench] copy bandwidth", file=sys.stderr, flush=True)
    copy_gbps = copy_bandwidth()
    others = None
    gpu_ids = {args.workload: ids.astype(np.int64)}
    if not args.no_other_configs:
        others = {}
        for name in ("char65", "zipf32k", "zipf152k"):
            if name != args.workload:
                print(f"[bench] other config {name}", file=sys.stderr, flush=True)
                others[name], gpu_ids[name] = bench_config(name)
        print("[bench] other config spec32k (verify)", file=sys.stderr, flush=True)
        others["spec32k"], (gpu_ids["spec32k_tokens"], gpu_ids["spec32k_nacc"]) = bench_verify()
        print("[bench] other config head128k (logits producer)", file=sys.stderr, flush=True)
        others["head128k"] = bench_head()
    cpu = None
    if not args.no_cpu_baseline:
        import tempfile

        print("[bench] CPU baseline and oracle parity", file=sys.stderr, flush=True)
        with tempfile.TemporaryDirectory() as td:
            ids_path = os.path.join(td, "gpu_ids.npz")
            np.savez(ids_path, **gpu_ids)
            cpu = run_cpu_baseline(args.workload, args.cpu_rows, args.cpu_reps, ids_path)
    parity = cpu.pop("parity", None) if cpu else None
    if others and parity:
        for name, v in parity.items():
            if name in others:
                others[name]["parity"] = v
    res = {
        "metric": METRIC,
        "value": rows_per_s,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": args.workload, "batch": B, "vocab": V, "logits_dtype": "fp32",
                   "rotating_input_sets": args.sets, "algorithmic_bytes_per_step": algo_bytes},
        "step_ms_spread": {"median": float(np.median(per_step)), "p10": float(np.percentile(per_step, 10)),
                           "p90": float(np.percentile(per_step, 90)), "max": float(per_step.max())},
        "step_hbm_gbps": gbps,
        "step_hbm_frac": gbps / PEAK_HBM_GBPS,
        "kernel_ms": {"k_sample_chunks": kernel_ms, "k_sample_final": merge_avg_ms},
        "fallback_rows_per_step": fallback,
        "roofline": {"bound": "hbm", "achieved": kernel_gbps, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": kernel_gbps / PEAK_HBM_GBPS if kernel_gbps else None,
                     "traffic": load_traffic(args.workload), "kernel": "k_sample_chunks",
                     "copy_gbps": copy_gbps, "frac_of_copy": kernel_gbps / copy_gbps if kernel_gbps else None},
        "parity": parity.get(args.workload) if parity else None,
        "end_to_end": e2e,
        "cpu_baseline": cpu,
        "other_configs": others,
    }
    print(json.dumps(res), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
