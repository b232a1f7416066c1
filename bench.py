#!/usr/bin/env python3
"""Benchmark of the fused GDN chunked forward on one MI355X.

Contract: ``python bench.py --gpus N --steps K --warmup W`` prints ONE JSON line.  A step is
one full forward of the headline workload (B=4, H=16, T=4096, C=64, dk=dv=128, bf16 inputs,
fp32 accumulation/state/output) through the C-ABI library: stage 1 (chunk-local gates, kkt,
(I+A)^-1) and stage 2 (the state scan fused with the output; it forms the gated causal score
q k^T from the q and k rows it stages).  Inputs are resident in HBM before timing starts; outputs
and the workspace are preallocated, so the timed region is launches only.  ``value`` is tokens/s
= B*T*K / t over exactly K steps: one HIP event pair on the launch stream brackets the K steps,
after a synchronize, with nothing else recorded inside the loop, and one synchronize follows.

Order of one run: the CPU baseline (a child process, before this process touches the GPU); a
256 MiB device-copy rate (a practical HBM ceiling measured in the same run); ``settle_s`` seconds
of untimed forwards (the GPU's clocks ramp over the first fraction of a second: without it a
20-step loop measured up to 15 % slower than a 200-step one); W warmup steps; the K timed steps;
then ``--event-steps`` forwards and as many stage-1 launches, each back to back under one event
pair on the launch stream, which give the per-kernel durations (stage 1 its loop's average,
stage 2 the forward's average minus stage 1's; they agree with the rocprofv3 kernel-trace
averages); then the secondary configurations.

Besides the required fields the line carries:
  * ``roofline`` — the dominant kernel (stage 2) against the MI355X HBM peak.  ``achieved`` is
    the forward's compulsory bytes (q, k, v, beta, g in, o and the final state out: 83 456 B per
    64-token chunk x 4096 chunks = 341.8 MB) over the kernel's event-timed average duration:
    stage 2 reads every input the forward needs and writes o and the state.  ``own_*`` are the
    same figures on the bytes stage 2 itself moves (it also reads T and G from stage 1's
    workspace: 90 624 B per chunk + the final state).  ``traffic`` is the counter-measured HBM
    bytes per launch recorded in profiles/hbm_traffic_gdn_forward.json, reported only when that
    record was taken from the library built from the current sources (its source hash), else
    null; ``kernel_avg_ms_rocprof`` / ``frac_rocprof`` are the kernel's rocprofv3 kernel-trace
    average (profiles/kernel_trace_gdn_forward.json, same source-hash rule) and the fraction
    recomputed from it;
  * ``stages`` — both kernels' average durations, bytes and flops, and their HBM / MFMA fractions;
  * ``forward`` — the whole forward's compulsory-byte and flop fractions at ``ms_per_step``,
    and the timed loop run REPEATS more times (``repeats_ms_per_step``, their median);
  * ``cpu_baseline`` — the fp32 numpy oracle (the reference's per-(b,h,c) loop) on this host's
    cores (oracle/cpu_baseline.py), with a one-core figure beside it;
  * ``secondary`` — the other benchmark configurations, each timed over back-to-back calls
    bracketed by one event pair on the launch stream (skipped with --no-secondary): the fused
    KDA forward at B=2, H=32, T=8192; the GDN long-context forward B=1, H=32, T=32768 with an
    initial state; the fp32 kkt + inverse over 4096 chunks; the fp32 DeltaNet forward B=1, H=4,
    T=512.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pto-fuser_amd"))
sys.path.insert(0, ROOT)

WORKLOAD = dict(B=4, H=16, T=4096, C=64, DK=128, DV=128)
SETTLE_S = 1.0      # untimed GPU work before the warmup steps (clock ramp)
REPEATS = 5         # further runs of the timed loop, reported as a median beside `value`
PEAK_HBM = 8.0e12          # MI355X HBM3E, bytes/s
PEAK_BF16 = 2.5e15         # dense bf16 MFMA, flop/s
PEAK_FP32 = 157.3e12       # dense fp32 MFMA, flop/s
METRIC = "GDN chunked-forward tokens/sec at B=4,H=16,T=4096 bf16; % MFMA/HBM roofline"
COUNTERS = os.path.join(ROOT, "profiles", "hbm_traffic_gdn_forward.json")
TRACE = os.path.join(ROOT, "profiles", "kernel_trace_gdn_forward.json")


def measured_traffic(kernel, lib_hash):
    """HBM bytes per launch of ``kernel`` from the recorded counter passes (FETCH_SIZE and
    WRITE_SIZE in KiB per dispatch, each scaled by what it reads for a plain copy of known
    size), or None when no record exists for the library built from the current sources."""
    try:
        with open(COUNTERS) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    if rec.get("source_hash") != lib_hash:
        return None
    kib = rec.get("kernels", {}).get(kernel)
    if kib is None:
        return None
    return int(sum(kib[c] * rec["scale"][c] * 1024 for c in ("FETCH_SIZE", "WRITE_SIZE")))


def traced_kernel_ms(kernel, lib_hash):
    """Average duration (ms) of ``kernel`` in the recorded rocprofv3 kernel trace, or None when
    no record exists for the library built from the current sources."""
    try:
        with open(TRACE) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    if rec.get("source_hash") != lib_hash:
        return None
    k = rec.get("kernels", {}).get(kernel)
    return None if k is None else k["avg_us"] / 1e3


def summarize_trace(trace_csv, lib_hash, out=None):
    """Write the kernel-trace record bench.py reads (``TRACE``) from the kernel_trace.csv of a
    ``rocprofv3 --kernel-trace --stats --output-format csv`` run of bench.py: per kernel (the keys
    of the counter record) the dispatch count and the average, median, min and max duration,
    tagged with the library's source hash."""
    import csv
    durs = {}
    with open(trace_csv) as f:
        for row in csv.DictReader(f):
            name = row["Kernel_Name"]
            if "Grid_Size" in row:
                grid = int(row["Grid_Size"])
            else:
                grid = int(row["Grid_Size_X"]) * int(row.get("Grid_Size_Y", 1)) * int(row.get("Grid_Size_Z", 1))
            key = _counter_key(name, grid)
            if key is not None:
                durs.setdefault(key, []).append(
                    (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3)
    kernels = {}
    for key, v in durs.items():
        v.sort()
        kernels[key] = {"dispatches": len(v), "avg_us": round(statistics.mean(v), 3),
                        "median_us": round(v[len(v) // 2], 3), "min_us": round(v[0], 3),
                        "max_us": round(v[-1], 3)}
    rec = {"workload": "GDN forward B4 H16 T4096 C64 dk=dv=128, bf16 in (bench.py headline); "
                       "long_*: bench.py gdn_config4_long_context; kda_*: bench.py kda_config5",
           "source_hash": lib_hash,
           "command": "rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o kt -- "
                      "python3 bench.py --steps 50 --warmup 10 --no-cpu-baseline",
           "kernels": kernels}
    with open(out or TRACE, "w") as f:
        json.dump(rec, f, indent=1)
    return rec


def _counter_key(name, grid):
    """Record key of a dispatch in the counter passes: the headline's two kernels (the 32-column
    scan and the 4096-chunk stage 1), the long-context secondary's two (the 16-column scan and
    the 16384-chunk stage 1) and the KDA secondary's two; None for anything else (the other
    secondaries, the calibration copies)."""
    W, L = WORKLOAD, LONG_WORKLOAD
    M = W["B"] * W["H"] * W["T"] // W["C"]
    ML = L["B"] * L["H"] * L["T"] // L["C"]
    if "scan_split_kernel<64, 128, 128, 2," in name:
        return "scan_output"
    if "scan_split_kernel<64, 128, 128, 1," in name:
        return "long_scan_output"
    bf16 = "DF16b" in name or "bf16" in name          # __bf16 as the demangler spells it
    if "chunk_local_kernel" in name and bf16 and grid == M * 256:
        return "chunk_local"
    if "chunk_local_kernel" in name and bf16 and grid == ML * 256:
        return "long_chunk_local"
    for k in ("kda_scan", "kda_local"):
        if k in name:
            return k
    return None


def summarize_counters(fetch_db, write_db, lib_hash, copy_mib, out=None):
    """Write the counter record bench.py reads (``COUNTERS``) from two rocprofv3 --pmc runs of
    ``bench.py --calibrate-copy MIB`` (FETCH_SIZE, then WRITE_SIZE): mean KiB per dispatch of each
    kernel, the factor that maps a plain copy's counter reading to its true bytes, and the model
    bytes of the headline kernels, tagged with the library's source hash."""
    import sqlite3
    import statistics
    per, copy = {}, {}
    for counter, db in (("FETCH_SIZE", fetch_db), ("WRITE_SIZE", write_db)):
        con = sqlite3.connect(db)
        rows = con.execute("select kernel_name, grid_size, value from counters_collection "
                           "where counter_name=?", (counter,)).fetchall()
        con.close()
        vals = {}
        for name, grid, v in rows:
            if "copyBuffer" in name:
                copy.setdefault(counter, []).append(v)
                continue
            key = _counter_key(name, grid)
            if key is not None:
                vals.setdefault(key, []).append(v)
        for key, v in vals.items():
            per.setdefault(key, {})[counter] = round(statistics.mean(v), 2)
            per[key]["dispatches"] = len(v)
    # the largest copies are the calibration ones (torch's own small copies read far less)
    copy_kib = max(copy["FETCH_SIZE"]), max(copy["WRITE_SIZE"])
    calib = copy_mib * 1024
    model = stage_model(**{k: WORKLOAD[k] for k in ("B", "H", "T", "C", "DK", "DV")}, esize=2)
    kda = kda_model(**KDA_WORKLOAD)
    model_bytes = {k: model[k]["bytes"] for k in model if k in per}
    lmodel = stage_model(**{k: LONG_WORKLOAD[k] for k in ("B", "H", "T", "C", "DK", "DV")},
                         esize=2)
    h0_bytes = LONG_WORKLOAD["B"] * LONG_WORKLOAD["H"] * LONG_WORKLOAD["DK"] * LONG_WORKLOAD["DV"] * 4
    for k in ("chunk_local", "scan_output"):
        if "long_" + k in per:
            model_bytes["long_" + k] = lmodel[k]["bytes"] + (h0_bytes if k == "scan_output" else 0)
    model_bytes.update({k: kda[k] for k in ("kda_local", "kda_scan") if k in per})
    rec = {"workload": "GDN forward B4 H16 T4096 C64 dk=dv=128, bf16 in (bench.py headline); "
                       "long-context GDN B1 H32 T32768 with h0 (long_*: bench.py "
                       "gdn_config4_long_context); KDA forward B2 H32 T8192 (bench.py kda_config5)",
           "source_hash": lib_hash,
           "commands": [f"rocprofv3 --pmc {c} -d <dir> -o <name> -- python bench.py --steps 3 "
                        f"--warmup 1 --no-cpu-baseline --event-steps 1 --calibrate-copy {copy_mib}"
                        for c in ("FETCH_SIZE", "WRITE_SIZE")],
           "scale": {"FETCH_SIZE": round(calib / copy_kib[0], 5),
                     "WRITE_SIZE": round(calib / copy_kib[1], 5)},
           "calibration": {"copy_bytes": calib * 1024, "FETCH_SIZE": copy_kib[0],
                           "WRITE_SIZE": copy_kib[1]},
           "kernels": {k: {c: v[c] for c in ("FETCH_SIZE", "WRITE_SIZE")} for k, v in per.items()},
           "model_bytes": model_bytes,
           "dispatches_averaged": min(v["dispatches"] for v in per.values())}
    with open(out or COUNTERS, "w") as f:
        json.dump(rec, f, indent=1)
    return rec


def compulsory_bytes(B, H, T, DK, DV, esize, h0=False, g_channels=1):
    """What any forward must move: q, k, v (esize bytes each) + beta and g (fp32; g has
    g_channels values per token) in, o (fp32) and the final state (fp32) out, h0 if given."""
    n = B * H * T
    state = B * H * DK * DV * 4
    return (n * (2 * DK + DV) * esize + n * 4 * (1 + g_channels) + n * DV * 4 + state
            + (state if h0 else 0))


def stage_model(B, H, T, C, DK, DV, esize):
    """Algorithmic flops and HBM bytes per launch of the two kernels.

    Unit = one (b,h) chunk of C tokens; a launch processes M = B*H*T/C units.  For bf16 operands
    the scan forms the causal score P from the q and k rows it stages, so P never goes through
    HBM; the fp32 path writes P in stage 1 and reads it in stage 2.
      stage 1 (chunk-local): reads k (C*DK*e; fp32 also q) + g, beta (2*C*4); writes T without
               the upper-right quadrant no kernel reads ((C*C - (C/2)^2)*e), G (C*4) and, fp32
               only, P (its lower blocks and the (0,1), (2,3) zero blocks the scan reads).
               flops: k k^T (2*C*C*DK), fp32 also q k^T, + the inverse (C^3/3).
      stage 2 (scan+output): reads q, k, v (2*C*DK*e + C*DV*e), T (C*C*e: the unread quadrant
               shares its 128-byte lines with the rows' read halves) and, fp32 only, P, G, beta
               (2*C*4); writes o (C*DV*4); plus the final state (DK*DV*4) once per chain.
               flops: k S, q S, k^T v_new (3 * 2*C*DK*DV) + T r, P v_new (2 * 2*C*C*DV), bf16
               also the score q k^T (2*C*C*DK).
    """
    M = B * H * (T // C)
    score_in_scan = esize == 2
    p_blocks = (C // 16) * (C // 16 + 1) // 2 + 2           # lower blocks + (0,1), (2,3)
    t_tile = C * C - (C // 2) ** 2                          # T elements any kernel reads
    s1_bytes = (1 if score_in_scan else 2) * C * DK * esize + 2 * C * 4 + t_tile * esize + C * 4
    s1_flops = (1 if score_in_scan else 2) * (2 * C * C * DK) + C ** 3 / 3
    s2_bytes = (2 * C * DK + C * DV) * esize + C * C * esize + 2 * C * 4 + C * DV * 4
    s2_flops = 3 * (2 * C * DK * DV) + 2 * (2 * C * C * DV)
    if score_in_scan:
        s2_flops += 2 * C * C * DK
    else:
        s1_bytes += p_blocks * 256 * esize
        s2_bytes += C * C * esize
    return {
        "chunk_local": {"units": M, "bytes_per_unit": s1_bytes, "flops_per_unit": s1_flops,
                        "bytes": M * s1_bytes, "flops": M * s1_flops},
        "scan_output": {"units": M, "bytes_per_unit": s2_bytes, "flops_per_unit": s2_flops,
                        "bytes": M * s2_bytes + B * H * DK * DV * 4, "flops": M * s2_flops},
    }


def cpu_baseline(runs: int = 5, timeout: float = 600.0):
    """The CPU oracle timed on this host's cores (oracle/cpu_baseline.py, run as a child process
    so that its worker pool forks from a process that has not initialised the GPU)."""
    cmd = [sys.executable, "-m", "oracle.cpu_baseline", "--B", str(WORKLOAD["B"]),
           "--H", str(WORKLOAD["H"]), "--T", str(WORKLOAD["T"]), "--C", str(WORKLOAD["C"]),
           "--runs", str(runs)]
    r = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError(f"cpu baseline failed ({r.returncode}):\n{r.stderr[-2000:]}")
    return json.loads(r.stdout.strip().splitlines()[-1])


KDA_WORKLOAD = dict(B=2, H=32, T=8192, C=64, DK=128, DV=128)
LONG_WORKLOAD = dict(B=1, H=32, T=32768, C=64, DK=128, DV=128)


def kda_model(B, H, T, C, DK, DV):
    """Algorithmic HBM bytes of the fused KDA forward per chunk of C tokens (bf16 operands):
    stage 1 reads q, k (bf16), g (fp32 per channel), beta and writes W, QE, KB (bf16),
    T diag(beta) (bf16, C x C), the chunk decay (fp32); stage 2 reads W, QE, KB, T diag(beta), v,
    the decay and writes o (fp32) (the causal score is formed on the chip).  ``compulsory`` is
    what any forward must move: q, k, v, g, beta in, o out."""
    M = B * H * (T // C)
    s1 = 2 * C * DK * 2 + C * DK * 4 + C * 4 + 3 * C * DK * 2 + C * C * 2 + DK * 4
    s2 = 3 * C * DK * 2 + C * C * 2 + C * DV * 2 + DK * 4 + C * DV * 4
    final = B * H * DK * DV * 4
    compulsory = M * (3 * C * DK * 2 + C * DK * 4 + C * 4 + C * DV * 4) + final
    return {"units": M, "bytes_per_unit": s1 + s2, "bytes": M * (s1 + s2) + final,
            "compulsory_bytes": compulsory, "kda_local": M * s1, "kda_scan": M * s2 + final}


def _event_ms(run, steps: int, warmup: int) -> float:
    """Time per call of ``run`` over ``steps`` back-to-back calls on the current stream, after
    warmup: one HIP event pair brackets the whole loop (an event record between calls would add
    its own few microseconds to every call)."""
    import torch
    for _ in range(warmup):
        run()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def device_copy_GBps(mib: int = 256, reps: int = 20) -> float:
    """HBM rate of a plain device-to-device copy of `mib` MiB (bytes read + written per second),
    timed like the secondary records: a practical ceiling to read the kernels' figures against."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, device="cuda:0", dtype=torch.float32)
    dst = torch.empty_like(src)
    ms = _event_ms(lambda: dst.copy_(src), reps, 3)
    return 2 * n * 4 / (ms * 1e-3) / 1e9


def gdn_config_secondary(B, H, T, dtype_name, h0_std, steps, warmup, kind="gdn"):
    """The fused forward at another configuration (GDN long context with h0; fp32 DeltaNet)."""
    import torch
    from pto_fuser_amd.forwards import make_delta_inputs
    from pto_fuser_amd.ops import gdn_chunk_forward, gdn_workspace
    dev = torch.device("cuda:0")
    C, DK, DV = 64, 128, 128
    dtype = torch.bfloat16 if dtype_name == "bf16" else torch.float32
    esize = 2 if dtype_name == "bf16" else 4
    d = make_delta_inputs(B, H, T, DK, DV, kind=kind, dtype=dtype, seed=4, h0_std=h0_std,
                          device=dev)
    o = torch.empty(B, H, T, DV, device=dev, dtype=torch.float32)
    hf = torch.empty(B, H, DK, DV, device=dev, dtype=torch.float32)
    ws = gdn_workspace(B, H, T, C, DK, DV, dtype, dev)
    ms = _event_ms(lambda: gdn_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], h0=d["h0"],
                                             out=o, final_out=hf, workspace=ws), steps, warmup)
    m = stage_model(B, H, T, C, DK, DV, esize)
    nbytes = m["chunk_local"]["bytes"] + m["scan_output"]["bytes"] + (
        B * H * DK * DV * 4 if h0_std is not None else 0)
    if kind == "deltanet":      # no gate to read in stage 1 (stage 2 still reads the zero G)
        nbytes -= B * H * T * 4
    comp = compulsory_bytes(B, H, T, DK, DV, esize, h0=h0_std is not None,
                            g_channels=0 if kind == "deltanet" else 1)
    flops = m["chunk_local"]["flops"] + m["scan_output"]["flops"]
    s = ms * 1e-3
    return {"workload": f"{'DeltaNet' if kind == 'deltanet' else 'GDN'} chunked forward B{B} H{H} "
                        f"T{T} C64 dk128 dv128, {dtype_name} in"
                        f"{', h0' if h0_std is not None else ''}, fp32 state/accum/o",
            "B": B, "H": H, "T": T, "dtype": dtype_name, "ms_per_step": round(ms, 5),
            "tokens_per_s": round(B * T / s, 1), "chains": B * H,
            "chunks_per_chain": T // C, "bytes": nbytes,
            "hbm_frac": round(nbytes / s / PEAK_HBM, 4),
            "compulsory_bytes": comp, "compulsory_hbm_frac": round(comp / s / PEAK_HBM, 4),
            "mfma_frac": round(flops / s / (PEAK_BF16 if dtype_name == "bf16" else PEAK_FP32), 4)}


def kkt_inverse_secondary(steps, warmup):
    """fp32 gated kkt + (I + A)^-1 over 4096 independent 64-token chunks (returns T only)."""
    import torch
    from pto_fuser_amd.forwards import make_delta_inputs
    from pto_fuser_amd.ops import kkt_inverse
    dev = torch.device("cuda:0")
    M, C, D = 4096, 64, 128
    d = make_delta_inputs(1, 1, M * C, D, D, kind="gdn", dtype=torch.float32, seed=3, device=dev)
    k, g, beta = d["k"].reshape(M * C, D), d["g"].reshape(-1), d["beta"].reshape(-1)
    ms = _event_ms(lambda: kkt_inverse(k, g, beta), steps, warmup)
    nbytes = M * (C * D * 4 + 2 * C * 4 + C * C * 4)      # k, g, beta in; T out
    flops = M * (2 * C * C * D + C ** 3 / 3)
    return {"workload": "gated kkt + unit-lower inverse, fp32, 4096 chunks C64 dk128 (T out)",
            "M": M, "ms_per_step": round(ms, 5), "chunks_per_s": round(M / (ms * 1e-3), 1),
            "bytes": nbytes, "hbm_frac": round(nbytes / (ms * 1e-3) / PEAK_HBM, 4),
            "mfma_fp32_frac": round(flops / (ms * 1e-3) / PEAK_FP32, 4)}


def kda_secondary(steps: int, warmup: int):
    """Fused KDA forward at KDA_WORKLOAD, timed like the other secondary records."""
    import torch
    from pto_fuser_amd.forwards import make_delta_inputs
    from pto_fuser_amd.ops import kda_chunk_forward, kda_workspace
    dev = torch.device("cuda:0")
    B, H, T, C, DK, DV = (KDA_WORKLOAD[k] for k in ("B", "H", "T", "C", "DK", "DV"))
    d = make_delta_inputs(B, H, T, DK, DV, kind="kda", dtype=torch.bfloat16, seed=5, device=dev)
    o = torch.empty(B, H, T, DV, device=dev, dtype=torch.float32)
    hf = torch.empty(B, H, DK, DV, device=dev, dtype=torch.float32)
    ws = kda_workspace(B, H, T, C, DK, DV, torch.bfloat16, dev)
    run = lambda: kda_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], out=o,  # noqa: E731
                                    final_out=hf, workspace=ws)
    ms = _event_ms(run, steps, warmup)
    m = kda_model(B, H, T, C, DK, DV)
    return {"workload": "KDA chunked forward B2 H32 T8192 C64 dk128 dv128, per-channel decay, "
                        "bf16 in, fp32 state/accum/o", **KDA_WORKLOAD,
            "ms_per_step": round(ms, 5), "tokens_per_s": round(B * T / (ms * 1e-3), 1),
            "kernels": ["kda_local", "kda_scan"], "bytes": m["bytes"],
            "bytes_per_unit": m["bytes_per_unit"], "units": m["units"],
            "hbm_frac": round(m["bytes"] / (ms * 1e-3) / PEAK_HBM, 4),
            "compulsory_bytes": m["compulsory_bytes"],
            "compulsory_hbm_frac": round(m["compulsory_bytes"] / (ms * 1e-3) / PEAK_HBM, 4)}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--event-steps", type=int, default=50,
                    help="forwards (and stage-1 launches) timed after the timed loop for the "
                         "per-kernel durations")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-runs", type=int, default=5)
    ap.add_argument("--no-secondary", action="store_true", help="skip the secondary records")
    ap.add_argument("--summarize-counters", nargs=2, metavar=("FETCH_DB", "WRITE_DB"),
                    help="write the counter record from two rocprofv3 --pmc result databases "
                         "(FETCH_SIZE, WRITE_SIZE) of a --calibrate-copy run, then exit")
    ap.add_argument("--summarize-trace", metavar="TRACE_CSV",
                    help="write the kernel-trace record from a rocprofv3 kernel_trace.csv, then exit")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="after the timed steps, run three plain device copies of MIB MiB: the "
                         "known-size kernel that scales the FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args(argv)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}): this "
              f"build has no multi-GPU path; the forward shards over (b,h) chains with no "
              f"communication, so per-GPU throughput at N GPUs is the N=1 figure.",
              file=sys.stderr)
        return 2
    if args.summarize_trace:
        from pto_fuser_amd import _build
        rec = summarize_trace(args.summarize_trace, _build.source_hash())
        print(json.dumps(rec["kernels"]))
        return 0
    if args.summarize_counters:
        from pto_fuser_amd import _build
        rec = summarize_counters(*args.summarize_counters, _build.source_hash(),
                                 args.calibrate_copy or 256)
        print(json.dumps({k: rec[k] for k in ("source_hash", "scale", "kernels", "model_bytes")}))
        return 0

    # the CPU baseline first: its child process forks workers, which must not inherit a GPU context
    cpu = None if args.no_cpu_baseline else cpu_baseline(runs=args.cpu_runs)

    import torch
    from pto_fuser_amd import _hip
    from pto_fuser_amd.forwards import make_delta_inputs
    from pto_fuser_amd.ops import gdn_workspace

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, H, T, C, DK, DV = (WORKLOAD[k] for k in ("B", "H", "T", "C", "DK", "DV"))
    dtype = torch.bfloat16
    d = make_delta_inputs(B, H, T, DK, DV, kind="gdn", dtype=dtype, seed=0, device=dev)
    o = torch.empty(B, H, T, DV, device=dev, dtype=torch.float32)
    hf = torch.empty(B, H, DK, DV, device=dev, dtype=torch.float32)
    ws = gdn_workspace(B, H, T, C, DK, DV, dtype, dev)
    lib = _hip.load()
    lib_hash = lib.pf_source_hash().decode()
    code = _hip.PF_DTYPE_BF16
    scale = DK ** -0.5
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    P = {n: _hip.ptr(t) for n, t in d.items()}

    def stage1():
        st = lib.pf_gdn_chunk_local_exec(P["q"], P["k"], P["beta"], P["g"], B, H, T, C, DK, DV,
                                         code, scale, ws.handle, sh)
        if st:
            _hip.check("pf_gdn_chunk_local_exec", st)

    def stage2():
        st = lib.pf_gdn_scan_output_exec(P["q"], P["k"], P["v"], P["beta"], None, _hip.ptr(o),
                                         _hip.ptr(hf), B, H, T, C, DK, DV, code, ws.handle, sh)
        if st:
            _hip.check("pf_gdn_scan_output_exec", st)

    def step():
        stage1()
        stage2()

    copy_GBps = device_copy_GBps()
    # settle: keep the GPU busy with untimed forwards for SETTLE_S seconds before the W warmup
    # steps, so that a short timed loop runs at the clocks a long one reaches (without it, 20
    # steps measured up to 15 % slower than 200, the GPU still ramping its clocks)
    t_settle = time.perf_counter()
    while time.perf_counter() - t_settle < SETTLE_S:
        for _ in range(50):
            step()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # the timed loop: one event pair on the launch stream brackets the K steps, one trailing sync
    e_start, e_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e_start.record(stream)
    for _ in range(args.steps):
        step()
    e_end.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e_start.elapsed_time(e_end) / args.steps
    # the same loop repeated REPEATS more times (reported beside the timed loop, not in `value`)
    repeat_ms = [_event_ms(step, args.steps, 0) for _ in range(REPEATS)]

    # per-kernel durations, after the timed loop: ``--event-steps`` forwards and as many stage-1
    # launches, each run back to back under one event pair on the launch stream.  Stage 1's
    # duration is its own loop's average; stage 2's is the forward's average minus stage 1's,
    # i.e. its share of a forward as the timed loop runs it (an event between the two kernels
    # would add a few microseconds to each, and stage 2 repeated alone reads a colder T).
    n_ev = max(1, args.event_steps)
    fwd_ms = _event_ms(step, n_ev, 2)
    k1_ms = _event_ms(stage1, n_ev, 2)
    k2_ms = fwd_ms - k1_ms

    model = stage_model(B, H, T, C, DK, DV, esize=2)
    comp = compulsory_bytes(B, H, T, DK, DV, esize=2)
    stages = {}
    for name, ms in (("chunk_local", k1_ms), ("scan_output", k2_ms)):
        m = model[name]
        sec = ms * 1e-3
        stages[name] = {
            "avg_ms": round(ms, 5), "bytes": m["bytes"], "flops": m["flops"],
            "bytes_per_unit": m["bytes_per_unit"], "flops_per_unit": m["flops_per_unit"],
            "units": m["units"],
            "hbm_GBps": round(m["bytes"] / sec / 1e9, 1),
            "hbm_frac": round(m["bytes"] / sec / PEAK_HBM, 4),
            "mfma_TFLOPs": round(m["flops"] / sec / 1e12, 2),
            "mfma_bf16_frac": round(m["flops"] / sec / PEAK_BF16, 4),
            "traffic": measured_traffic(name, lib_hash),
        }
    ds = stages["scan_output"]
    k2 = k2_ms * 1e-3
    k2_trace_ms = traced_kernel_ms("scan_output", lib_hash)
    roofline = {"kernel": "scan_output", "bound": "hbm",
                "achieved": round(comp / k2 / 1e9, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                "frac": round(comp / k2 / PEAK_HBM, 4), "traffic": ds["traffic"],
                "bytes": comp, "bytes_per_unit": comp // model["scan_output"]["units"],
                "units": model["scan_output"]["units"], "kernel_avg_ms": round(k2_ms, 5),
                "own_bytes": ds["bytes"], "own_achieved": ds["hbm_GBps"],
                "own_frac": ds["hbm_frac"],
                "device_copy_GBps": round(copy_GBps, 1),
                "frac_of_device_copy": round(comp / k2 / 1e9 / copy_GBps, 4),
                # the same kernel's average in the recorded rocprofv3 kernel trace
                # (profiles/kernel_trace_gdn_forward.json, same source hash), and the fraction
                # recomputed from it
                "kernel_avg_ms_rocprof": None if k2_trace_ms is None else round(k2_trace_ms, 5),
                "frac_rocprof": None if k2_trace_ms is None else
                round(comp / (k2_trace_ms * 1e-3) / PEAK_HBM, 4),
                "source_hash": lib_hash}
    total_bytes = sum(model[n]["bytes"] for n in model)
    total_flops = sum(model[n]["flops"] for n in model)
    fs = ms_per_step * 1e-3

    line = {
        "metric": METRIC,
        "value": round(B * T / fs, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_s": SETTLE_S,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded Gaussian q/k/v, sigmoid beta, -softplus*0.1 log-decay)",
        "config": {"workload": "GDN chunked forward B4 H16 T4096 C64 dk128 dv128, bf16 in, "
                               "fp32 state/accum/o", **WORKLOAD},
        "roofline": roofline,
        "stages": stages,
        "forward": {"compulsory_bytes": comp, "hbm_frac": round(comp / fs / PEAK_HBM, 4),
                    "own_bytes": total_bytes, "own_hbm_frac": round(total_bytes / fs / PEAK_HBM, 4),
                    "flops": total_flops,
                    "mfma_bf16_frac": round(total_flops / fs / PEAK_BF16, 4),
                    "event_steps": args.event_steps,
                    "repeats_ms_per_step": [round(x, 5) for x in repeat_ms],
                    "repeats_median_ms": round(statistics.median(repeat_ms), 5)},
    }
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        line["calibration_copy_bytes"] = n * 4
    if not args.no_secondary:
        sec_steps, sec_warm = max(1, min(args.steps, 50)), min(max(args.warmup, 5), 10)
        line["secondary"] = {
            "kda_config5": kda_secondary(sec_steps, sec_warm),
            "gdn_config4_long_context": gdn_config_secondary(
                LONG_WORKLOAD["B"], LONG_WORKLOAD["H"], LONG_WORKLOAD["T"], "bf16", 0.02,
                sec_steps, sec_warm),
            "kkt_inverse_config3": kkt_inverse_secondary(sec_steps, sec_warm),
            "deltanet_config1": gdn_config_secondary(1, 4, 512, "fp32", None, sec_steps,
                                                     sec_warm, kind="deltanet"),
        }
    if cpu is not None:
        line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
