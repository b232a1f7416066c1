"""bench.py's host-side pieces on the CPU: the algorithmic byte / flop models behind `roofline`,
the recorded counter traffic, the CPU baseline child and the one-GPU contract (--gpus N > 1 exits
with a message)."""
import json
import subprocess
import sys

import pytest

import bench

C, DK, DV = 64, 128, 128


def test_stage_model_per_chunk_bytes_and_flops():
    m = bench.stage_model(4, 16, 4096, C, DK, DV, 2)
    s1, s2 = m["chunk_local"], m["scan_output"]
    assert s1["units"] == s2["units"] == 4 * 16 * 64
    # stage 1 (bf16): k + g, beta in; T without its upper-right quadrant (bf16) and G out
    t = C * C - 32 * 32
    assert s1["bytes_per_unit"] == C * DK * 2 + 2 * C * 4 + t * 2 + C * 4
    # stage 2 (bf16): q, k, v, T (bf16, whole 128-byte rows) + G, beta in; o (fp32) out; plus the
    # final state per chain.  P is formed on the chip.
    assert s2["bytes_per_unit"] == (2 * C * DK + C * DV) * 2 + C * C * 2 + 2 * C * 4 + C * DV * 4 == 90624
    assert s2["bytes"] == 4096 * 90624 + 64 * DK * DV * 4
    # flops per chunk: kk^T + inverse; kS, qS, k^T v_new + T r, P v_new + the score qk^T
    assert s1["flops_per_unit"] == pytest.approx(2 * C * C * DK + C ** 3 / 3)
    assert s2["flops_per_unit"] == 6 * C * DK * DV + 4 * C * C * DV + 2 * C * C * DK
    # fp32 operands double the operand bytes, and P goes through HBM (12 blocks written, read
    # as whole rows)
    f = bench.stage_model(1, 1, 64, C, DK, DV, 4)
    assert f["scan_output"]["bytes_per_unit"] - s2["bytes_per_unit"] == \
        (2 * C * DK + C * DV + C * C) * 2 + C * C * 4
    assert f["chunk_local"]["bytes_per_unit"] == 2 * C * DK * 4 + 2 * C * 4 + t * 4 + 12 * 256 * 4 + C * 4


def test_compulsory_bytes_of_the_headline():
    """q, k, v bf16 + beta, g fp32 in; o fp32 and the final state out: 341.8 MB, i.e. 83 456 B per
    64-token chunk (82 432 B of token data + 1/64 of the chain's 64 KiB final state)."""
    comp = bench.compulsory_bytes(4, 16, 4096, DK, DV, 2)
    assert comp == 341_835_776
    assert comp == 4096 * (3 * C * 128 * 2 + 2 * C * 4 + C * DV * 4) + 64 * DK * DV * 4
    assert bench.compulsory_bytes(1, 32, 32768, DK, DV, 2, h0=True) == 1_354_760_192
    # KDA: g holds DK values per token
    assert bench.compulsory_bytes(2, 32, 8192, DK, DV, 2, g_channels=DK) == \
        bench.kda_model(2, 32, 8192, C, DK, DV)["compulsory_bytes"]


def test_measured_traffic_keyed_to_the_source_hash(tmp_path, monkeypatch):
    """Counter traffic is the recorded FETCH_SIZE / WRITE_SIZE KiB scaled by the copy factors, and
    only for the build it was recorded from: another source hash gives None."""
    rec = {"source_hash": "abc", "scale": {"FETCH_SIZE": 2.0, "WRITE_SIZE": 1.0},
           "kernels": {"scan_output": {"FETCH_SIZE": 100.0, "WRITE_SIZE": 50.0}}}
    path = tmp_path / "c.json"
    path.write_text(json.dumps(rec))
    monkeypatch.setattr(bench, "COUNTERS", str(path))
    assert bench.measured_traffic("scan_output", "abc") == (200 + 50) * 1024
    assert bench.measured_traffic("scan_output", "def") is None
    assert bench.measured_traffic("no_such_kernel", "abc") is None
    monkeypatch.setattr(bench, "COUNTERS", str(tmp_path / "missing.json"))
    assert bench.measured_traffic("scan_output", "abc") is None


def test_recorded_counters_match_the_byte_model():
    """The committed counter record (whatever build it belongs to) agrees with the algorithmic
    bytes of its kernels: reads to within 0.5 % (no kernel re-reads), and so do the writes of
    every kernel but the scans.  The scans store o non-temporally, a 64-byte half of a 128-byte
    line per instruction, and a line whose halves reach memory separately is counted twice: their
    writes may run up to 15 % over o and the final state."""
    with open(bench.COUNTERS) as f:
        rec = json.load(f)
    m = bench.stage_model(4, 16, 4096, C, DK, DV, 2)
    scans = {"scan_output": bench.WORKLOAD, "long_scan_output": bench.LONG_WORKLOAD}
    for k, kib in rec["kernels"].items():
        traffic = sum(kib[c] * rec["scale"][c] * 1024 for c in ("FETCH_SIZE", "WRITE_SIZE"))
        if k in scans:
            L = scans[k]
            o_final = L["B"] * L["H"] * (L["T"] * L["DV"] + L["DK"] * L["DV"]) * 4
            writes = kib["WRITE_SIZE"] * rec["scale"]["WRITE_SIZE"] * 1024
            reads = traffic - writes
            assert abs(reads / (rec["model_bytes"][k] - o_final) - 1) < 5e-3, (k, reads)
            assert 0 <= writes / o_final - 1 < 0.15, (k, writes)
        else:
            assert abs(traffic / rec["model_bytes"][k] - 1) < 5e-3, (k, traffic)
        if k in m:
            assert rec["model_bytes"][k] == m[k]["bytes"], k


def test_cpu_baseline_child_reports_cores():
    r = subprocess.run([sys.executable, "-m", "oracle.cpu_baseline", "--B", "1", "--H", "2",
                        "--T", "128", "--runs", "1", "--workers", "2"], capture_output=True,
                       text=True, cwd=bench.ROOT, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    d = json.loads(r.stdout.strip().splitlines()[-1])
    assert d["cores"] == 2 and d["kind"] == "port" and d["unit"] == "tokens/s"
    assert d["value"] > 0 and d["single_core_value"] > 0 and d["host_cpus"] >= 1


def test_kda_model():
    m = bench.kda_model(2, 32, 8192, C, DK, DV)
    assert m["units"] == 2 * 32 * 128
    # stage 1: q, k, g, beta in; W, QE, KB, T diag(beta), the decay out
    s1 = 2 * C * DK * 2 + C * DK * 4 + C * 4 + 3 * C * DK * 2 + C * C * 2 + DK * 4
    # stage 2: W, QE, KB, T diag(beta), v, the decay in; o out (the causal score stays on the chip)
    s2 = 3 * C * DK * 2 + C * C * 2 + C * DV * 2 + DK * 4 + C * DV * 4
    assert m["bytes_per_unit"] == s1 + s2 == 230656
    # compulsory: q, k, v, g, beta in and o out, plus the final state
    assert m["compulsory_bytes"] == m["units"] * (3 * C * DK * 2 + C * DK * 4 + C * 4 + C * DV * 4) \
        + 2 * 32 * DK * DV * 4
    assert m["compulsory_bytes"] < m["bytes"]


def test_multi_gpu_request_exits_with_message():
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True, text=True,
                       cwd=bench.ROOT, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_trace_record_roundtrip(tmp_path, monkeypatch):
    """--summarize-trace groups a kernel_trace.csv by the counter keys (kernel name and grid) and
    tags the record with the source hash; bench reads the stage-2 average back only for that
    hash."""
    M = 4 * 16 * 64
    rows = [("void pf::scan_split_kernel<64, 128, 128, 2, 4>(pf::ScanOutArgs)", 256 * 512, 1000, 91000),
            ("void pf::scan_split_kernel<64, 128, 128, 2, 4>(pf::ScanOutArgs)", 256 * 512, 2000, 91000),
            ("void pf::chunk_local_kernel<__bf16, __bf16, 64, 128, false, true>(pf::ChunkLocalArgs)",
             M * 256, 0, 21000),
            ("void at::native::copy_kernel(...)", 1 << 20, 0, 5000)]
    csv_path = tmp_path / "kt_kernel_trace.csv"
    with open(csv_path, "w") as f:
        f.write('"Kernel_Name","Grid_Size","Start_Timestamp","End_Timestamp"\n')
        for name, grid, t0, t1 in rows:
            f.write(f'"{name}",{grid},{t0},{t1}\n')
    out = tmp_path / "trace.json"
    monkeypatch.setattr(bench, "TRACE", str(out))
    rec = bench.summarize_trace(str(csv_path), "abc123")
    assert rec["kernels"]["scan_output"]["dispatches"] == 2
    assert rec["kernels"]["scan_output"]["avg_us"] == pytest.approx(89.5)
    assert rec["kernels"]["chunk_local"]["avg_us"] == pytest.approx(21.0)
    assert set(rec["kernels"]) == {"scan_output", "chunk_local"}
    assert bench.traced_kernel_ms("scan_output", "abc123") == pytest.approx(0.0895)
    assert bench.traced_kernel_ms("scan_output", "other") is None
