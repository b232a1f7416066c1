"""bench.py's host-side pieces on the CPU: the algorithmic byte / flop models behind `roofline`,
the recorded counter traffic, and the one-GPU contract (--gpus N > 1 exits with a message)."""
import subprocess
import sys

import pytest

import bench

C, DK, DV = 64, 128, 128


def test_stage_model_per_chunk_bytes_and_flops():
    m = bench.stage_model(4, 16, 4096, C, DK, DV, 2)
    s1, s2 = m["chunk_local"], m["scan_output"]
    assert s1["units"] == s2["units"] == 4 * 16 * 64
    # stage 1: k, q (bf16) + g, beta in; T without its upper-right quadrant and 12 P blocks
    # (bf16), G out
    tp = C * C - 32 * 32
    assert s1["bytes_per_unit"] == 2 * C * DK * 2 + 2 * C * 4 + tp * 2 + 12 * 16 * 16 * 2 + C * 4
    # stage 2: q, k, v, T, P (bf16, whole 128-byte rows) + G, beta in; o (fp32) out; plus the
    # final state per chain
    assert s2["bytes_per_unit"] == (2 * C * DK + C * DV) * 2 + 2 * C * C * 2 + 2 * C * 4 + C * DV * 4 == 98816
    assert s2["bytes"] == 4096 * 98816 + 64 * DK * DV * 4
    # flops per chunk: kk^T + qk^T + inverse; kS, qS, k^T v_new + T r, P v_new
    assert s1["flops_per_unit"] == pytest.approx(4 * C * C * DK + C ** 3 / 3)
    assert s2["flops_per_unit"] == 6 * C * DK * DV + 4 * C * C * DV
    # fp32 operands double the operand bytes, not the fp32 gate / output bytes
    f = bench.stage_model(1, 1, 64, C, DK, DV, 4)
    assert f["scan_output"]["bytes_per_unit"] - s2["bytes_per_unit"] == (2 * C * DK + C * DV + 2 * C * C) * 2


def test_measured_traffic_matches_the_byte_model():
    """The counter figures recorded in bench.py (FETCH x2, WRITE x1) agree with the algorithmic
    bytes of the headline launch to within 0.2 %: neither kernel re-reads."""
    m = bench.stage_model(4, 16, 4096, C, DK, DV, 2)
    for k in ("chunk_local", "scan_output"):
        traffic = bench.measured_traffic(k)
        assert traffic is not None
        assert abs(traffic / m[k]["bytes"] - 1) < 2e-3, (k, traffic, m[k]["bytes"])
    assert bench.measured_traffic("no_such_kernel") is None


def test_kda_model():
    m = bench.kda_model(2, 32, 8192, C, DK, DV)
    assert m["units"] == 2 * 32 * 128
    s1 = 3 * C * DK * 2 + C * DK * 4 + C * 4 + 4 * C * DK * 2 + 12 * 256 * 2 + DK * 4
    s2 = 4 * C * DK * 2 + C * C * 2 + DK * 4 + C * DV * 4
    assert m["bytes_per_unit"] == s1 + s2
    # compulsory: q, k, v, g, beta in and o out, plus the final state
    assert m["compulsory_bytes"] == m["units"] * (3 * C * DK * 2 + C * DK * 4 + C * 4 + C * DV * 4) \
        + 2 * 32 * DK * DV * 4
    assert m["compulsory_bytes"] < m["bytes"]


def test_multi_gpu_request_exits_with_message():
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True, text=True,
                       cwd=bench.ROOT, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""
