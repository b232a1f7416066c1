"""GPU parity of the fused KDA forward (per-channel decay) against the oracle.

kda_reference (oracle/gdn_oracle.py, restating examples/attention/_kda_full.py:42-76) consumes
the bf16-rounded inputs upcast to float; the fused path computes in fp32 with bf16 MFMA operands.
Tolerance, as for the other bf16 forwards: max abs err <= 2e-2 against the fp32 oracle on o AND
the final state h; fp32 operands (fp32 MFMA throughout) max rel err <= 1e-4.  Config 5 is the benchmark configuration B2 H32 T8192 with
g = -softplus(N) * 0.05 per channel.
"""
import numpy as np
import pytest
import torch

from conftest import announce, record_error
from oracle.gdn_oracle import kda_reference, max_abs
from pto_fuser_amd import kda_chunk_forward
from pto_fuser_amd.forwards import as_oracle_inputs, make_delta_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BF16_TOL = 2e-2
FP32_TOL = 1e-4


def _run(inp):
    d = {n: (None if t is None else t.to(DEV)) for n, t in inp.items()}
    o, h = kda_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], h0=d["h0"])
    torch.cuda.synchronize()
    return o.cpu().numpy(), h.cpu().numpy()


def _check(case, o, h, o_ref, h_ref):
    for name, got, ref in (("o", o, o_ref), ("h", h, h_ref)):
        e = record_error(case, name, got, ref, f"max abs <= {BF16_TOL}")
        assert e["abs"] <= BF16_TOL, (case, name, e)


def _check_fp32(case, o, h, o_ref, h_ref):
    """fp32 operands: max rel err <= 1e-4 (relative to the reference's largest magnitude)."""
    for name, got, ref in (("o", o, o_ref), ("h", h, h_ref)):
        e = record_error(case, name, got, ref, f"max rel <= {FP32_TOL}")
        assert e["rel"] <= FP32_TOL, (case, name, e)


def _oracle(inp, dtype=np.float64):
    x = as_oracle_inputs(inp)
    return kda_reference(x["q"], x["k"], x["v"], x["beta"], x["g"], C=64, h0=x["h0"], dtype=dtype)


@pytest.mark.parametrize("B,H,T,h0", [(1, 3, 64, True), (2, 2, 64, False), (1, 2, 128, False),
                                      (2, 3, 256, True), (1, 4, 1024, True), (1, 1, 192, False)])
def test_kda_bf16_matches_oracle(B, H, T, h0):
    announce(f"KDA bf16 B{B} H{H} T{T} h0={h0}")
    inp = make_delta_inputs(B, H, T, kind="kda", dtype=torch.bfloat16, seed=B * 31 + H * 7 + T,
                            h0_std=0.02 if h0 else None)
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp)
    _check(f"KDA bf16 B{B} H{H} T{T}{' h0' if h0 else ''}", o, h, o_ref, h_ref)


def test_kda_bf16_strong_decay():
    """Faster per-channel decay (g up to ~ -1 per token): e^-G inside a chunk grows large, the
    form the reference computes (k e^-G) is kept as is."""
    announce("KDA bf16 B1 H2 T512 strong decay")
    inp = make_delta_inputs(1, 2, 512, kind="kda", dtype=torch.bfloat16, seed=11, gate_scale=0.3)
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp)
    _check("KDA bf16 B1 H2 T512 strong decay", o, h, o_ref, h_ref)


@pytest.mark.parametrize("B,H,T", [(8, 64, 128), (7, 37, 64)])
def test_kda_bf16_many_chains(B, H, T):
    """512 and 259 chains (several generations of scan workgroups), with the XCD-aware chain
    mapping (B*H % 8 == 0) and without, with h0."""
    announce(f"KDA bf16 B{B} H{H} T{T} h0 (many chains)")
    inp = make_delta_inputs(B, H, T, kind="kda", dtype=torch.bfloat16, seed=B * 30 + H,
                            h0_std=0.02)
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp)
    _check(f"KDA bf16 B{B} H{H} T{T} h0 (many chains)", o, h, o_ref, h_ref)


def test_kda_bf16_extreme_decay():
    """g up to ~ -4 per token: a channel's within-chunk cumulative log decay reaches -65, so
    e^-G of the key operand reaches ~1e28 and e^G of the query operand ~1e-28 (both still inside
    the fp32 / bf16 exponent range, as in the reference's fp32 factors), with h0."""
    announce("KDA bf16 B1 H2 T256 extreme decay h0")
    inp = make_delta_inputs(1, 2, 256, kind="kda", dtype=torch.bfloat16, seed=13, gate_scale=1.0,
                            h0_std=0.02)
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp)
    _check("KDA bf16 B1 H2 T256 extreme decay h0", o, h, o_ref, h_ref)


def test_kda_bf16_config5():
    announce("KDA bf16 B2 H32 T8192")
    inp = make_delta_inputs(2, 32, 8192, kind="kda", dtype=torch.bfloat16, seed=5)
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp, dtype=np.float32)
    _check("KDA bf16 config 5 B2 H32 T8192", o, h, o_ref, h_ref)


def test_kda_state_passing():
    """Running [0,T) equals running [0,T/2) and then [T/2,T) from the first half's final state."""
    announce("KDA bf16 state passing B1 H4 T1024")
    inp = make_delta_inputs(1, 4, 1024, kind="kda", dtype=torch.bfloat16, seed=13)
    d = {n: (None if t is None else t.to(DEV)) for n, t in inp.items()}
    o, h = kda_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"])
    half = {n: (None if t is None else t[:, :, :512].contiguous()) for n, t in d.items() if n != "h0"}
    rest = {n: (None if t is None else t[:, :, 512:].contiguous()) for n, t in d.items() if n != "h0"}
    o1, h1 = kda_chunk_forward(half["q"], half["k"], half["v"], half["beta"], half["g"])
    o2, h2 = kda_chunk_forward(rest["q"], rest["k"], rest["v"], rest["beta"], rest["g"], h0=h1)
    torch.cuda.synchronize()
    eo = record_error("KDA state passing B1 H4 T1024", "o", torch.cat([o1, o2], 2).cpu().numpy(),
                      o.cpu().numpy(), "max abs <= 1e-3")
    eh = record_error("KDA state passing B1 H4 T1024", "h", h2.cpu().numpy(), h.cpu().numpy(),
                      "max abs <= 1e-3")
    assert eo["abs"] <= 1e-3 and eh["abs"] <= 1e-3, (eo, eh)


def test_kda_deterministic():
    announce("KDA bf16 determinism B2 H4 T1024")
    inp = make_delta_inputs(2, 4, 1024, kind="kda", dtype=torch.bfloat16, seed=17)
    o1, h1 = _run(inp)
    o2, h2 = _run(inp)
    assert np.array_equal(o1, o2) and np.array_equal(h1, h2)


def test_kda_linear_in_v_config5():
    """Size-independent property at config 5's full size: o and the final state are linear in v,
    bit for bit.  Doubling v is exact in bf16, and both KDA kernels only scale by it (U = T(beta
    v) stored in bf16, the fp32 MFMA accumulations, the bf16 packing of the state), each step
    commuting with a factor of two."""
    announce("KDA bf16 linearity in v B2 H32 T8192")
    inp = make_delta_inputs(2, 32, 8192, kind="kda", dtype=torch.bfloat16, seed=5)
    o1, h1 = _run(inp)
    o2, h2 = _run(dict(inp, v=inp["v"] * 2))
    assert np.array_equal(o2, 2 * o1), max_abs(o2, 2 * o1)
    assert np.array_equal(h2, 2 * h1), max_abs(h2, 2 * h1)


@pytest.mark.parametrize("B,H,T,h0", [(1, 2, 64, False), (2, 3, 256, True), (1, 2, 512, True)])
def test_kda_fp32_matches_oracle(B, H, T, h0):
    """fp32 operands through the fp32 kernels (one chunk per sequence included)."""
    announce(f"KDA fp32 B{B} H{H} T{T} h0={h0}")
    inp = make_delta_inputs(B, H, T, kind="kda", dtype=torch.float32, seed=B * 13 + H * 5 + T,
                            h0_std=0.02 if h0 else None)
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp)
    _check_fp32(f"KDA fp32 B{B} H{H} T{T}{' h0' if h0 else ''}", o, h, o_ref, h_ref)


def test_kda_fp32_strong_decay_and_chunk_128():
    """fp32 with faster decay, at C = 128 (run as 64-token chunks: the same result as C = 64,
    bit for bit, and within the fp32 bound of the oracle chunked at 128)."""
    announce("KDA fp32 B1 H2 T512 strong decay C128")
    inp = make_delta_inputs(1, 2, 512, kind="kda", dtype=torch.float32, seed=17, gate_scale=0.3,
                            h0_std=0.02)
    d = {n: (None if t is None else t.to(DEV)) for n, t in inp.items()}
    o128, h128 = kda_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], h0=d["h0"],
                                   chunk_size=128)
    o64, h64 = kda_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], h0=d["h0"])
    torch.cuda.synchronize()
    x = as_oracle_inputs(inp)
    o_ref, h_ref = kda_reference(x["q"], x["k"], x["v"], x["beta"], x["g"], C=128, h0=x["h0"],
                                 dtype=np.float64)
    _check_fp32("KDA fp32 B1 H2 T512 strong decay C128", o128.cpu().numpy(), h128.cpu().numpy(),
                o_ref, h_ref)
    assert torch.equal(o128, o64) and torch.equal(h128, h64)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_kda_without_final_state(dtype):
    """output_final_state=False: no state is written, None is returned, o is bit-identical."""
    announce(f"KDA {dtype} without final state B1 H4 T512")
    inp = make_delta_inputs(1, 4, 512, kind="kda", dtype=dtype, seed=13, h0_std=0.02)
    d = {n: (None if t is None else t.to(DEV)) for n, t in inp.items()}
    o1, h1 = kda_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], h0=d["h0"])
    o2, h2 = kda_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], h0=d["h0"],
                               output_final_state=False)
    torch.cuda.synchronize()
    assert h2 is None and h1 is not None
    assert torch.equal(o1, o2)
