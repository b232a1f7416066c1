"""GPU parity of the fused delta-rule forward and the chunk-local stages against the oracle.

The oracle consumes the dtype-rounded inputs upcast to float64/float32, so the measured error
is the kernel's arithmetic.  Tolerances (stated per test): fp32 inputs max rel err <= 1e-4;
bf16 inputs with fp32 accumulation max abs err <= 2e-2 against the fp32 oracle, on o AND the
final state h.  Config numbers refer to the benchmark configurations (1: DeltaNet fp32 B1 H4
T512; 2: GDN bf16 B4 H16 T4096; 3: kkt + inverse fp32 over 4096 chunks; 4: GDN bf16 B1 H32
T32768 with h0).
"""
import numpy as np
import pytest
import torch

from conftest import announce, record_error
from oracle.gdn_oracle import (deltanet_reference, gdn_reference, max_abs, max_rel,
                               tri_inv_reference, within_chunk_cumsum)
from pto_fuser_amd import gdn_chunk_forward, kkt_inverse, tri_inv
from pto_fuser_amd.forwards import as_oracle_inputs, make_delta_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
FP32_TOL = 1e-4      # max rel err, fp32 path
BF16_TOL = 2e-2      # max abs err, bf16 inputs / fp32 accumulation


def _run(inp):
    d = {n: (None if t is None else t.to(DEV)) for n, t in inp.items()}
    o, h = gdn_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], h0=d["h0"])
    torch.cuda.synchronize()
    return o.cpu().numpy(), h.cpu().numpy()


def _check(case, o, h, o_ref, h_ref, bf16):
    """The bound of the north star: bf16 inputs max abs <= 2e-2, fp32 max rel <= 1e-4, on o and
    the final state; every comparison's magnitudes are recorded for the session summary."""
    tol = f"max abs <= {BF16_TOL}" if bf16 else f"max rel <= {FP32_TOL}"
    for name, got, ref in (("o", o, o_ref), ("h", h, h_ref)):
        e = record_error(case, name, got, ref, tol)
        err = e["abs"] if bf16 else e["rel"]
        assert err <= (BF16_TOL if bf16 else FP32_TOL), (case, name, e)


def _oracle(inp, dtype=np.float64):
    x = as_oracle_inputs(inp)
    g = x["g"] if x["g"] is not None else np.zeros(x["beta"].shape)
    return gdn_reference(x["q"], x["k"], x["v"], x["beta"], g, h0=x["h0"], C=64, dtype=dtype)


@pytest.mark.parametrize("C", [16, 32, 48, 64, 128])
def test_tri_inv_matches_oracle(C):
    announce(f"tri_inv C={C} M=96")
    rng = np.random.default_rng(C)
    A = np.tril(rng.standard_normal((96, C, C)) * 0.1, -1).astype(np.float32)
    A[:, np.arange(C), np.arange(C)] = 5.0                  # diagonal must be ignored
    A += np.triu(np.ones((C, C), np.float32), 1) * 7.0      # so must the upper triangle
    got = tri_inv(torch.from_numpy(A).to(DEV)).cpu().numpy()
    ref = tri_inv_reference(np.tril(A, -1))
    e = record_error(f"tri_inv C={C} M=96", "T", got, ref, f"max rel <= {FP32_TOL}")
    assert e["rel"] <= FP32_TOL, e
    assert np.all(np.triu(got, 1) == 0) and np.all(got[:, np.arange(C), np.arange(C)] == 1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_kkt_inverse_config3(dtype):
    """Config 3: 4096 independent 64x64 blocks, A = I + strict-lower(beta k k^T e^{dG}), inverted."""
    M, C, D = 4096, 64, 128
    announce(f"kkt_inverse M={M} dtype={dtype}")
    inp = make_delta_inputs(1, 1, M * C, D, D, kind="gdn", dtype=dtype, seed=3)
    k = inp["k"].reshape(M * C, D)
    Tm, A = kkt_inverse(k.to(DEV), inp["g"].reshape(-1).to(DEV), inp["beta"].reshape(-1).to(DEV),
                        return_A=True)
    torch.cuda.synchronize()
    x = as_oracle_inputs(inp)
    G = within_chunk_cumsum(x["g"], C).reshape(M, C)
    kk = x["k"].reshape(M, C, D)
    bt = x["beta"].reshape(M, C)
    dG = G[:, :, None] - G[:, None, :]
    A_ref = np.tril(kk @ kk.transpose(0, 2, 1) * np.where(dG <= 0, np.exp(np.minimum(dG, 0)), 0)
                    * bt[:, :, None], -1)
    T_ref = tri_inv_reference(A_ref)
    case = f"kkt+inverse config 3 {str(dtype).replace('torch.', '')}"
    ea = record_error(case, "A", A.cpu().numpy(), A_ref, f"max rel <= {FP32_TOL}")
    et = record_error(case, "T", Tm.cpu().numpy(), T_ref, f"max rel <= {FP32_TOL}")
    assert ea["rel"] <= FP32_TOL and et["rel"] <= FP32_TOL, (ea, et)


def test_deltanet_fp32_config1():
    announce("DeltaNet fp32 B1 H4 T512")
    inp = make_delta_inputs(1, 4, 512, kind="deltanet", dtype=torch.float32, seed=0)
    o, h = _run(inp)
    x = as_oracle_inputs(inp)
    ref = deltanet_reference(x["q"], x["k"], x["v"], x["beta"], C=64, dtype=np.float64)
    _check("DeltaNet fp32 config 1 B1 H4 T512", o, h, ref["o"].reshape(o.shape), ref["final"],
           bf16=False)


@pytest.mark.parametrize("B,H,T", [(1, 2, 64), (1, 2, 128), (2, 1, 192), (2, 3, 256), (1, 8, 1024),
                                   (4, 16, 1024)])
def test_gdn_fp32_with_h0(B, H, T):
    announce(f"GDN fp32 B{B} H{H} T{T} h0")
    inp = make_delta_inputs(B, H, T, kind="gdn", dtype=torch.float32, seed=B * 100 + H, h0_std=0.02)
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp)
    _check(f"GDN fp32 B{B} H{H} T{T} h0", o, h, o_ref, h_ref, bf16=False)


@pytest.mark.parametrize("B,H,T,h0", [(1, 3, 64, False), (2, 2, 64, True), (1, 4, 128, True),
                                      (1, 2, 192, False)])
def test_gdn_bf16_short_sequences(B, H, T, h0):
    """bf16 at one, two and three chunks per chain: T = C takes the single-chunk path of the
    scan launcher, T = 2C and 3C the shortest runs of the pipelined kernel."""
    announce(f"GDN bf16 B{B} H{H} T{T} h0={h0}")
    inp = make_delta_inputs(B, H, T, kind="gdn", dtype=torch.bfloat16, seed=T + B * 10 + H,
                            h0_std=0.02 if h0 else None)
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp)
    _check(f"GDN bf16 B{B} H{H} T{T}{' h0' if h0 else ''}", o, h, o_ref, h_ref, bf16=True)


def _gate_case(name, T, seed, B=1, H=2):
    """Per-token log decay g [B, H, T] for the score-gate cases of the scan kernel."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(B, H, T, generator=gen)
    sp = torch.nn.functional.softplus
    if name == "mixed_sign":          # g > 0 in places: the clamp of e^{min(G_i - G_j, 0)} acts
        return x * 0.05 - 0.03
    if name == "steep":               # > 80 of decay inside a 16-token block
        return -sp(x) * 12.0
    if name == "near_limit":          # about 70 per block: the factored gate's largest key factor
        return -torch.full_like(x, 70.0 / 15)
    if name == "alternating":         # steep and gentle chunks in one sequence
        g = -sp(x) * 0.1
        steep = (torch.arange(T) // 64) % 2 == 1
        g[..., steep] = -sp(x[..., steep]) * 12.0
        return g
    raise ValueError(name)


@pytest.mark.parametrize("name", ["mixed_sign", "steep", "near_limit", "alternating"])
def test_gdn_bf16_score_gates(name):
    """The scan forms the causal score's gate e^{min(G_i - G_j, 0)} from per-chunk factor tables
    when G falls through the chunk and no 16-token block decays by more than 80, and per
    element otherwise (a rising G, steeper blocks); both paths against the oracle."""
    T = 1024
    announce(f"GDN bf16 score gates {name} B1 H2 T{T}")
    inp = make_delta_inputs(1, 2, T, kind="gdn", dtype=torch.bfloat16, seed=11, h0_std=0.02)
    inp["g"] = _gate_case(name, T, 12).float()
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp)
    assert np.isfinite(o).all() and np.isfinite(h).all()
    _check(f"GDN bf16 score gates {name}", o, h, o_ref, h_ref, bf16=True)


# The scan launcher takes 32-column state slices (four workgroups per chain) when B*H >= 64, the
# headline's instantiation, and 16-column slices below that; the tests above at B*H <= 6 run the
# 16-column kernel.  The cases below run the 32-column one at its edges: one, two and three
# chunks per chain (the loaders' end-of-chain clamps), a nonzero h0, both score-gate paths, and
# B*H not a multiple of 8 (the slice mapping without XCD grouping).
@pytest.mark.parametrize("T", [64, 128, 192, 1024])
def test_gdn_bf16_wide_slices_h0(T):
    B, H = 4, 16
    announce(f"GDN bf16 32-column slices B{B} H{H} T{T} h0")
    inp = make_delta_inputs(B, H, T, kind="gdn", dtype=torch.bfloat16, seed=40 + T, h0_std=0.02)
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp)
    _check(f"GDN bf16 B{B} H{H} T{T} h0 (32-col)", o, h, o_ref, h_ref, bf16=True)


@pytest.mark.parametrize("name", ["mixed_sign", "steep", "near_limit", "alternating"])
def test_gdn_bf16_wide_slices_score_gates(name):
    """Both score-gate paths (factor tables, per element) in the 32-column kernel."""
    B, H, T = 4, 16, 1024
    announce(f"GDN bf16 score gates {name} B{B} H{H} T{T} (32-col)")
    inp = make_delta_inputs(B, H, T, kind="gdn", dtype=torch.bfloat16, seed=13, h0_std=0.02)
    inp["g"] = _gate_case(name, T, 14, B, H).float()
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp)
    assert np.isfinite(o).all() and np.isfinite(h).all()
    _check(f"GDN bf16 score gates {name} B{B} H{H} (32-col)", o, h, o_ref, h_ref, bf16=True)


@pytest.mark.parametrize("B,H,T", [(3, 22, 512), (5, 13, 192)])
def test_gdn_bf16_wide_slices_unaligned_chains(B, H, T):
    """B*H = 66 and 65: 32-column slices, chains not grouped by XCD (B*H % 8 != 0)."""
    announce(f"GDN bf16 B{B} H{H} T{T} h0 (32-col, B*H % 8 != 0)")
    inp = make_delta_inputs(B, H, T, kind="gdn", dtype=torch.bfloat16, seed=B * 50 + H,
                            h0_std=0.02)
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp)
    _check(f"GDN bf16 B{B} H{H} T{T} h0 (32-col)", o, h, o_ref, h_ref, bf16=True)


@pytest.mark.parametrize("B,H,T", [(16, 32, 128), (7, 73, 192)])
def test_gdn_bf16_many_chains(B, H, T):
    """512 and 511 chains: eight and about eight scan workgroups per CU over the run (several
    generations of workgroups), with the XCD-aware chain mapping (B*H % 8 == 0) and without."""
    announce(f"GDN bf16 B{B} H{H} T{T} h0 (many chains)")
    inp = make_delta_inputs(B, H, T, kind="gdn", dtype=torch.bfloat16, seed=B * 70 + H,
                            h0_std=0.02)
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp)
    _check(f"GDN bf16 B{B} H{H} T{T} h0 (many chains)", o, h, o_ref, h_ref, bf16=True)


@pytest.mark.parametrize("B,H,T", [(4, 16, 1024), (1, 2, 256)])
def test_deltanet_bf16_fused(B, H, T):
    """DeltaNet (g = None) through the fused bf16 forward, against deltanet_reference
    (forwards/deltanet.py:114-143 of the reference): the 32- and the 16-column scan."""
    announce(f"DeltaNet bf16 fused B{B} H{H} T{T}")
    inp = make_delta_inputs(B, H, T, kind="deltanet", dtype=torch.bfloat16, seed=60 + H)
    assert inp["g"] is None
    o, h = _run(inp)
    x = as_oracle_inputs(inp)
    ref = deltanet_reference(x["q"], x["k"], x["v"], x["beta"], C=64, dtype=np.float64)
    _check(f"DeltaNet bf16 fused B{B} H{H} T{T}", o, h, ref["o"].reshape(o.shape), ref["final"],
           bf16=True)


def test_deltanet_bf16_longest_chain():
    """No decay at the longest chain the forward takes in one call at this size (T = 32768,
    512 chunks) with h0: the state's bf16 rounding never washes out, so this is where its error
    builds up most; it levels off near 1e-2 on h (|h| up to ~3)."""
    announce("DeltaNet bf16 fused B1 H2 T32768 h0")
    inp = make_delta_inputs(1, 2, 32768, kind="deltanet", dtype=torch.bfloat16, seed=3, h0_std=0.02)
    o, h = _run(inp)
    x = as_oracle_inputs(inp)
    ref = deltanet_reference(x["q"], x["k"], x["v"], x["beta"], C=64, h0=x["h0"], dtype=np.float64)
    _check("DeltaNet bf16 fused B1 H2 T32768 h0", o, h, ref["o"].reshape(o.shape), ref["final"],
           bf16=True)


def test_gdn_bf16_config2():
    announce("GDN bf16 B4 H16 T4096")
    inp = make_delta_inputs(4, 16, 4096, kind="gdn", dtype=torch.bfloat16, seed=0)
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp, dtype=np.float32)
    _check("GDN bf16 config 2 B4 H16 T4096", o, h, o_ref, h_ref, bf16=True)


def test_gdn_bf16_config4_long_context():
    announce("GDN bf16 B1 H32 T32768 h0")
    inp = make_delta_inputs(1, 32, 32768, kind="gdn", dtype=torch.bfloat16, seed=4, h0_std=0.02)
    o, h = _run(inp)
    o_ref, h_ref = _oracle(inp, dtype=np.float32)
    _check("GDN bf16 config 4 B1 H32 T32768 h0", o, h, o_ref, h_ref, bf16=True)
    # the state carries 512 chunks of bf16 operand rounding: keep 2x headroom under the bound
    assert max_abs(h, h_ref) <= BF16_TOL / 2, max_abs(h, h_ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gdn_chunk_size_128(dtype):
    """C = 128 (the reference's chunk) runs the 64-token kernels over T / 64 chunks: against the
    oracle chunked at 128 within the stated bound, and equal to the C = 64 call bit for bit (the
    same kernels on the same data)."""
    B, H, T = 1, 4, 1024
    announce(f"GDN {dtype} C128 B{B} H{H} T{T} h0")
    inp = make_delta_inputs(B, H, T, kind="gdn", dtype=dtype, seed=31, h0_std=0.02)
    d = {n: (None if t is None else t.to(DEV)) for n, t in inp.items()}
    o128, h128 = gdn_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], h0=d["h0"],
                                   chunk_size=128)
    o64, h64 = gdn_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], h0=d["h0"])
    torch.cuda.synchronize()
    x = as_oracle_inputs(inp)
    o_ref, h_ref = gdn_reference(x["q"], x["k"], x["v"], x["beta"], x["g"], h0=x["h0"], C=128,
                                 dtype=np.float64)
    bf16 = dtype == torch.bfloat16
    _check(f"GDN {'bf16' if bf16 else 'fp32'} C128 B{B} H{H} T{T} h0", o128.cpu().numpy(),
           h128.cpu().numpy(), o_ref, h_ref, bf16=bf16)
    assert torch.equal(o128, o64) and torch.equal(h128, h64)
    with pytest.raises(ValueError, match="multiple of the chunk size"):
        gdn_chunk_forward(d["q"][:, :, :192], d["k"][:, :, :192], d["v"][:, :, :192],
                          d["beta"][:, :, :192], d["g"][:, :, :192], chunk_size=128)


def test_gdn_deterministic():
    announce("GDN bf16 determinism B2 H8 T1024")
    inp = make_delta_inputs(2, 8, 1024, kind="gdn", dtype=torch.bfloat16, seed=7)
    o1, h1 = _run(inp)
    o2, h2 = _run(inp)
    assert np.array_equal(o1, o2) and np.array_equal(h1, h2)


def test_gdn_state_passing_config4():
    """Size-independent property at the long-context shape (config 4, with h0): running [0,T)
    equals running [0,T/2) and then [T/2,T) from the first half's final state.  Both runs see
    the same bf16 operands; they differ only in where the kernel's deferred state factor is
    folded back in, so the difference stays far below the oracle tolerance (5e-3 abs)."""
    announce("GDN bf16 state passing B1 H32 T32768 h0")
    inp = make_delta_inputs(1, 32, 32768, kind="gdn", dtype=torch.bfloat16, seed=4, h0_std=0.02)
    d = {n: (None if t is None else t.to(DEV)) for n, t in inp.items()}
    o, h = gdn_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], h0=d["h0"])
    T2 = 16384
    part = lambda n, sl: d[n][:, :, sl].contiguous()   # noqa: E731
    first = {n: part(n, slice(0, T2)) for n in ("q", "k", "v", "beta", "g")}
    second = {n: part(n, slice(T2, None)) for n in ("q", "k", "v", "beta", "g")}
    o1, h1 = gdn_chunk_forward(first["q"], first["k"], first["v"], first["beta"], first["g"],
                               h0=d["h0"])
    o2, h2 = gdn_chunk_forward(second["q"], second["k"], second["v"], second["beta"],
                               second["g"], h0=h1)
    torch.cuda.synchronize()
    err_o = record_error("GDN state passing config 4", "o", torch.cat([o1, o2], 2).cpu().numpy(),
                         o.cpu().numpy(), "max abs <= 5e-3")["abs"]
    err_h = record_error("GDN state passing config 4", "h", h2.cpu().numpy(), h.cpu().numpy(),
                         "max abs <= 5e-3")["abs"]
    assert err_o <= 5e-3 and err_h <= 5e-3, (err_o, err_h)


def test_gdn_linear_in_v_config2():
    """Size-independent property at the headline shape (config 2, h0 = 0): o and the final state
    are linear in v.  Doubling v is exact in bf16 and every step of the kernel (beta v, the
    fp32 MFMA accumulations, the bf16 packing of the state and of v_new, the fused
    multiply-adds) commutes with a factor of two, so the result is exactly twice the original,
    bit for bit."""
    announce("GDN bf16 linearity in v B4 H16 T4096")
    inp = make_delta_inputs(4, 16, 4096, kind="gdn", dtype=torch.bfloat16, seed=0)
    o1, h1 = _run(inp)
    inp2 = dict(inp, v=inp["v"] * 2)
    o2, h2 = _run(inp2)
    assert np.array_equal(o2, 2 * o1), max_abs(o2, 2 * o1)
    assert np.array_equal(h2, 2 * h1), max_abs(h2, 2 * h1)


@pytest.mark.parametrize("dtype,B,H,T", [(torch.bfloat16, 2, 4, 512), (torch.float32, 1, 4, 512),
                                         (torch.float32, 4, 16, 1024)])
def test_gdn_without_final_state(dtype, B, H, T):
    """output_final_state=False passes a NULL final-state pointer: no state is written, None is
    returned, and o is bit-identical to the call that also writes the state (the fp32 cases at
    32 and 512 slices: one and two generations of scan workgroups)."""
    announce(f"GDN {dtype} without final state B{B} H{H} T{T}")
    inp = make_delta_inputs(B, H, T, kind="gdn", dtype=dtype, seed=11, h0_std=0.02)
    d = {n: (None if t is None else t.to(DEV)) for n, t in inp.items()}
    o1, h1 = gdn_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], h0=d["h0"])
    o2, h2 = gdn_chunk_forward(d["q"], d["k"], d["v"], d["beta"], d["g"], h0=d["h0"],
                               output_final_state=False)
    torch.cuda.synchronize()
    assert h2 is None and h1 is not None
    assert torch.equal(o1, o2)
