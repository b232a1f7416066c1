"""The compile stack on the GPU: staged programs, every fused-registry key through its adapter,
HIP-graph capture and replay, and compile_program with on-device verification.

Gates: the reference's frob_rel < 2e-2 for bf16 programs against the fp32 oracle / the canonical
program; lowered vs canonical programs and graph replay vs eager within the same bound; replays
of one graph bit-identical to each other.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle.gdn_oracle import gdn_reference, kda_reference, kkt_reference
from pto_fuser_amd import (Features, FusedNode, GraphReplayExecutor, Policy, StagedExecutor,
                           canonicalize, compile_program, decide, frob_rel)
from pto_fuser_amd.forwards import (build_gdn_program, build_kda_program, build_kkt_fused_program,
                                    build_scan_fused_program, build_scan_staged_program,
                                    make_gdn_inputs, make_kda_inputs, make_kkt_inputs,
                                    make_scan_inputs, prepare_gdn_bindings, prepare_kda_bindings)
from pto_fuser_amd.template import FuseContractionEpilogue

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-2


def _frob(got, ref):
    got = np.asarray(got, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def _gdn(B, H, nc, C, D, seed=0):
    inp = make_gdn_inputs(B, H, nc, C, D, device=DEV, seed=seed)
    binds = prepare_gdn_bindings(inp["q"], inp["k"], inp["v"], inp["beta"], inp["g_in"])
    T = nc * C
    x = {n: t.double().cpu().numpy() for n, t in inp.items()}
    ref, _ = gdn_reference(x["q"].reshape(B, H, T, D), x["k"].reshape(B, H, T, D),
                           x["v"].reshape(B, H, T, D), x["beta"].reshape(B, H, T),
                           x["g_in"].reshape(B, H, T), C=C, dtype=np.float64)
    return binds, build_gdn_program(B, H, nc, C, D, D ** -0.5), ref.reshape(B, H, nc, C, D)


@pytest.mark.parametrize("B,H,nc,C,D", [(1, 4, 2, 128, 128), (2, 3, 3, 64, 128)])
def test_gdn_program_staged_and_lowered(B, H, nc, C, D):
    announce(f"gdn program staged+lowered B{B} H{H} nc{nc} C{C} D{D}")
    binds, prog, ref = _gdn(B, H, nc, C, D)
    ex = StagedExecutor()
    staged = ex.run(canonicalize(prog), binds)["o"]
    lowered = compile_program(prog, Features(B, H, nc, C, D), verify=False).program
    assert {n.kernel for n in lowered.nodes if isinstance(n, FusedNode)} >= {"chunk_h_scan"}
    fused = ex.run(lowered, binds)["o"]
    partial = ex.run(FuseContractionEpilogue(B, H, nc, C, D).apply(canonicalize(prog)).program,
                     binds)["o"]
    torch.cuda.synchronize()
    for name, t in (("staged", staged), ("lowered", fused), ("epilogue-fused", partial)):
        assert _frob(t.cpu(), ref) < TOL, (name, _frob(t.cpu(), ref))


def test_kda_program_staged_and_lowered():
    B, H, nc, C, D = 1, 4, 2, 64, 128
    announce("kda program staged+lowered")
    inp = make_kda_inputs(B, H, nc, C, D, device=DEV, seed=1)
    binds = prepare_kda_bindings(inp["q"], inp["k"], inp["v"], inp["beta"], inp["g_in"])
    prog = build_kda_program(B, H, nc, C, D, D ** -0.5)
    T = nc * C
    x = {n: t.double().cpu().numpy() for n, t in inp.items()}
    ref, _ = kda_reference(x["q"].reshape(B, H, T, D), x["k"].reshape(B, H, T, D),
                           x["v"].reshape(B, H, T, D), x["beta"].reshape(B, H, T),
                           x["g_in"].reshape(B, H, T, D), C=C, dtype=np.float64)
    ex = StagedExecutor()
    lowered = compile_program(prog, Features(B, H, nc, C, D, per_dim_gate=True),
                              verify=False).program
    partial = FuseContractionEpilogue(B, H, nc, C, D).apply(canonicalize(prog)).program
    for name, p in (("staged", canonicalize(prog)), ("lowered", lowered), ("prologue", partial)):
        o = ex.run(p, binds)["o"]
        torch.cuda.synchronize()
        assert _frob(o.cpu().reshape(B, H, T, D), ref) < TOL, name


def test_kkt_gated_token_layout_node():
    nc, H = 3, 4
    announce("kkt_gated token layout node")
    inp = make_kkt_inputs(nc, H, C=64, D=128, device=DEV, seed=2)
    L = StagedExecutor().run(build_kkt_fused_program(nc, H), inp)["L"]
    torch.cuda.synchronize()
    ref = kkt_reference(inp["k"].double().cpu().numpy(), inp["g_sum"].cpu().numpy(),
                        inp["beta"].cpu().numpy(), nc, H, 64, dtype=np.float64)
    assert L.shape == (nc * 64, H, 64) and _frob(L.float().cpu(), ref) < 1e-2


def test_scan_stage_fusion_decision():
    B, H, nc = 1, 4, 4
    announce("scan stage staged vs fused decision")
    inp = make_scan_inputs(B, H, nc, device=DEV, seed=3)
    ex = StagedExecutor()
    staged, fused = build_scan_staged_program(B, H, nc), build_scan_fused_program(B, H, nc)
    d = decide("chunk_h_scan", "chunk_h_scan", lambda: ex.run(staged, inp),
               lambda: ex.run(fused, inp), iters=5, warmup=1)
    assert d.gated_ok and d.deterministic, d.detail


def test_graph_replay_matches_eager_across_replays():
    """Capture the lowered GDN program once; replay it three times on new operands with eager
    work and synchronisations in between; every replay equals an eager run on the same
    operands, and two replays of the same operands are bit-identical."""
    B, H, nc, C, D = 1, 4, 2, 64, 128
    announce("graph replay lowered gdn")
    binds0, prog, _ = _gdn(B, H, nc, C, D, seed=4)
    lowered = compile_program(prog, Features(B, H, nc, C, D), verify=False).program
    gr = GraphReplayExecutor().capture(lowered, binds0)
    ex = StagedExecutor()
    first = None
    for seed in (5, 6, 7):
        binds, _, _ = _gdn(B, H, nc, C, D, seed=seed)
        out = gr.replay(binds)["o"]
        eager = ex.run(lowered, binds)["o"]
        torch.cuda.synchronize()
        assert frob_rel(out, eager) < 1e-5
        if first is None:
            first = (binds, out)
    again = gr.replay(first[0])["o"]
    torch.cuda.synchronize()
    assert torch.equal(again, first[1])


def test_compile_program_verified_on_device():
    B, H, nc, C, D = 1, 4, 2, 128, 128
    announce("compile_program verify=True gdn")
    binds, prog, ref = _gdn(B, H, nc, C, D, seed=8)
    res = compile_program(prog, Features(B, H, nc, C, D), bindings=binds, iters=5, warmup=2)
    assert res.report.verified
    for rec in res.report.records:
        if rec.attempted:
            assert rec.frob is not None and rec.t_cand_ms is not None
        if rec.kept:
            assert rec.frob < TOL and rec.deterministic and rec.faster
    o = StagedExecutor().run(res.program, binds)["o"]
    torch.cuda.synchronize()
    assert _frob(o.cpu(), ref) < TOL
    print(res.report)


def _kda(B, H, nc, C, D, seed=0):
    inp = make_kda_inputs(B, H, nc, C, D, device=DEV, seed=seed)
    binds = prepare_kda_bindings(inp["q"], inp["k"], inp["v"], inp["beta"], inp["g_in"])
    T = nc * C
    x = {n: t.double().cpu().numpy() for n, t in inp.items()}
    ref, _ = kda_reference(x["q"].reshape(B, H, T, D), x["k"].reshape(B, H, T, D),
                           x["v"].reshape(B, H, T, D), x["beta"].reshape(B, H, T),
                           x["g_in"].reshape(B, H, T, D), C=C, dtype=np.float64)
    return binds, build_kda_program(B, H, nc, C, D, D ** -0.5), ref.reshape(B, H, nc, C, D)


@pytest.mark.parametrize("family", ["gdn", "kda"])
def test_whole_forward_program_matches_oracle_and_staged(family):
    """Policy(whole_forward=True) collapses the canonical program into one fused-forward node;
    its output matches the fp64 oracle and the staged program within the bf16 bound."""
    B, H, nc, C, D = (2, 3, 3, 64, 128) if family == "gdn" else (1, 4, 3, 64, 128)
    announce(f"whole-forward program {family} B{B} H{H} nc{nc}")
    binds, prog, ref = (_gdn if family == "gdn" else _kda)(B, H, nc, C, D, seed=21)
    f = Features(B, H, nc, C, D, per_dim_gate=family == "kda")
    whole = compile_program(prog, f, policy=Policy(whole_forward=True), verify=False).program
    assert [n.kernel for n in whole.nodes] == [f"{family}_forward"]
    ex = StagedExecutor()
    o = ex.run(whole, binds)["o"]
    staged = ex.run(canonicalize(prog), binds)["o"]
    torch.cuda.synchronize()
    assert o.shape == (B, H, nc, C, D) and o.dtype == torch.float32
    assert _frob(o.cpu(), ref) < TOL, _frob(o.cpu(), ref)
    assert frob_rel(o, staged) < TOL


@pytest.mark.parametrize("family", ["gdn", "kda"])
def test_whole_forward_at_the_reference_chunk_128(family):
    """The reference's compiled_forward shape (examples/attention/gdn.py:75-88: B=1, H=16, nc=8,
    C=128, D=128) lowers to the fused two-kernel forward (run as 64-token chunks) and matches the
    oracle chunked at 128 within the bf16 bound; verified and kept by compile_program."""
    B, H, nc, C, D = 1, 16, 8, 128, 128
    announce(f"whole-forward program {family} C128 B{B} H{H} nc{nc}")
    binds, prog, ref = (_gdn if family == "gdn" else _kda)(B, H, nc, C, D, seed=41)
    f = Features(B, H, nc, C, D, per_dim_gate=family == "kda")
    res = compile_program(prog, f, policy=Policy(whole_forward=True), bindings=binds, iters=5,
                          warmup=2)
    assert [n.kernel for n in res.program.nodes] == [f"{family}_forward"], str(res.report)
    assert res.report.records[0].kept, str(res.report)
    o = StagedExecutor().run(res.program, binds)["o"]
    torch.cuda.synchronize()
    assert o.shape == (B, H, nc, C, D)
    err = _frob(o.cpu(), ref)
    print(f"{family} C128 whole forward vs oracle: frob {err:.2e}")
    assert err < TOL, err


def test_whole_gdn_forward_fp32_program():
    """fp32 work dtype: the whole-forward node runs the fused fp32 path (1e-4 relative)."""
    B, H, nc, C, D = 1, 2, 3, 64, 128
    announce("whole-forward program gdn fp32")
    inp = make_gdn_inputs(B, H, nc, C, D, device=DEV, seed=22, dtype=torch.float32)
    binds = prepare_gdn_bindings(inp["q"], inp["k"], inp["v"], inp["beta"], inp["g_in"],
                                 work=torch.float32)
    T = nc * C
    x = {n: t.double().cpu().numpy() for n, t in inp.items()}
    ref, _ = gdn_reference(x["q"].reshape(B, H, T, D), x["k"].reshape(B, H, T, D),
                           x["v"].reshape(B, H, T, D), x["beta"].reshape(B, H, T),
                           x["g_in"].reshape(B, H, T), C=C, dtype=np.float64)
    prog = build_gdn_program(B, H, nc, C, D, D ** -0.5, work=torch.float32)
    whole = compile_program(prog, Features(B, H, nc, C, D, dtype=torch.float32),
                            policy=Policy(whole_forward=True), verify=False).program
    o = StagedExecutor().run(whole, binds)["o"]
    torch.cuda.synchronize()
    got = o.double().cpu().numpy().reshape(B, H, T, D)
    assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-4


def test_whole_kda_forward_fp32_program():
    """fp32 work dtype: the whole KDA node runs the fused fp32 kernels (1e-4 relative), one
    chunk per sequence included."""
    for B, H, nc in ((1, 2, 3), (1, 3, 1)):
        C, D = 64, 128
        announce(f"whole-forward program kda fp32 B{B} H{H} nc{nc}")
        inp = make_kda_inputs(B, H, nc, C, D, device=DEV, seed=23 + nc, dtype=torch.float32)
        binds = prepare_kda_bindings(inp["q"], inp["k"], inp["v"], inp["beta"], inp["g_in"],
                                     work=torch.float32)
        T = nc * C
        x = {n: t.double().cpu().numpy() for n, t in inp.items()}
        ref, _ = kda_reference(x["q"].reshape(B, H, T, D), x["k"].reshape(B, H, T, D),
                               x["v"].reshape(B, H, T, D), x["beta"].reshape(B, H, T),
                               x["g_in"].reshape(B, H, T, D), C=C, dtype=np.float64)
        prog = build_kda_program(B, H, nc, C, D, D ** -0.5, work=torch.float32)
        whole = compile_program(prog, Features(B, H, nc, C, D, dtype=torch.float32,
                                               per_dim_gate=True),
                                policy=Policy(whole_forward=True), verify=False).program
        assert [n.kernel for n in whole.nodes if isinstance(n, FusedNode)] == ["kda_forward"]
        o = StagedExecutor().run(whole, binds)["o"]
        torch.cuda.synchronize()
        got = o.double().cpu().numpy().reshape(B, H, T, D)
        assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-4


@pytest.mark.parametrize("family", ["gdn", "kda"])
def test_compile_program_keeps_whole_forward_verified(family):
    """With bindings the driver captures the whole-forward candidate into a HIP graph, gates it
    against the canonical program (frob, replay determinism, time) and keeps it."""
    B, H, nc, C, D = 1, 4, 2, 64, 128
    announce(f"compile_program verify=True whole-forward {family}")
    binds, prog, ref = (_gdn if family == "gdn" else _kda)(B, H, nc, C, D, seed=23)
    f = Features(B, H, nc, C, D, per_dim_gate=family == "kda")
    res = compile_program(prog, f, policy=Policy(whole_forward=True), bindings=binds, iters=5,
                          warmup=2)
    first = res.report.records[0]
    assert first.name == f"fuse-{family}-forward"
    assert first.kept and first.frob < TOL and first.deterministic and first.faster, str(res.report)
    assert [n.kernel for n in res.program.nodes] == [f"{family}_forward"]
    gr = GraphReplayExecutor().capture(res.program, binds)
    for _ in range(3):
        out = gr.replay(binds)["o"]
        torch.cuda.synchronize()
        assert _frob(out.cpu(), ref) < TOL
