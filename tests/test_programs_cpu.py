"""Program numerics on the CPU (no device): the canonical builders against the oracle, and every
lowering against its canonical program, with the HIP kernels replaced by the oracle stand-ins of
tests/cpu_kernels.py.  This pins what the GPU tests cannot separate from kernel error: that the
builders compute the delta-rule forward, and that each rewrite's layouts, permutes and operand
names are right.  fp32 work dtype throughout; tolerance max rel 1e-4 vs the fp32 oracle, 1e-5
between lowerings."""
import numpy as np
import pytest
import torch

from cpu_kernels import cpu_fused_registry, cpu_opaque_registry
from oracle.gdn_oracle import deltanet_reference, gdn_reference, kda_reference, max_rel
from pto_fuser_amd import Features, FusedNode, StagedExecutor, canonicalize, compile_program
from pto_fuser_amd.forwards import (build_deltanet_program, build_gdn_program, build_kda_program,
                                    build_scan_fused_program, build_scan_staged_program,
                                    make_gdn_inputs, make_inputs, make_kda_inputs,
                                    make_scan_inputs, prepare_gdn_bindings, prepare_kda_bindings)
from pto_fuser_amd.template import FuseChunkOFlash, FuseContractionEpilogue
from pto_fuser_amd.transforms import LowerResidentScan

F32 = torch.float32
B, H, nc, C, D = 2, 2, 3, 16, 32


def _exec():
    return StagedExecutor(registry=cpu_opaque_registry(), fused=cpu_fused_registry())


def _np(t):
    return t.detach().double().numpy()


def _gdn_case():
    inp = make_gdn_inputs(B, H, nc, C, D, dtype=F32, seed=1)
    binds = prepare_gdn_bindings(inp["q"], inp["k"], inp["v"], inp["beta"], inp["g_in"], work=F32)
    prog = build_gdn_program(B, H, nc, C, D, D ** -0.5, work=F32)
    return inp, binds, prog


def test_gdn_program_computes_the_reference():
    inp, binds, prog = _gdn_case()
    o = _exec().run(prog, binds)["o"]
    T = nc * C
    ref, _ = gdn_reference(_np(inp["q"]).reshape(B, H, T, D), _np(inp["k"]).reshape(B, H, T, D),
                           _np(inp["v"]).reshape(B, H, T, D), _np(inp["beta"]).reshape(B, H, T),
                           _np(inp["g_in"]).reshape(B, H, T), C=C, dtype=np.float64)
    assert max_rel(_np(o).reshape(B, H, T, D), ref) < 1e-4


def test_gdn_lowerings_match_canonical():
    _, binds, prog = _gdn_case()
    ex = _exec()
    ref = ex.run(canonicalize(prog), binds)["o"]
    full = compile_program(prog, Features(B, H, nc, C, D, dtype=F32), verify=False).program
    assert {n.kernel for n in full.nodes if isinstance(n, FusedNode)} == \
        {"chunk_h_scan", "kkt_gated_native", "qkv_flash_native_v2"}
    for lowered in (full,
                    LowerResidentScan(B, H, nc, C, D, F32).apply(canonicalize(prog)).program,
                    FuseContractionEpilogue(B, H, nc, C, D).apply(canonicalize(prog)).program,
                    FuseChunkOFlash(B, H, nc, C, D).apply(canonicalize(prog)).program):
        got = ex.run(lowered, binds)["o"]
        assert max_rel(_np(got), _np(ref)) < 1e-5


def test_kda_program_and_lowering():
    inp = make_kda_inputs(B, H, nc, C, D, dtype=F32, seed=2)
    binds = prepare_kda_bindings(inp["q"], inp["k"], inp["v"], inp["beta"], inp["g_in"], work=F32)
    prog = build_kda_program(B, H, nc, C, D, D ** -0.5, work=F32)
    ex = _exec()
    o = ex.run(prog, binds)["o"]
    T = nc * C
    ref, _ = kda_reference(_np(inp["q"]).reshape(B, H, T, D), _np(inp["k"]).reshape(B, H, T, D),
                           _np(inp["v"]).reshape(B, H, T, D), _np(inp["beta"]).reshape(B, H, T),
                           _np(inp["g_in"]).reshape(B, H, T, D), C=C, dtype=np.float64)
    assert max_rel(_np(o).reshape(B, H, T, D), ref) < 1e-4
    res = compile_program(prog, Features(B, H, nc, C, D, dtype=F32, per_dim_gate=True),
                          verify=False)
    assert {n.kernel for n in res.program.nodes if isinstance(n, FusedNode)} == \
        {"chunk_h_scan", "qkvp_flash_native_v2"}
    assert max_rel(_np(ex.run(res.program, binds)["o"]), _np(o)) < 1e-5


def test_deltanet_program_outputs_match_reference():
    inp = make_inputs(B, H, nc, C, D, dtype=F32, seed=3)
    out = _exec().run(build_deltanet_program(B, H, nc, C, D, D ** -0.5, work=F32), inp)
    T = nc * C
    ref = deltanet_reference(_np(inp["q"]).reshape(B, H, T, D), _np(inp["k"]).reshape(B, H, T, D),
                             _np(inp["v"]).reshape(B, H, T, D), _np(inp["beta"]).reshape(B, H, T),
                             C=C, dtype=np.float64)
    for name in ("A", "T", "W", "U", "v_new", "h_state", "o"):
        assert max_rel(_np(out[name]), ref[name]) < 1e-4, name


@pytest.mark.parametrize("perdim", [False, True])
def test_scan_stage_programs_agree(perdim):
    Bs, Hs, ncs, Cs, Ds = 2, 3, 4, 16, 32
    inp = make_scan_inputs(Bs, Hs, ncs, Cs, Ds, dtype=F32, seed=4)
    fused = build_scan_fused_program(Bs, Hs, ncs)
    staged = build_scan_staged_program(Bs, Hs, ncs, Cs, Ds, work=F32)
    ex = _exec()
    a, b = ex.run(staged, inp), ex.run(fused, inp)
    for n in ("h_out", "final"):
        assert a[n].shape == b[n].shape
        assert max_rel(_np(b[n]), _np(a[n])) < 1e-5


def test_product_registries_refuse_cpu_tensors():
    """The product path has no CPU fallback: the real registries raise on host tensors."""
    _, binds, prog = _gdn_case()
    with pytest.raises(ValueError, match="HIP device"):
        StagedExecutor().run(prog, binds)
