"""The opt-in whole-forward rewrites (canonical GDN / KDA program -> one fused-forward node) and
their registry recipes, checked structurally on the CPU; the device parity of the rewritten
programs is in test_gpu_compile.py."""
import torch

from pto_fuser_amd import Features, FusedNode, Policy, canonicalize, compile_program
from pto_fuser_amd.forwards import (KDA_PROGRAM_INPUTS, build_deltanet_program, build_gdn_program,
                                    build_kda_program, make_gdn_inputs, make_kda_inputs,
                                    prepare_gdn_bindings, prepare_kda_bindings)
from pto_fuser_amd import _build
from pto_fuser_amd.fused import _per_token_gate, default_fused_registry
from pto_fuser_amd.transforms import FuseGdnForward, FuseKdaForward

SCALE = 128 ** -0.5


def _fused(prog):
    return [n for n in prog.nodes if isinstance(n, FusedNode)]


def test_default_policy_does_not_propose_whole_forward():
    f = Features(1, 4, 4, 64, 128)
    names = [p.name for p in Policy().pipeline(canonicalize(build_gdn_program(1, 4, 4, 64, 128,
                                                                            SCALE)), f)]
    assert "fuse-gdn-forward" not in names and "fuse-kda-forward" not in names


def test_whole_gdn_forward_replaces_the_program():
    B, H, nc, C, D = 2, 3, 4, 64, 128
    res = compile_program(build_gdn_program(B, H, nc, C, D, SCALE), Features(B, H, nc, C, D),
                          policy=Policy(whole_forward=True), verify=False)
    prog = res.program
    assert len(prog.nodes) == 1
    (node,) = _fused(prog)
    assert node.kernel == "gdn_forward" and node.outputs == ["o"]
    assert node.inputs == ["qF", "kF", "vF", "g_native", "beta_native"]
    assert node.params == {"B": B, "H": H, "nc": nc, "C": C, "D": D, "scale": SCALE}
    # first in the pipeline; every later transform then finds nothing to match
    assert res.report.records[0].name == "fuse-gdn-forward" and res.report.records[0].kept
    assert all(not r.matched for r in res.report.records[1:])


def test_whole_kda_forward_replaces_the_program():
    B, H, nc, C, D = 1, 2, 3, 64, 128
    f = Features(B, H, nc, C, D, per_dim_gate=True)
    prog = compile_program(build_kda_program(B, H, nc, C, D, 0.3), f,
                           policy=Policy(whole_forward=True), verify=False).program
    (node,) = _fused(prog)
    assert len(prog.nodes) == 1 and node.kernel == "kda_forward"
    assert node.params["scale"] == 0.3 and node.params["nc"] == nc


def test_whole_forward_matches_only_its_family_and_supported_shapes():
    gdn = canonicalize(build_gdn_program(1, 2, 2, 64, 128, SCALE))
    kda = canonicalize(build_kda_program(1, 2, 2, 64, 128, SCALE))
    assert FuseGdnForward(1, 2, 2, 64, 128).match(gdn) == 1
    assert FuseGdnForward(1, 2, 2, 64, 128).match(kda) == 0
    assert FuseKdaForward(1, 2, 2, 64, 128).match(kda) == 1
    assert FuseKdaForward(1, 2, 2, 64, 128).match(gdn) == 0
    # the reference's 128-token chunk runs on the 64-token kernels; other chunk / head sizes do not
    assert FuseGdnForward(1, 2, 2, 128, 128).match(
        canonicalize(build_gdn_program(1, 2, 2, 128, 128, SCALE))) == 1
    assert FuseGdnForward(1, 2, 2, 32, 128).match(
        canonicalize(build_gdn_program(1, 2, 2, 32, 128, SCALE))) == 0
    assert FuseGdnForward(1, 2, 2, 64, 64).match(
        canonicalize(build_gdn_program(1, 2, 2, 64, 64, SCALE))) == 0
    # KDA at C = 128: one 128-token chunk is two kernel chunks
    assert FuseKdaForward(1, 2, 1, 128, 128).match(
        canonicalize(build_kda_program(1, 2, 1, 128, 128, SCALE))) == 1
    # the fused KDA forward runs bf16 and fp32 operands at any length, one chunk included
    assert FuseKdaForward(1, 2, 2, 64, 128, work=torch.float32).match(kda) == 1
    assert FuseKdaForward(1, 2, 1, 64, 128, work=torch.float32).match(
        canonicalize(build_kda_program(1, 2, 1, 64, 128, SCALE, work=torch.float32))) == 1
    assert FuseKdaForward(1, 2, 1, 64, 128).match(
        canonicalize(build_kda_program(1, 2, 1, 64, 128, SCALE))) == 1
    # fp32 GDN runs the fp32 fused path
    assert FuseGdnForward(1, 2, 2, 64, 128, work=torch.float32).match(gdn) == 1
    # DeltaNet's program has no gate coefficients: not a whole-forward site
    dn = canonicalize(build_deltanet_program(1, 2, 2, 64, 128, SCALE))
    assert FuseGdnForward(1, 2, 2, 64, 128).match(dn) == 0


def test_whole_forward_is_idempotent():
    t = FuseGdnForward(1, 2, 2, 64, 128)
    once = t.apply(canonicalize(build_gdn_program(1, 2, 2, 64, 128, SCALE))).program
    assert t.match(once) == 0
    again = t.apply(once)
    assert not again.changed and again.program is once


def test_whole_forward_after_a_stage_lowering_still_matches():
    """A program already carrying the resident scan still computes the same forward from the same
    inputs; the whole rewrite replaces it as well."""
    from pto_fuser_amd.transforms import LowerResidentScan
    prog = canonicalize(build_gdn_program(1, 2, 2, 64, 128, SCALE))
    lowered = LowerResidentScan(1, 2, 2, 64, 128).apply(prog).program
    assert any(n.kernel == "chunk_h_scan" for n in _fused(lowered))
    whole = FuseGdnForward(1, 2, 2, 64, 128).apply(lowered).program
    assert [n.kernel for n in _fused(whole)] == ["gdn_forward"]


def test_registry_whole_forward_contracts():
    reg = default_fused_registry()
    for key in ("gdn_forward", "kda_forward"):
        c = reg.contract(key)
        assert c.in_slots == ["q", "k", "v", "g_native", "beta_native"]
        assert c.out_names == ["o"] and c.out_dtype == torch.float32
        r = reg.recipe(key)
        assert r.src_file == _build.LIB_NAME and r.src_dir == _build.LIB_DIR
        assert r.setup_sym == "" and r.teardown_sym == ""     # workspaces live in the ops module
        assert r.defines({"B": 1, "H": 2, "nc": 2, "C": 64, "D": 128, "x": 0}) == \
            {"B": 1, "H": 2, "nc": 2, "C": 64, "D": 128}


def test_bindings_carry_the_fp32_cumulative_gates():
    B, H, nc, C, D = 1, 2, 3, 64, 128
    gi = make_gdn_inputs(B, H, nc, C, D, seed=3)
    gb = prepare_gdn_bindings(gi["q"], gi["k"], gi["v"], gi["beta"], gi["g_in"])
    assert gb["g_native"].dtype == torch.float32 and gb["g_native"].shape == (B * H * nc, C)
    ki = make_kda_inputs(B, H, nc, C, D, seed=3)
    kb = prepare_kda_bindings(ki["q"], ki["k"], ki["v"], ki["beta"], ki["g_in"])
    assert set(KDA_PROGRAM_INPUTS) <= set(kb)
    assert kb["g_native"].dtype == torch.float32 and kb["g_native"].shape == (B * H * nc, C, D)
    assert kb["beta_native"].dtype == torch.float32 and kb["beta_native"].shape == (B * H * nc, C)
    assert torch.equal(kb["beta_native"], ki["beta"].float().reshape(B * H * nc, C))


def test_per_token_gate_inverts_the_chunk_cumsum():
    """The adapter recovers the per-token gate the fused kernels take from the bindings'
    cumulative one: exactly the binding's input where the cumsum is exact (integers), and to
    float rounding on the example's distribution."""
    g = torch.randint(-5, 1, (6, 64, 3)).float()
    assert torch.equal(_per_token_gate(g.cumsum(1)), g)
    gi = make_gdn_inputs(1, 2, 3, 64, 128, seed=5)
    G = gi["g_in"].float().cumsum(3).reshape(-1, 64)
    back = _per_token_gate(G).reshape(gi["g_in"].shape)
    assert torch.allclose(back, gi["g_in"].float(), atol=1e-5, rtol=0)
    assert torch.allclose(_per_token_gate(G).cumsum(1), G, atol=1e-5, rtol=0)
