"""Transform layer (no device): canonical form, annotation levers, structural rewrites — each
matches only its own family, emits the expected node, is idempotent and leaves a valid Program
(reference tests/test_transform.py)."""
from pto_fuser_amd import (EinsumNode, EnableDirectReads, EnableFusedStore, FusedNode,
                           FuseContractionEpilogue, canonicalize)
from pto_fuser_amd.forwards import build_gdn_program, build_kda_program
from pto_fuser_amd.transforms import LowerPerDimScan, LowerResidentScan


def _gdn(B=1, H=4, nc=2, C=128, D=128):
    return build_gdn_program(B, H, nc, C, D, D ** -0.5)


def _kda(B=1, H=4, nc=2, C=128, D=128):
    return build_kda_program(B, H, nc, C, D, D ** -0.5)


def test_canonicalize_forces_nn():
    einsums = [n for n in canonicalize(_gdn()).nodes if isinstance(n, EinsumNode)]
    assert einsums and all(n.read_mode == "NN" and not n.fuse_out for n in einsums)


def test_enable_direct_reads_is_idempotent():
    canon = canonicalize(_gdn())
    t = EnableDirectReads()
    n = t.match(canon)
    assert n == sum(isinstance(x, EinsumNode) for x in canon.nodes) > 0
    res = t.apply(canon)
    assert res.changed and res.sites == n
    assert all(x.read_mode == "auto" for x in res.program.nodes if isinstance(x, EinsumNode))
    assert t.match(res.program) == 0


def test_enable_fused_store_is_idempotent():
    t = EnableFusedStore()
    res = t.apply(canonicalize(_gdn()))
    assert res.changed and all(x.fuse_out for x in res.program.nodes if isinstance(x, EinsumNode))
    assert t.match(res.program) == 0


def test_scans_match_only_their_family():
    assert LowerResidentScan(1, 4, 2, 128, 128).match(_gdn()) == 1
    assert LowerResidentScan(1, 4, 2, 128, 128).match(_kda()) == 0
    assert LowerPerDimScan(1, 4, 2, 128, 128).match(_kda()) == 1
    assert LowerPerDimScan(1, 4, 2, 128, 128).match(_gdn()) == 0


def test_generator_matches_both_forwards():
    assert FuseContractionEpilogue(1, 4, 2, 128, 128).match(_gdn()) == 2
    assert FuseContractionEpilogue(1, 4, 2, 128, 128).match(_kda()) == 1


def test_generator_emits_stage_kernels():
    gdn = FuseContractionEpilogue(1, 4, 2, 128, 128).apply(canonicalize(_gdn())).program
    assert {n.kernel for n in gdn.nodes if isinstance(n, FusedNode)} == \
        {"kkt_gated_native", "gated_qk_native"}
    kda = FuseContractionEpilogue(1, 4, 2, 128, 128).apply(canonicalize(_kda())).program
    kk = {n.kernel for n in kda.nodes if isinstance(n, FusedNode)}
    assert len(kk) == 1 and next(iter(kk)).startswith("qk_prologue")


def test_resident_scan_idempotent_and_valid():
    t = LowerResidentScan(1, 4, 2, 128, 128)
    prog = t.apply(canonicalize(_gdn())).program
    fused = [n for n in prog.nodes if isinstance(n, FusedNode) and n.kernel == "chunk_h_scan"]
    assert len(fused) == 1 and "perdim_decay" not in fused[0].params
    assert t.match(prog) == 0
    assert "S0" not in {getattr(n, "output", None) for n in prog.nodes}
    assert prog.outputs == ["o"]


def test_perdim_scan_marks_the_decay():
    prog = LowerPerDimScan(1, 4, 2, 128, 128).apply(canonicalize(_kda())).program
    fused = [n for n in prog.nodes if isinstance(n, FusedNode) and n.kernel == "chunk_h_scan"]
    assert len(fused) == 1 and fused[0].params.get("perdim_decay") is True


def test_transforms_compose_into_valid_program():
    prog = LowerResidentScan(1, 4, 2, 128, 128).apply(canonicalize(_gdn())).program
    prog = FuseContractionEpilogue(1, 4, 2, 128, 128).apply(prog).program
    assert {n.kernel for n in prog.nodes if isinstance(n, FusedNode)} == \
        {"chunk_h_scan", "kkt_gated_native", "gated_qk_native"}
    assert prog.outputs == ["o"]


def test_templates_carry_the_full_batch():
    """Every emitted stage node names M = B·H·nc chunks and its C, D — not the reference's
    B = 1 / C = 128 envelope."""
    B, H, nc, C, D = 3, 2, 2, 64, 128
    prog = FuseContractionEpilogue(B, H, nc, C, D).apply(canonicalize(_gdn(B, H, nc, C, D))).program
    for n in prog.nodes:
        if isinstance(n, FusedNode):
            assert n.params["nc"] * n.params["H"] == B * H * nc
            assert n.params["C"] == C and n.params["D"] == D
