"""Score templates (no device).

The templates are rows of data (``ScoreTemplate``) served by one matcher and one emitter.  These
tests check the table as a whole rather than each row by hand: every row fires on exactly the
contraction of its own forward and on nothing else, the node it emits follows the row, the steps
it absorbs leave a valid program, and a new row is all a new kernel needs.  The program numerics
of every rewrite are checked on the CPU in test_programs_cpu.py."""
import pytest

from pto_fuser_amd import (Dataflow, EinsumNode, FuseChunkOFlash, FusedNode,
                           FuseContractionEpilogue, FusePerDimChunkOFlash, Program, ScoreTemplate,
                           TensorOp, VecGlueNode, canonicalize, default_fused_registry,
                           epilogue_report, extract_epilogue_unit)
from pto_fuser_amd.forwards import build_gdn_program, build_kda_program
from pto_fuser_amd.template import CHUNK_O_GATED, KKT_GATED, QK_PROLOGUE, default_templates

DIMS = (2, 3, 2, 64, 128)          # B, H, nc, C, D
BUILD = {"gdn": build_gdn_program, "kda": build_kda_program}

# (row, forward it belongs to, the contraction output it anchors on)
ROWS = [(KKT_GATED, "gdn", "Araw"), (CHUNK_O_GATED, "gdn", "Aqk"), (QK_PROLOGUE, "kda", "Aqk")]


def _prog(family, dims=DIMS):
    return canonicalize(BUILD[family](*dims, dims[-1] ** -0.5))


def _anchor(program, out):
    (i,) = [i for i, n in enumerate(program.nodes) if isinstance(n, EinsumNode) and n.output == out]
    return i


def _fused(program):
    return [n for n in program.nodes if isinstance(n, FusedNode)]


@pytest.mark.parametrize("row,family,out", ROWS, ids=[r[0].name for r in ROWS])
def test_each_row_matches_only_its_own_contraction(row, family, out):
    for fam in BUILD:
        prog = _prog(fam)
        flow = Dataflow(prog)
        hits = [n.output for n in (flow.nodes[i] for i in flow.find(
            lambda n: isinstance(n, EinsumNode))) if row.matches(
                extract_epilogue_unit(prog, _anchor(prog, n.output)))]
        assert hits == ([out] if fam == family else []), (row.name, fam)


def test_rows_are_mutually_exclusive():
    """No contraction of either forward is claimed by two rows (the matcher takes the first)."""
    for fam in BUILD:
        prog = _prog(fam)
        for i, n in enumerate(prog.nodes):
            if isinstance(n, EinsumNode):
                unit = extract_epilogue_unit(prog, i)
                assert sum(t.matches(unit) for t in default_templates()) <= 1


@pytest.mark.parametrize("row,family,out", ROWS, ids=[r[0].name for r in ROWS])
def test_emitted_node_follows_the_row(row, family, out):
    B, H, nc, C, D = DIMS
    prog = _prog(family)
    res = FuseContractionEpilogue(*DIMS).apply(prog)
    unit = extract_epilogue_unit(prog, _anchor(prog, out))
    (node,) = [n for n in _fused(res.program) if n.kernel in row.kernels]
    assert node.kernel == row.kernels[1]                    # C·D = 8192 picks the v2 key
    assert node.inputs == list(row.inputs)
    assert node.outputs == [unit.boundary_out]
    assert node.params["nc"] * node.params["H"] == B * H * nc
    assert (node.params["C"], node.params["D"]) == (C, D)
    for k, v in row.params:
        assert node.params[k] == v
    # the absorbed steps are gone, nothing else is
    absorbed = row.absorbed(Dataflow(prog), unit)
    gone = {n.output for i, n in enumerate(prog.nodes) if i in absorbed}
    left = {getattr(n, "output", None) for n in res.program.nodes}
    assert not (gone - {unit.boundary_out}) & left
    assert unit.boundary_out in {o for n in _fused(res.program) for o in n.outputs}


def test_small_tiles_take_the_plain_key():
    small = (1, 2, 2, 16, 64)                               # C·D = 1024
    for family in BUILD:
        keys = {n.kernel for n in _fused(FuseContractionEpilogue(*small).apply(
            _prog(family, small)).program)}
        assert keys and not any(k.endswith("_v2") for k in keys)


def test_every_emitted_key_is_registered():
    keys = set(default_fused_registry().keys())
    for t in default_templates():
        assert set(t.kernels) <= keys
    for flash in (FuseChunkOFlash, FusePerDimChunkOFlash):
        assert flash.spec.kernel in keys


def test_prescaled_right_operand_is_absorbed_left_stays():
    """KDA's k ⊙ invP feeds only the score and goes into the kernel; q ⊙ P also feeds the
    inter-chunk term and must stay."""
    prog = _prog("kda")
    out = FuseContractionEpilogue(*DIMS).apply(prog).program
    names = {getattr(n, "output", None) for n in out.nodes}
    assert "k_eff" not in names and "q_eff" in names


@pytest.mark.parametrize("flash,family", [(FuseChunkOFlash, "gdn"),
                                          (FusePerDimChunkOFlash, "kda")])
def test_flash_takes_score_and_apply(flash, family):
    prog = _prog(family)
    other = "kda" if family == "gdn" else "gdn"
    t = flash(*DIMS)
    assert t.match(prog) == 1 and t.match(_prog(other)) == 0
    flow = Dataflow(prog)
    apply_idx = flow.sole_reader(extract_epilogue_unit(prog, _anchor(prog, "Aqk")).boundary_out)
    apply = prog.nodes[apply_idx]
    res = t.apply(prog).program
    (node,) = [n for n in _fused(res) if n.kernel == t.spec.kernel]
    assert node.outputs == [apply.output]
    assert node.inputs[len(t.spec.inputs)] == apply.inputs[1]      # v is the apply's operand
    assert node.params["causal"] is True
    assert not any(isinstance(n, EinsumNode) and n.output in ("Aqk", apply.output)
                   for n in res.nodes)
    assert t.match(res) == 0


def test_a_new_row_is_a_new_kernel():
    """A template row of one's own makes the generator fire on a program it did not know."""
    nodes = [EinsumNode("nid,njd->nij", ["x", "y"], "s"),
             VecGlueNode("mul", ["s", "w"], "sw"),
             TensorOp("contiguous", ["sw"], "S"),
             VecGlueNode("add", ["S", "S"], "out")]
    prog = canonicalize(Program(nodes, ["x", "y", "w"], ["out"]))
    row = ScoreTemplate(name="toy", family="toy", operands=("x", "y"),
                        epilogue=("mul", "contiguous"), gate="w", kernels=("toy", "toy_v2"),
                        inputs=("x", "y", "w"), absorbs="toy")
    assert FuseContractionEpilogue(1, 1, 1, 16, 16).match(prog) == 0
    t = FuseContractionEpilogue(1, 1, 1, 16, 16, templates=[row])
    res = t.apply(prog)
    assert res.sites == 1 and [n.kernel for n in _fused(res.program)] == ["toy"]
    assert [type(n).__name__ for n in res.program.nodes] == ["FusedNode", "VecGlueNode"]
    assert _fused(res.program)[0].outputs == ["S"]


def test_a_gate_mismatch_is_not_matched():
    nodes = [EinsumNode("nid,njd->nij", ["x", "y"], "s"),
             VecGlueNode("mul", ["s", "other"], "sw"),
             TensorOp("contiguous", ["sw"], "S")]
    prog = Program(nodes, ["x", "y", "other"], ["S"])
    row = ScoreTemplate(name="toy", family="toy", operands=("x", "y"),
                        epilogue=("mul", "contiguous"), gate="w", kernels=("toy", "toy_v2"),
                        inputs=("x", "y", "w"))
    assert FuseContractionEpilogue(1, 1, 1, 16, 16, templates=[row]).match(prog) == 0


def test_report_agrees_with_the_generator():
    for family in BUILD:
        prog = _prog(family)
        rows = epilogue_report(prog).rows
        einsums = sum(isinstance(n, EinsumNode) for n in prog.nodes)
        assert len(rows) == einsums
        hits = [r for r in rows if r[2].startswith("template ")]
        assert len(hits) == FuseContractionEpilogue(*DIMS).match(prog) > 0
        assert all(r[2] == "staged (no template)" for r in rows if r not in hits)
        assert f"{len(hits)} of {einsums}" in str(epilogue_report(prog))
