"""Rewrite machinery and the structural transforms (no device).

The dataflow view and the edit buffer first (they carry every rewrite), then the transforms as a
table: each names the forward it applies to and how many sites it finds there; for all of them
the same properties must hold — no site in the other forward, none left after ``apply``
(idempotence), a valid program with the same inputs and outputs, and every emitted kernel key
registered.  Policy ordering closes the file."""
import pytest

from pto_fuser_amd import (Dataflow, EinsumNode, EnableDirectReads, EnableFusedStore, Features,
                           FuseChunkOFlash, FusedNode, FuseContractionEpilogue,
                           FusePerDimChunkOFlash, Policy, Program, ProgramEdit, TensorOp,
                           VecGlueNode, canonicalize, default_fused_registry)
from pto_fuser_amd.forwards import build_gdn_program, build_kda_program
from pto_fuser_amd.policy import STAGES
from pto_fuser_amd.transforms import (FuseGdnForward, FuseKdaForward, LowerPerDimScan,
                                      LowerResidentScan)

DIMS = (2, 2, 3, 64, 128)
BUILD = {"gdn": build_gdn_program, "kda": build_kda_program}


def _prog(family):
    return canonicalize(BUILD[family](*DIMS, DIMS[-1] ** -0.5))


def _toy():
    """x -> a = x·y -> b = tril(a) -> c = b·z ; d = a + a."""
    return Program([EinsumNode("nid,njd->nij", ["x", "y"], "a"),
                    VecGlueNode("tril", ["a"], "b"),
                    EinsumNode("nij,nje->nie", ["b", "z"], "c"),
                    VecGlueNode("add", ["c", "c"], "d")], ["x", "y", "z"], ["d"])


# ---- Dataflow ---------------------------------------------------------------------------------
def test_dataflow_indices():
    f = Dataflow(_toy())
    assert f.producer("a") == 0 and f.producer("x") is None
    assert f.readers("a") == [1] and f.readers("c") == [3, 3]
    assert f.sole_reader("a") == 1 and f.sole_reader("c") is None
    assert f.binds("x") and f.binds("d") and not f.binds("nope")
    assert f.find(lambda n: isinstance(n, EinsumNode)) == [0, 2]
    assert f.outputs_of([0, 2]) == ["a", "c"]


def test_dataflow_chain_stops_at_fanout_and_rejection():
    f = Dataflow(_toy())
    assert f.chain("a", lambda n: True) == [1, 2]          # c has two reads -> stop
    assert f.chain("a", lambda n: isinstance(n, VecGlueNode)) == [1]


# ---- ProgramEdit ------------------------------------------------------------------------------
def test_edit_replace_keeps_order_and_original_indices():
    p = _toy()
    edit = ProgramEdit(p)
    edit.replace([0, 1], [EinsumNode("nid,njd->nij", ["x", "y"], "b")])
    edit.insert(len(p.nodes), [TensorOp("contiguous", ["d"], "e")])
    out = edit.build()
    assert [getattr(n, "output", None) for n in out.nodes] == ["b", "c", "d", "e"]
    assert out.inputs == p.inputs and out.outputs == p.outputs
    assert edit.removed == frozenset({0, 1})
    assert [getattr(n, "output", None) for n in p.nodes] == ["a", "b", "c", "d"]   # untouched


def test_edit_rejects_bad_indices_and_broken_dataflow():
    p = _toy()
    with pytest.raises(IndexError):
        ProgramEdit(p).remove(4)
    with pytest.raises(ValueError):
        ProgramEdit(p).replace([], [])
    with pytest.raises(ValueError, match="reads 'b'"):
        ProgramEdit(p).remove(1).build()                 # c still reads the dropped b


# ---- canonical form and annotation levers ------------------------------------------------------
def test_canonicalize_is_idempotent_and_pure():
    raw = BUILD["gdn"](*DIMS, 0.1)
    c1 = canonicalize(raw)
    assert canonicalize(c1) == c1
    assert all(n.read_mode == "NN" and not n.fuse_out
               for n in c1.nodes if isinstance(n, EinsumNode))
    assert raw.nodes is not c1.nodes


@pytest.mark.parametrize("lever,field,value", [(EnableDirectReads, "read_mode", "auto"),
                                               (EnableFusedStore, "fuse_out", True)])
def test_annotation_lever(lever, field, value):
    prog = _prog("gdn")
    n_einsum = sum(isinstance(n, EinsumNode) for n in prog.nodes)
    t = lever()
    assert t.match(prog) == n_einsum and t.stage == "annotation"
    res = t.apply(prog)
    assert res.changed and res.sites == n_einsum and field in res.note
    assert all(getattr(n, field) == value for n in res.program.nodes if isinstance(n, EinsumNode))
    again = t.apply(res.program)
    assert not again.changed and again.program is res.program


# ---- structural transforms, as a table -------------------------------------------------------
TABLE = [  # (factory, family, sites in that family, kernels it emits)
    (lambda: LowerResidentScan(*DIMS), "gdn", 1, {"chunk_h_scan"}),
    (lambda: LowerPerDimScan(*DIMS), "kda", 1, {"chunk_h_scan"}),
    (lambda: FuseChunkOFlash(*DIMS), "gdn", 1, {"qkv_flash_native_v2"}),
    (lambda: FusePerDimChunkOFlash(*DIMS), "kda", 1, {"qkvp_flash_native_v2"}),
    (lambda: FuseGdnForward(*DIMS), "gdn", 1, {"gdn_forward"}),
    (lambda: FuseKdaForward(*DIMS), "kda", 1, {"kda_forward"}),
]
IDS = ["resident-scan", "perdim-scan", "chunk-o-flash", "perdim-flash", "gdn-whole", "kda-whole"]


@pytest.mark.parametrize("make,family,sites,kernels", TABLE, ids=IDS)
def test_structural_transform_properties(make, family, sites, kernels):
    t = make()
    prog, other = _prog(family), _prog("kda" if family == "gdn" else "gdn")
    assert t.match(prog) == sites and t.match(other) == 0
    assert t.stage in STAGES
    res = t.apply(prog)
    assert res.changed and res.sites == sites
    assert res.program.inputs == prog.inputs and res.program.outputs == prog.outputs
    emitted = {n.kernel for n in res.program.nodes if isinstance(n, FusedNode)}
    assert emitted == kernels
    assert emitted <= set(default_fused_registry().keys())
    assert t.match(res.program) == 0                      # idempotent
    assert len(res.program.nodes) < len(prog.nodes)
    assert not t.apply(other).changed


def test_perdim_scan_flags_the_decay_shape():
    def scan_params(prog):
        (n,) = [n for n in prog.nodes if isinstance(n, FusedNode) and n.kernel == "chunk_h_scan"]
        return n.params
    assert scan_params(LowerPerDimScan(*DIMS).apply(_prog("kda")).program)["perdim_decay"]
    assert "perdim_decay" not in scan_params(LowerResidentScan(*DIMS).apply(_prog("gdn")).program)


def test_rewrites_compose_on_both_forwards():
    for family, tail in (("gdn", {"kkt_gated_native_v2"}), ("kda", set())):
        prog = _prog(family)
        scan = LowerResidentScan(*DIMS) if family == "gdn" else LowerPerDimScan(*DIMS)
        flash = FuseChunkOFlash(*DIMS) if family == "gdn" else FusePerDimChunkOFlash(*DIMS)
        for t in (scan, flash, FuseContractionEpilogue(*DIMS)):
            prog = t.apply(prog).program
        keys = {n.kernel for n in prog.nodes if isinstance(n, FusedNode)}
        assert keys == {"chunk_h_scan", flash.spec.kernel} | tail
        assert prog.outputs == ["o"]


# ---- policy ---------------------------------------------------------------------------------
def test_policy_orders_by_stage_and_drops_non_matching():
    f = Features(*DIMS)
    plan = Policy().pipeline(_prog("gdn"), f)
    stages = [STAGES.index(p.transform.stage) for p in plan]
    assert stages == sorted(stages)
    names = [p.name for p in plan]
    assert "lower-perdim-scan" not in names and "fuse-perdim-chunk-o-flash" not in names
    assert names.index("fuse-chunk-o-flash") < names.index("fuse-contraction-epilogue")
    assert not any(p.transform.stage == "whole" for p in plan)
    whole = Policy(whole_forward=True).pipeline(_prog("gdn"), f)
    assert whole[0].name == FuseGdnForward(*DIMS).name
