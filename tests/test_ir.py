"""IR structure (no device): dataflow validation, multi-output fused nodes, builders' contracts
(reference tests/test_ir.py and tests/test_fusion.py structural parts)."""
import pytest
import torch

from pto_fuser_amd import (EinsumNode, FusedNode, OpaqueNode, Program, TensorOp, VecGlueNode,
                           default_fused_registry)
from pto_fuser_amd.forwards import (build_deltanet_program, build_gdn_program, build_kda_program,
                                    build_kkt_fused_program, build_scan_fused_program,
                                    build_scan_staged_program, make_gdn_inputs, make_kda_inputs,
                                    prepare_gdn_bindings, prepare_kda_bindings)
from pto_fuser_amd.ir import node_outputs


def test_program_validates_dataflow():
    prog = Program([EinsumNode("ij,jk->ik", ["a", "b"], "c"),
                    VecGlueNode("scale", ["c"], "d", params={"scalar": 0.5})],
                   inputs=["a", "b"], outputs=["d"])
    assert prog.outputs == ["d"]


def test_use_before_def_raises():
    with pytest.raises(ValueError, match="before it is produced"):
        Program([EinsumNode("ij,jk->ik", ["a", "missing"], "c")], inputs=["a", "b"], outputs=["c"])


def test_undeclared_output_raises():
    with pytest.raises(ValueError, match="never produced"):
        Program([EinsumNode("ij,jk->ik", ["a", "b"], "c")], inputs=["a", "b"], outputs=["nope"])


def test_fused_node_is_multi_output():
    n = FusedNode(kernel="chunk_h_scan", inputs=["w", "u", "k", "decay"],
                  outputs=["h_out", "final"], params={"B": 1, "H": 2, "nc": 3})
    assert node_outputs(n) == ["h_out", "final"] and n.output == "h_out"
    with pytest.raises(ValueError):
        Program(nodes=[FusedNode(kernel="k", inputs=["x"], outputs=["a", "b"])],
                inputs=["x"], outputs=["a", "c"])


def test_deltanet_program_is_well_formed():
    prog = build_deltanet_program(B=1, H=2, nc=3, C=64, D=128, scale=0.1)
    assert prog.inputs == ["q", "k", "v", "beta"]
    assert prog.outputs == ["A", "T", "W", "U", "v_new", "h_state", "o"]
    assert sum(isinstance(n, OpaqueNode) for n in prog.nodes) == 1
    # kkt, W, U, 2 per chunk, o_inter, Aqk, o_intra
    assert sum(isinstance(n, EinsumNode) for n in prog.nodes) == 3 + 2 * 3 + 3


def test_full_programs_bind_their_inputs():
    """The builders' input names are exactly what the binding preparation returns."""
    B, H, nc, C, D = 1, 2, 2, 32, 64
    for make, build, prep in ((make_gdn_inputs, build_gdn_program, prepare_gdn_bindings),
                              (make_kda_inputs, build_kda_program, prepare_kda_bindings)):
        inp = make(B, H, nc, C, D)
        prog = build(B, H, nc, C, D, D ** -0.5)
        binds = prep(inp["q"], inp["k"], inp["v"], inp["beta"], inp["g_in"])
        assert prog.outputs == ["o"]
        assert sorted(prog.inputs) == sorted(binds)
        assert not any(isinstance(n, FusedNode) for n in prog.nodes)


def test_stage_programs_share_io():
    staged, fused = build_scan_staged_program(2, 4, 3), build_scan_fused_program(2, 4, 3)
    assert staged.inputs == fused.inputs == ["w", "u", "k", "decay"]
    assert staged.outputs == fused.outputs == ["h_out", "final"]
    assert len(staged.nodes) > len(fused.nodes) == 1
    kkt = build_kkt_fused_program(4, 8)
    assert isinstance(kkt.nodes[0], FusedNode) and kkt.outputs == ["L"]


def test_fused_registry_contracts():
    reg = default_fused_registry()
    scan = reg.contract("chunk_h_scan")
    assert scan.in_slots == ["w", "u", "k", "decay"] and scan.out_names == ["h_out", "final"]
    kkt = reg.contract("kkt_gated")
    assert kkt.in_slots == ["k", "g_sum", "beta"] and kkt.out_names == ["L"]
    for key in ("gated_qk", "kkt_gated_native", "kkt_gated_native_v2", "gated_qk_native",
                "gated_qk_native_v2", "qk_prologue", "qk_prologue_v2", "qkv_flash_native",
                "qkv_flash_native_v2", "qkvp_flash_native", "qkvp_flash_native_v2"):
        assert reg.contract(key).out_names in (["L"], ["o"])
    assert reg.contract("qkv_flash_native_v2").out_dtype == torch.float32
    with pytest.raises(KeyError):
        reg.kernel("nope", {})
    with pytest.raises(ValueError):
        reg.register("chunk_h_scan", None)


def test_tensorop_names_are_host_plumbing():
    prog = build_gdn_program(1, 2, 2, 32, 64, 0.125)
    ops = {n.op for n in prog.nodes if isinstance(n, TensorOp)}
    assert ops <= {"reshape", "contiguous", "transpose", "permute", "cast", "slice", "stack",
                   "zeros"}
