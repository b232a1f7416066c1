"""Template emission (no device): epilogue-unit extraction, template matching, the generator,
the chunk_o flash transforms and the report (reference tests/test_template.py)."""
from pto_fuser_amd import (EinsumNode, FuseChunkOFlash, FusedNode, FuseContractionEpilogue,
                           FusePerDimChunkOFlash, canonicalize, epilogue_report,
                           extract_epilogue_unit)
from pto_fuser_amd.forwards import build_gdn_program, build_kda_program
from pto_fuser_amd.template import (GatedChunkOTemplate, GatedKKTTemplate, PerDimPrologueTemplate,
                                    default_templates)


def _gdn():
    return canonicalize(build_gdn_program(1, 4, 2, 128, 128, 128 ** -0.5))


def _kda():
    return canonicalize(build_kda_program(1, 4, 2, 128, 128, 128 ** -0.5))


def _idx(program, out):
    return next(i for i, n in enumerate(program.nodes)
                if isinstance(n, EinsumNode) and n.output == out)


def test_extract_kkt_epilogue_unit():
    prog = _gdn()
    unit = extract_epilogue_unit(prog, _idx(prog, "Araw"))
    assert unit.epilogue_ops == ["mul", "tril", "contiguous"]
    assert unit.boundary_out == "A" and unit.anchor.inputs == ["kF", "kF"]


def test_extract_kda_prologue():
    prog = _kda()
    unit = extract_epilogue_unit(prog, _idx(prog, "Aqk"))
    assert unit.epilogue_ops == ["tril", "contiguous"]
    assert set(unit.prologue) == {"q_eff", "k_eff"}


def test_templates_match_their_own_pattern():
    gdn, kda = _gdn(), _kda()
    kkt = extract_epilogue_unit(gdn, _idx(gdn, "Araw"))
    aqk = extract_epilogue_unit(gdn, _idx(gdn, "Aqk"))
    pro = extract_epilogue_unit(kda, _idx(kda, "Aqk"))
    assert GatedKKTTemplate().matches(gdn, kkt) and not GatedKKTTemplate().matches(gdn, aqk)
    assert GatedChunkOTemplate().matches(gdn, aqk) and not GatedChunkOTemplate().matches(gdn, kkt)
    assert PerDimPrologueTemplate().matches(kda, pro)
    assert not PerDimPrologueTemplate().matches(gdn, kkt)


def test_generator_emits_expected_nodes():
    prog = FuseContractionEpilogue(1, 4, 2, 128, 128, v2=False).apply(_gdn()).program
    fused = {n.kernel: n for n in prog.nodes if isinstance(n, FusedNode)}
    assert set(fused) == {"kkt_gated_native", "gated_qk_native"}
    assert fused["kkt_gated_native"].inputs == ["kF", "g_native", "beta_native"]
    assert fused["kkt_gated_native"].outputs == ["A"]
    assert fused["gated_qk_native"].inputs == ["qF", "kF", "g_native", "beta_native_ones"]
    assert fused["gated_qk_native"].outputs == ["Aqk_c"]
    assert fused["gated_qk_native"].params.get("causal") is True
    v2 = FuseContractionEpilogue(1, 4, 2, 128, 128, v2=True).apply(_gdn()).program
    assert {n.kernel for n in v2.nodes if isinstance(n, FusedNode)} == \
        {"kkt_gated_native_v2", "gated_qk_native_v2"}


def test_report_matches_two_and_flags_the_rest():
    verdicts = {a: v for a, _, v in epilogue_report(_gdn()).rows}
    assert verdicts["Araw"] == "template kkt-gated-native"
    assert verdicts["Aqk"] == "template chunk-o-gated-native"
    assert verdicts["o_inter_m"] == "staged (no matching template)"
    assert sum(v.startswith("template ") for v in verdicts.values()) == 2


def test_generator_never_emits_without_a_template():
    prog = FuseContractionEpilogue(1, 4, 2, 128, 128).apply(_gdn()).program
    assert any(isinstance(n, EinsumNode) and n.output == "o_inter_m" for n in prog.nodes)


def test_default_templates_are_registered():
    assert {t.name for t in default_templates()} == \
        {"kkt-gated-native", "chunk-o-gated-native", "qk-prologue"}


def test_prologue_kernel_shape_gate():
    kda = FuseContractionEpilogue(1, 4, 2, 128, 128).apply(_kda()).program
    pro = [n for n in kda.nodes if isinstance(n, FusedNode)]
    assert len(pro) == 1 and pro[0].kernel == "qk_prologue_v2"        # C·D = 16384
    assert pro[0].inputs == ["qF", "kF", "coef_ag", "coef_bg"] and pro[0].outputs == ["Aqk_c"]
    small = canonicalize(build_kda_program(1, 4, 2, 16, 64, 0.125))
    pro = [n for n in FuseContractionEpilogue(1, 4, 2, 16, 64).apply(small).program.nodes
           if isinstance(n, FusedNode)]
    assert pro[0].kernel == "qk_prologue"                             # C·D = 1024


def test_chunk_o_flash_transform():
    gdn = _gdn()
    t = FuseChunkOFlash(1, 4, 2, 128, 128)
    assert t.match(gdn) == 1 and t.match(_kda()) == 0
    prog = t.apply(gdn).program
    flash = [n for n in prog.nodes if isinstance(n, FusedNode) and n.kernel == "qkv_flash_native_v2"]
    assert len(flash) == 1
    assert flash[0].outputs == ["o_intra"] and flash[0].params.get("causal") is True
    assert flash[0].inputs == ["qF", "kF", "vn_flat", "g_native", "beta_native_ones"]
    assert not any(isinstance(n, EinsumNode) and n.output in ("Aqk", "o_intra") for n in prog.nodes)
    assert t.match(prog) == 0


def test_perdim_chunk_o_flash_transform():
    kda = _kda()
    t = FusePerDimChunkOFlash(1, 4, 2, 128, 128)
    assert t.match(kda) == 1 and t.match(_gdn()) == 0
    prog = t.apply(kda).program
    flash = [n for n in prog.nodes if isinstance(n, FusedNode)
             and n.kernel == "qkvp_flash_native_v2"]
    assert len(flash) == 1 and flash[0].outputs == ["o_intra"]
    assert flash[0].inputs == ["qF", "kF", "vn_flat", "coef_ag", "coef_bg"]
    outs = {getattr(n, "output", None) for n in prog.nodes}
    assert "k_eff" not in outs and "q_eff" in outs
    assert t.match(prog) == 0
