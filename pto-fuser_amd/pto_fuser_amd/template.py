"""Template emission: a contraction plus the glue around it -> one stage kernel
(src/pto_fuser/template.py:1-436).

For each contraction the generator extracts its *epilogue unit* — the einsum, the chain of
single-consumer glue after it (mul / scale / tril / contiguous) and the per-operand ``mul``
prescales before it — and matches it against templates, each backed by a HIP kernel that is
parity-tested on the GPU.  A contraction no template matches stays staged.

Templates (all run ``pf_gated_qk_exec``):
  kkt-gated-native      A = tril((kF·kFᵀ) ⊙ coefA, -1)              -> kkt_gated_native[_v2]
  chunk-o-gated-native  Aqk = (qF·kFᵀ) ⊙ coef_o                      -> gated_qk_native[_v2]
  qk-prologue           tril((qF ⊙ coef_ag)·(kF ⊙ coef_bg)ᵀ)         -> qk_prologue[_v2]
and two standalone score-to-output transforms (``pf_qkv_flash_exec``):
  FuseChunkOFlash        Aqk chain + the o_intra contraction         -> qkv_flash_native_v2
  FusePerDimChunkOFlash  per-channel Aqk chain + o_intra             -> qkvp_flash_native_v2

Shape parameters.  The reference emits ``{"nc": nc, "H": H}`` for the scalar templates, which
its launch turns into M = nc·H chunks with the default C = D = 128 — correct only at B = 1 and
C = 128 (its templates are exercised only there).  Here every template emits ``H = B·H`` (the
number of chains, so M = B·H·nc), ``C`` and ``D``: the nodes are correct at any batch.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

from .ir import EinsumNode, FusedNode, Program, TensorOp, VecGlueNode
from .transform import Transform, TransformResult, producer_index, splice
from .transforms.chunked import select_prologue_kernel

__all__ = ["EpilogueUnit", "extract_epilogue_unit", "Dims", "Template", "GatedKKTTemplate",
           "GatedChunkOTemplate", "PerDimPrologueTemplate", "default_templates",
           "FuseContractionEpilogue", "FuseChunkOFlash", "FusePerDimChunkOFlash",
           "EpilogueReport", "epilogue_report"]


@dataclass
class EpilogueUnit:
    """A contraction and the glue a stage kernel could absorb around it.  ``epilogue``: the
    (index, node) chain after the einsum; ``prologue``: operand -> (index of the ``mul`` that
    produced it, its inputs); ``boundary_out``: the name the rest of the program consumes."""
    anchor_idx: int
    anchor: EinsumNode
    epilogue: List[Tuple[int, object]]
    prologue: Dict[str, Tuple[int, List[str]]]
    boundary_out: str

    @property
    def epilogue_ops(self) -> List[str]:
        return [n.op for _, n in self.epilogue]


def _only_consumer(program: Program, name: str) -> Optional[int]:
    hits = [i for i, n in enumerate(program.nodes) if name in n.inputs]
    return hits[0] if len(hits) == 1 else None


def extract_epilogue_unit(program: Program, anchor_idx: int) -> EpilogueUnit:
    anchor = program.nodes[anchor_idx]
    epilogue: List[Tuple[int, object]] = []
    cur = anchor.output
    while True:
        c = _only_consumer(program, cur)
        if c is None:
            break
        n = program.nodes[c]
        absorbable = ((isinstance(n, VecGlueNode) and n.op in ("mul", "scale", "tril")) or
                      (isinstance(n, TensorOp) and n.op == "contiguous"))
        if not absorbable:
            break
        epilogue.append((c, n))
        cur = n.output
    prod = producer_index(program)
    prologue: Dict[str, Tuple[int, List[str]]] = {}
    for operand in anchor.inputs:
        p = prod.get(operand)
        if p is not None:
            pn = program.nodes[p]
            if isinstance(pn, VecGlueNode) and pn.op == "mul":
                prologue[operand] = (p, list(pn.inputs))
    return EpilogueUnit(anchor_idx, anchor, epilogue, prologue, cur)


@dataclass
class Dims:
    B: int
    H: int
    nc: int
    C: int
    D: int
    v2: Optional[bool] = None

    @property
    def N(self) -> int:
        return self.B * self.H

    def params(self, **extra) -> dict:
        return {"nc": self.nc, "H": self.N, "C": self.C, "D": self.D, **extra}


class Template:
    name: str = "template"
    family: str = ""

    def matches(self, program: Program, unit: EpilogueUnit) -> bool:   # pragma: no cover
        raise NotImplementedError

    def emit(self, program: Program, unit: EpilogueUnit, dims: Dims) -> Tuple[FusedNode, set]:
        raise NotImplementedError                                        # pragma: no cover


def _glue_operand(unit: EpilogueUnit, op: str) -> Optional[str]:
    """The operand of the first ``op`` glue of the epilogue that is not the chain itself."""
    chain = {unit.anchor.output} | {n.output for _, n in unit.epilogue}
    for _, n in unit.epilogue:
        if isinstance(n, VecGlueNode) and n.op == op:
            others = [x for x in n.inputs if x not in chain]
            return others[0] if others else None
    return None


def _unit_drop(unit: EpilogueUnit) -> set:
    return {unit.anchor_idx} | {i for i, _ in unit.epilogue}


class GatedKKTTemplate(Template):
    """kkt: ``A = tril((kF·kFᵀ) ⊙ coefA, -1)``; the gate is recomputed from g_native and
    beta_native inside the kernel, the score never reaches HBM."""
    name = "kkt-gated-native"
    family = "scalar-gate"

    def matches(self, program, unit) -> bool:
        a, b = unit.anchor.inputs
        return (unit.anchor.equation == "nid,njd->nij" and a == b == "kF"
                and unit.epilogue_ops == ["mul", "tril", "contiguous"])

    def emit(self, program, unit, dims):
        node = FusedNode(kernel="kkt_gated_native_v2" if dims.v2 else "kkt_gated_native",
                         inputs=["kF", "g_native", "beta_native"], outputs=[unit.boundary_out],
                         params=dims.params(),
                         subsumes=["kkt einsum + coefA mul + tril (score kept on chip)"])
        return node, _unit_drop(unit)


class GatedChunkOTemplate(Template):
    """chunk_o score: ``Aqk = (qF·kFᵀ) ⊙ coef_o`` (causal incl. diagonal, beta = 1)."""
    name = "chunk-o-gated-native"
    family = "scalar-gate"

    def matches(self, program, unit) -> bool:
        a, b = unit.anchor.inputs
        return (unit.anchor.equation == "nid,njd->nij" and a == "qF" and b == "kF"
                and unit.epilogue_ops == ["mul", "contiguous"]
                and _glue_operand(unit, "mul") == "coef_o")

    def emit(self, program, unit, dims):
        node = FusedNode(kernel="gated_qk_native_v2" if dims.v2 else "gated_qk_native",
                         inputs=["qF", "kF", "g_native", "beta_native_ones"],
                         outputs=[unit.boundary_out], params=dims.params(causal=True),
                         subsumes=["chunk_o Aqk einsum + coef_o mul + contiguous"])
        return node, _unit_drop(unit)


class PerDimPrologueTemplate(Template):
    """KDA chunk_o score: ``tril((qF ⊙ coef_ag)·(kF ⊙ coef_bg)ᵀ)``; the operand prescales are
    applied while the tiles are staged into LDS.  ``q_eff`` stays (it also feeds o_inter);
    ``k_eff`` is dropped when this unit is its only reader."""
    name = "qk-prologue"
    family = "per-dim-prologue"

    def matches(self, program, unit) -> bool:
        a, b = unit.anchor.inputs
        pa, pb = unit.prologue.get(a), unit.prologue.get(b)
        return bool(pa and pb and unit.anchor.equation == "nid,njd->nij"
                    and pa[1] == ["qF", "coef_ag"] and pb[1] == ["kF", "coef_bg"]
                    and unit.epilogue_ops == ["tril", "contiguous"])

    def emit(self, program, unit, dims):
        if dims.v2 is None:
            kernel = select_prologue_kernel(dims.C, dims.D)
        else:
            kernel = "qk_prologue_v2" if dims.v2 else "qk_prologue"
        node = FusedNode(kernel=kernel, inputs=["qF", "kF", "coef_ag", "coef_bg"],
                         outputs=[unit.boundary_out], params=dims.params(),
                         subsumes=["chunk_o k_eff mul + Aqk einsum + tril + contiguous"])
        drop = _unit_drop(unit)
        kmul = unit.prologue[unit.anchor.inputs[1]][0]
        if _only_consumer(program, program.nodes[kmul].output) == unit.anchor_idx:
            drop.add(kmul)
        return node, drop


def default_templates() -> List[Template]:
    """In match-priority order."""
    return [GatedKKTTemplate(), GatedChunkOTemplate(), PerDimPrologueTemplate()]


class FuseContractionEpilogue(Transform):
    """Emit every contraction whose epilogue unit a template matches."""
    name = "fuse-contraction-epilogue"
    summary = "contraction + epilogue glue -> gated-score stage kernel (template)"

    def __init__(self, B, H, nc, C, D, v2: Optional[bool] = None,
                 templates: Optional[List[Template]] = None) -> None:
        self.dims = Dims(B, H, nc, C, D, v2)
        self.templates = templates if templates is not None else default_templates()

    def _hits(self, program: Program) -> List[Tuple[int, Template]]:
        out = []
        for i, n in enumerate(program.nodes):
            if isinstance(n, EinsumNode):
                unit = extract_epilogue_unit(program, i)
                t = next((t for t in self.templates if t.matches(program, unit)), None)
                if t is not None:
                    out.append((i, t))
        return out

    def match(self, program: Program) -> int:
        return len(self._hits(program))

    def apply(self, program: Program) -> TransformResult:
        fired, prog = [], program
        while True:                       # indices shift after each splice: re-scan
            hits = self._hits(prog)
            if not hits:
                break
            i, t = hits[0]
            node, drop = t.emit(prog, extract_epilogue_unit(prog, i), self.dims)
            prog = splice(prog, drop, min(drop), [node])
            fired.append(t.name)
        return TransformResult(prog, bool(fired), len(fired),
                               "emitted: " + (", ".join(fired) if fired else "none"))


class _ChunkOFlashBase(Transform):
    """The chunk_o score -> output chain (score einsum, its epilogue, the ``nij,nje->nie``
    contraction with v_new) replaced by one flash kernel; the score stays in LDS."""
    kernel = ""

    def __init__(self, B, H, nc, C, D) -> None:
        self.dims = Dims(B, H, nc, C, D)

    def _unit_ok(self, program: Program, unit: EpilogueUnit) -> bool:   # pragma: no cover
        raise NotImplementedError

    def _inputs(self, v_name: str) -> List[str]:                       # pragma: no cover
        raise NotImplementedError

    def _site(self, program: Program):
        for i, n in enumerate(program.nodes):
            if not (isinstance(n, EinsumNode) and n.equation == "nid,njd->nij"):
                continue
            unit = extract_epilogue_unit(program, i)
            if not self._unit_ok(program, unit):
                continue
            c = _only_consumer(program, unit.boundary_out)
            if c is None:
                continue
            cn = program.nodes[c]
            if (isinstance(cn, EinsumNode) and cn.equation == "nij,nje->nie"
                    and cn.inputs[0] == unit.boundary_out):
                return i, unit, c
        return None

    def match(self, program: Program) -> int:
        return 1 if self._site(program) is not None else 0

    def _extra_drop(self, program: Program, unit: EpilogueUnit) -> set:
        return set()

    def apply(self, program: Program) -> TransformResult:
        site = self._site(program)
        if site is None:
            return TransformResult(program, False, 0, "no chunk_o score -> output chain")
        i, unit, c = site
        o_intra = program.nodes[c]
        node = FusedNode(kernel=self.kernel, inputs=self._inputs(o_intra.inputs[1]),
                         outputs=[o_intra.output],
                         params=self.dims.params(DV=self.dims.D, causal=True),
                         subsumes=["chunk_o score einsum + epilogue + o_intra A·v "
                                   "(score kept in LDS)"])
        drop = _unit_drop(unit) | {c} | self._extra_drop(program, unit)
        return TransformResult(splice(program, drop, min(drop), [node]), True, 1,
                               f"emitted {self.kernel}")


class FuseChunkOFlash(_ChunkOFlashBase):
    """GDN chunk_o: ``Aqk = (qF·kFᵀ) ⊙ coef_o`` -> contiguous -> ``Aqk·v_new``."""
    name = "fuse-chunk-o-flash"
    summary = "chunk_o q·kᵀ -> gate/mask -> ·v as one qkv_flash_native_v2 (score in LDS)"
    kernel = "qkv_flash_native_v2"

    def _unit_ok(self, program, unit) -> bool:
        return (unit.anchor.inputs == ["qF", "kF"] and unit.epilogue_ops == ["mul", "contiguous"]
                and _glue_operand(unit, "mul") == "coef_o")

    def _inputs(self, v_name):
        return ["qF", "kF", v_name, "g_native", "beta_native_ones"]


class FusePerDimChunkOFlash(_ChunkOFlashBase):
    """KDA chunk_o: ``tril((qF ⊙ coef_ag)·(kF ⊙ coef_bg)ᵀ)`` -> contiguous -> ``·v_new``."""
    name = "fuse-perdim-chunk-o-flash"
    summary = "per-channel chunk_o prescale·q·kᵀ -> tril -> ·v as one qkvp_flash_native_v2"
    kernel = "qkvp_flash_native_v2"

    def _unit_ok(self, program, unit) -> bool:
        a, b = unit.anchor.inputs
        pa, pb = unit.prologue.get(a), unit.prologue.get(b)
        return bool(pa and pb and pa[1] == ["qF", "coef_ag"] and pb[1] == ["kF", "coef_bg"]
                    and unit.epilogue_ops == ["tril", "contiguous"])

    def _inputs(self, v_name):
        return ["qF", "kF", v_name, "coef_ag", "coef_bg"]

    def _extra_drop(self, program, unit) -> set:
        kmul = unit.prologue[unit.anchor.inputs[1]][0]
        return {kmul} if _only_consumer(program, program.nodes[kmul].output) == unit.anchor_idx \
            else set()


@dataclass
class EpilogueReport:
    rows: List[Tuple[str, str, str]] = field(default_factory=list)

    def __str__(self) -> str:
        lines = ["contraction-epilogue units (template = parity-tested stage kernel):"]
        for anchor, epi, verdict in self.rows:
            lines.append(f"  {anchor:<12} epilogue[{epi:<22}] -> {verdict}")
        matched = sum(v.startswith("template ") for _, _, v in self.rows)
        lines.append(f"  -- {matched}/{len(self.rows)} contractions match a template; the rest "
                     f"stay staged")
        return "\n".join(lines)


def epilogue_report(program: Program, templates: Optional[List[Template]] = None) -> EpilogueReport:
    """Which template emits each contraction, or why it stays staged (structural only)."""
    templates = templates if templates is not None else default_templates()
    rep = EpilogueReport()
    for i, n in enumerate(program.nodes):
        if not isinstance(n, EinsumNode):
            continue
        unit = extract_epilogue_unit(program, i)
        t = next((t for t in templates if t.matches(program, unit)), None)
        rep.rows.append((n.output, "+".join(unit.epilogue_ops) or "(none)",
                         f"template {t.name}" if t else "staged (no matching template)"))
    return rep
