"""Template emission: a score contraction and the glue around it -> one HIP stage kernel.

The reference's generator (src/pto_fuser/template.py) extracts, for each contraction, the glue a
kernel could absorb and matches it against hand-written templates.  Here the templates are data:
each ``ScoreTemplate`` row names the contraction it replaces (equation, operands, optional
per-operand prescales), the epilogue signature (the ops of the single-reader chain after it),
the gate operand the epilogue multiplies by, the two registry keys of its kernel (the reference's
plain and ``_v2`` forms) and the inputs of the fused node.  One matcher and one emitter serve
every row, so adding a kernel is adding a row.

  kkt-gated-native      tril((kF kFᵀ) ⊙ coefA, -1)                   kkt_gated_native[_v2]
  chunk-o-gated-native  (qF kFᵀ) ⊙ coef_o                            gated_qk_native[_v2]
  qk-prologue           tril((qF ⊙ coef_ag)(kF ⊙ coef_bg)ᵀ)          qk_prologue[_v2]

All three run ``pf_gated_qk_exec``.  The score-to-output fusions (``FuseChunkOFlash``,
``FusePerDimChunkOFlash``) take a matched chunk_o score and the ``nij,nje->nie`` contraction that
consumes it into one ``pf_qkv_flash_exec`` launch; the score stays in LDS.

Shapes: every emitted node carries ``H = B·H`` (the number of chains), ``C`` and ``D``, so it is
correct at any batch; the reference's templates emit ``{"nc", "H"}`` only and are correct at
B = 1, C = D = 128 (its launch defaults).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

from .dataflow import Dataflow, ProgramEdit
from .ir import EinsumNode, FusedNode, Node, Program, TensorOp, VecGlueNode
from .transform import Transform

__all__ = ["EpilogueUnit", "extract_epilogue_unit", "Dims", "ScoreTemplate", "Template",
           "KKT_GATED", "CHUNK_O_GATED", "QK_PROLOGUE", "default_templates",
           "FuseContractionEpilogue", "FuseChunkOFlash", "FusePerDimChunkOFlash",
           "EpilogueReport", "epilogue_report"]

SCORE_EQ = "nid,njd->nij"        # per-chunk a bᵀ
APPLY_EQ = "nij,nje->nie"        # per-chunk score · v


def _absorbable(node: Node) -> bool:
    """Glue a stage kernel's epilogue can take over: gate / scale multiplies, the triangular
    mask, and the contiguous copy that materialises the result."""
    return ((isinstance(node, VecGlueNode) and node.op in ("mul", "scale", "tril")) or
            (isinstance(node, TensorOp) and node.op == "contiguous"))


@dataclass
class EpilogueUnit:
    """A contraction and the glue a stage kernel could absorb around it: ``epilogue`` is the
    single-reader chain after the contraction as (step index, node); ``prologue`` maps each
    operand produced by a ``mul`` to (that step's index, its inputs); ``boundary_out`` is the name
    the rest of the program reads."""
    anchor_idx: int
    anchor: EinsumNode
    epilogue: List[Tuple[int, Node]]
    prologue: Dict[str, Tuple[int, List[str]]]
    boundary_out: str

    @property
    def epilogue_ops(self) -> List[str]:
        return [n.op for _, n in self.epilogue]

    @property
    def steps(self) -> set:
        return {self.anchor_idx} | {i for i, _ in self.epilogue}

    def gate_operand(self, op: str = "mul") -> Optional[str]:
        """The operand of the first ``op`` in the epilogue that does not come from the chain."""
        chain = {self.anchor.output} | {n.output for _, n in self.epilogue}
        for _, n in self.epilogue:
            if n.op == op:
                rest = [x for x in n.inputs if x not in chain]
                return rest[0] if rest else None
        return None


def _unit(flow: Dataflow, idx: int) -> EpilogueUnit:
    anchor = flow.nodes[idx]
    chain = flow.chain(anchor.output, _absorbable)
    prologue = {}
    for operand in anchor.inputs:
        p = flow.producer(operand)
        if p is not None and isinstance(flow.nodes[p], VecGlueNode) and flow.nodes[p].op == "mul":
            prologue[operand] = (p, list(flow.nodes[p].inputs))
    out = flow.nodes[chain[-1]].output if chain else anchor.output
    return EpilogueUnit(idx, anchor, [(i, flow.nodes[i]) for i in chain], prologue, out)


def extract_epilogue_unit(program: Program, anchor_idx: int) -> EpilogueUnit:
    return _unit(Dataflow(program), anchor_idx)


@dataclass
class Dims:
    B: int
    H: int
    nc: int
    C: int
    D: int
    v2: Optional[bool] = None

    def params(self, **extra) -> dict:
        return {"nc": self.nc, "H": self.B * self.H, "C": self.C, "D": self.D, **extra}

    def use_v2(self) -> bool:
        """The ``_v2`` key unless told otherwise: chosen by the cost model from C·D (both keys
        run the same HIP kernel; the choice only keeps programs comparable with the
        reference's)."""
        return self.C * self.D >= 4096 if self.v2 is None else bool(self.v2)


@dataclass(frozen=True)
class ScoreTemplate:
    name: str
    family: str
    operands: Tuple[str, str]                 # contraction operands (or their prescale sources)
    epilogue: Tuple[str, ...]                 # op signature of the absorbed chain
    kernels: Tuple[str, str]                  # (plain, v2) registry keys
    inputs: Tuple[str, ...]                   # inputs of the emitted node
    gate: Optional[str] = None                # operand the epilogue's mul must use
    prescales: Optional[Tuple[str, str]] = None   # coefficient multiplied into each operand
    params: Tuple[Tuple[str, object], ...] = ()
    absorbs: str = ""

    def matches(self, unit: EpilogueUnit) -> bool:
        a = unit.anchor
        if a.equation != SCORE_EQ or tuple(unit.epilogue_ops) != self.epilogue:
            return False
        if self.gate is not None and unit.gate_operand("mul") != self.gate:
            return False
        if self.prescales is None:
            return tuple(a.inputs) == self.operands
        for operand, src, coef in zip(a.inputs, self.operands, self.prescales):
            pro = unit.prologue.get(operand)
            if pro is None or pro[1] != [src, coef]:
                return False
        return True

    def node(self, unit: EpilogueUnit, dims: Dims) -> FusedNode:
        return FusedNode(kernel=self.kernels[1] if dims.use_v2() else self.kernels[0],
                         inputs=list(self.inputs), outputs=[unit.boundary_out],
                         params=dims.params(**dict(self.params)), subsumes=[self.absorbs])

    def absorbed(self, flow: Dataflow, unit: EpilogueUnit) -> set:
        """Steps the emitted node replaces: the unit, plus a prescaled operand that nothing but
        this contraction reads (the left prescale also feeds other steps and stays)."""
        steps = set(unit.steps)
        if self.prescales is not None:
            b = unit.anchor.inputs[1]
            idx, _ = unit.prologue[b]
            if flow.sole_reader(b) == unit.anchor_idx:
                steps.add(idx)
        return steps


Template = ScoreTemplate

KKT_GATED = ScoreTemplate(
    name="kkt-gated-native", family="scalar-gate", operands=("kF", "kF"),
    epilogue=("mul", "tril", "contiguous"), gate="coefA",
    kernels=("kkt_gated_native", "kkt_gated_native_v2"),
    inputs=("kF", "g_native", "beta_native"),
    absorbs="kkt einsum + coefA gate + strict-lower mask (score kept on chip)")
CHUNK_O_GATED = ScoreTemplate(
    name="chunk-o-gated-native", family="scalar-gate", operands=("qF", "kF"),
    epilogue=("mul", "contiguous"), gate="coef_o",
    kernels=("gated_qk_native", "gated_qk_native_v2"),
    inputs=("qF", "kF", "g_native", "beta_native_ones"), params=(("causal", True),),
    absorbs="chunk_o q·kᵀ einsum + coef_o gate/mask")
QK_PROLOGUE = ScoreTemplate(
    name="qk-prologue", family="per-dim-prologue", operands=("qF", "kF"),
    epilogue=("tril", "contiguous"), prescales=("coef_ag", "coef_bg"),
    kernels=("qk_prologue", "qk_prologue_v2"), inputs=("qF", "kF", "coef_ag", "coef_bg"),
    absorbs="per-channel k prescale + chunk_o q·kᵀ einsum + causal mask")


def default_templates() -> List[ScoreTemplate]:
    """In match-priority order."""
    return [KKT_GATED, CHUNK_O_GATED, QK_PROLOGUE]


def _matching(flow: Dataflow, templates: Sequence[ScoreTemplate]):
    for i in flow.find(lambda n: isinstance(n, EinsumNode)):
        unit = _unit(flow, i)
        t = next((t for t in templates if t.matches(unit)), None)
        yield i, unit, t


class FuseContractionEpilogue(Transform):
    """Every contraction whose unit a template matches becomes that template's stage kernel."""
    name = "fuse-contraction-epilogue"
    summary = "score contraction + gate/mask epilogue -> gated-score stage kernel (template)"
    stage = "epilogue"
    no_site_note = "no contraction matches a template"

    def __init__(self, B: int, H: int, nc: int, C: int, D: int, v2: Optional[bool] = None,
                 templates: Optional[List[ScoreTemplate]] = None) -> None:
        self.dims = Dims(B, H, nc, C, D, v2)
        self.templates = list(templates) if templates is not None else default_templates()

    def sites(self, flow: Dataflow):
        return [(unit, t) for _, unit, t in _matching(flow, self.templates) if t is not None]

    def rewrite(self, flow: Dataflow, site, edit: ProgramEdit) -> str:
        unit, t = site
        edit.replace(t.absorbed(flow, unit), [t.node(unit, self.dims)])
        return f"template {t.name}"


@dataclass(frozen=True)
class FlashSpec:
    """A score template whose output feeds a ``score · v`` contraction, and the flash kernel
    that computes both in one launch."""
    score: ScoreTemplate
    kernel: str
    inputs: Tuple[str, ...]            # node inputs before v (v is the consumer's second operand)
    extra: Tuple[str, ...] = ()        # node inputs after v


class _ScoreToOutput(Transform):
    stage = "fusion"
    spec: FlashSpec
    no_site_note = "no chunk_o score -> output chain"

    def __init__(self, B: int, H: int, nc: int, C: int, D: int) -> None:
        self.dims = Dims(B, H, nc, C, D)

    def sites(self, flow: Dataflow):
        out = []
        for i in flow.find(lambda n: isinstance(n, EinsumNode) and n.equation == SCORE_EQ):
            unit = _unit(flow, i)
            if not self.spec.score.matches(unit):
                continue
            c = flow.sole_reader(unit.boundary_out)
            consumer = None if c is None else flow.nodes[c]
            if (isinstance(consumer, EinsumNode) and consumer.equation == APPLY_EQ
                    and consumer.inputs[0] == unit.boundary_out):
                out.append((unit, c))
        return out

    def rewrite(self, flow: Dataflow, site, edit: ProgramEdit) -> str:
        unit, c = site
        apply = flow.nodes[c]
        node = FusedNode(kernel=self.spec.kernel,
                         inputs=[*self.spec.inputs, apply.inputs[1], *self.spec.extra],
                         outputs=[apply.output],
                         params=self.dims.params(DV=self.dims.D, causal=True),
                         subsumes=[self.spec.score.absorbs + " + score·v (score kept in LDS)"])
        edit.replace(self.spec.score.absorbed(flow, unit) | {c}, [node])
        return f"emitted {self.spec.kernel}"


class FuseChunkOFlash(_ScoreToOutput):
    """GDN chunk_o: ``(qF kFᵀ) ⊙ coef_o`` -> contiguous -> ``· v_new`` as qkv_flash_native_v2."""
    name = "fuse-chunk-o-flash"
    summary = "chunk_o q·kᵀ -> gate/mask -> ·v as one qkv_flash_native_v2 (score in LDS)"
    spec = FlashSpec(CHUNK_O_GATED, "qkv_flash_native_v2", ("qF", "kF"),
                     ("g_native", "beta_native_ones"))


class FusePerDimChunkOFlash(_ScoreToOutput):
    """KDA chunk_o: ``tril((qF ⊙ coef_ag)(kF ⊙ coef_bg)ᵀ)`` -> contiguous -> ``· v_new``."""
    name = "fuse-perdim-chunk-o-flash"
    summary = "per-channel chunk_o prescale·q·kᵀ -> mask -> ·v as one qkvp_flash_native_v2"
    spec = FlashSpec(QK_PROLOGUE, "qkvp_flash_native_v2", ("qF", "kF"), ("coef_ag", "coef_bg"))


@dataclass
class EpilogueReport:
    rows: List[Tuple[str, str, str]] = field(default_factory=list)

    def __str__(self) -> str:
        width = max((len(r[0]) for r in self.rows), default=8)
        lines = ["contraction   epilogue                 lowering"]
        for out, epi, verdict in self.rows:
            lines.append(f"{out:<{max(width, 13)}} {epi:<24} {verdict}")
        hit = sum(v.startswith("template ") for _, _, v in self.rows)
        lines.append(f"{hit} of {len(self.rows)} contractions match a template; the rest stay "
                     f"staged")
        return "\n".join(lines)


def epilogue_report(program: Program,
                    templates: Optional[List[ScoreTemplate]] = None) -> EpilogueReport:
    """Per contraction: its epilogue signature and the template that would emit it (or
    'staged')."""
    rep = EpilogueReport()
    for _, unit, t in _matching(Dataflow(program), templates or default_templates()):
        rep.rows.append((unit.anchor.output, "+".join(unit.epilogue_ops) or "-",
                         f"template {t.name}" if t else "staged (no template)"))
    return rep
