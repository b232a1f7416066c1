"""Program rewrites: the Transform interface, the canonical form, the annotation levers.

Interface (the reference's, src/pto_fuser/transform.py:49-65: a kebab-case ``name``, a
``summary``, ``match(program) -> sites`` and ``apply(program) -> TransformResult``; a transform
never touches the device — whether it is worth trying is the cost model's call, whether it is
right and faster the compile driver's).  Here every transform is written as two hooks over the
shared dataflow view:

* ``sites(flow)``  — the non-overlapping places the rewrite applies to (any objects);
* ``rewrite(flow, site, edit)`` — record the replacement of one site in a ``ProgramEdit`` and
  return a one-line note.

``match`` counts the sites; ``apply`` rewrites all of them against the original indices in one
pass.  ``stage`` places a transform in the policy's pipeline (see policy.py).

The two annotation levers flip the ``read_mode`` / ``fuse_out`` fields of every contraction.
They are annotations only on MI355X: they are what the reference's contraction library
(pto-einsum) reads to pick operand layouts, and the contraction backend here (the staged
executor's fp32 GEMMs) chooses its own layouts.  They are kept so that programs, reports and the
lowered-kernel contract read as the reference's do.
"""
from __future__ import annotations

from dataclasses import dataclass, replace
from typing import Any, List

from .dataflow import Dataflow, ProgramEdit
from .ir import EinsumNode, Program

__all__ = ["TransformResult", "Transform", "canonicalize", "AnnotationLever",
           "EnableDirectReads", "EnableFusedStore"]


@dataclass
class TransformResult:
    program: Program
    changed: bool
    sites: int
    note: str = ""


class Transform:
    name: str = "transform"
    summary: str = ""
    stage: str = "structural"          # whole | structural | fusion | epilogue | annotation
    no_site_note: str = "no site"

    def sites(self, flow: Dataflow) -> List[Any]:          # pragma: no cover - abstract
        raise NotImplementedError

    def rewrite(self, flow: Dataflow, site: Any, edit: ProgramEdit) -> str:  # pragma: no cover
        raise NotImplementedError

    def match(self, program: Program) -> int:
        return len(self.sites(Dataflow(program)))

    def apply(self, program: Program) -> TransformResult:
        flow = Dataflow(program)
        found = self.sites(flow)
        if not found:
            return TransformResult(program, False, 0, self.no_site_note)
        edit = ProgramEdit(program)
        notes = [self.rewrite(flow, site, edit) for site in found]
        return TransformResult(edit.build(), True, len(found), "; ".join(n for n in notes if n))

    def __str__(self) -> str:
        return self.name


def canonicalize(program: Program) -> Program:
    """The baseline every lowering is verified against: each contraction annotated to read
    contiguous operands (``read_mode="NN"``) and store a contiguous result (``fuse_out=False``)."""
    nodes = [replace(n, read_mode="NN", fuse_out=False) if isinstance(n, EinsumNode) else n
             for n in program.nodes]
    return Program(nodes=nodes, inputs=list(program.inputs), outputs=list(program.outputs))


class AnnotationLever(Transform):
    """Set one EinsumNode annotation ``field`` from ``before`` to ``after`` wherever it holds
    ``before``."""
    stage = "annotation"
    field: str = ""
    before: Any = None
    after: Any = None
    no_site_note = "every contraction already annotated"

    def sites(self, flow: Dataflow) -> List[int]:
        return flow.find(lambda n: isinstance(n, EinsumNode)
                         and getattr(n, self.field) == self.before)

    def rewrite(self, flow: Dataflow, site: int, edit: ProgramEdit) -> str:
        edit.replace([site], [replace(flow.nodes[site], **{self.field: self.after})])
        return ""

    def apply(self, program: Program) -> TransformResult:
        res = super().apply(program)
        if res.changed:
            res.note = f"{res.sites} contraction(s): {self.field} {self.before!r} -> {self.after!r}"
        return res


class EnableDirectReads(AnnotationLever):
    name = "enable-direct-reads"
    summary = "contraction read_mode NN -> auto (operands read as they lie)"
    field, before, after = "read_mode", "NN", "auto"


class EnableFusedStore(AnnotationLever):
    name = "enable-fused-store"
    summary = "contraction fuse_out False -> True (result may keep the consumer's layout)"
    field, before, after = "fuse_out", False, True
