"""Transforms: pure ``Program -> Program`` rewrites (src/pto_fuser/transform.py:1-183).

A transform matches a structural pattern and rewrites it; it never measures or touches the
device.  Whether it is worth trying is the cost model's and policy's call, whether the rewrite is
correct and faster is the compile driver's.  Each carries a kebab-case ``name``, a ``summary``,
construction options (the forward's dims), ``match`` (number of rewritable sites, 0 = not
applicable) and ``apply`` (returns a ``TransformResult``).

This module holds the IR helpers, the canonical form, and the two universal annotation levers;
the forward-shaped rewrites live in ``transforms/`` and ``template.py``.
"""
from __future__ import annotations

from dataclasses import dataclass, replace
from typing import Dict, List

from .ir import EinsumNode, Node, Program, node_outputs

__all__ = ["TransformResult", "Transform", "producer_index", "consumer_map", "splice",
           "canonicalize", "EnableDirectReads", "EnableFusedStore"]


@dataclass
class TransformResult:
    program: Program
    changed: bool
    sites: int
    note: str = ""


class Transform:
    name: str = "transform"
    summary: str = ""

    def match(self, program: Program) -> int:      # pragma: no cover - abstract
        raise NotImplementedError

    def apply(self, program: Program) -> TransformResult:   # pragma: no cover - abstract
        raise NotImplementedError

    def __str__(self) -> str:
        return self.name


def producer_index(program: Program) -> Dict[str, int]:
    """name -> index of the step that binds it (the last one wins)."""
    out: Dict[str, int] = {}
    for i, node in enumerate(program.nodes):
        for name in node_outputs(node):
            out[name] = i
    return out


def consumer_map(program: Program) -> Dict[str, List[int]]:
    """name -> indices of the steps that read it."""
    out: Dict[str, List[int]] = {}
    for i, node in enumerate(program.nodes):
        for name in node.inputs:
            out.setdefault(name, []).append(i)
    return out


def splice(program: Program, drop: set, insert_at: int, new_nodes: List[Node]) -> Program:
    """Remove the steps at ``drop`` and insert ``new_nodes`` just before the step that was at
    ``insert_at`` (appended if that index is past the end).  The result is re-validated."""
    nodes: List[Node] = []
    placed = False
    for i, node in enumerate(program.nodes):
        if i == insert_at:
            nodes.extend(new_nodes)
            placed = True
        if i not in drop:
            nodes.append(node)
    if not placed:
        nodes.extend(new_nodes)
    return Program(nodes=nodes, inputs=list(program.inputs), outputs=list(program.outputs))


def _rebuild(program: Program, nodes: List[Node]) -> Program:
    return Program(nodes=nodes, inputs=list(program.inputs), outputs=list(program.outputs))


def canonicalize(program: Program) -> Program:
    """The always-valid baseline: every contraction reads contiguous operands (``NN``) and
    returns a contiguous result (no fused store)."""
    return _rebuild(program, [replace(n, read_mode="NN", fuse_out=False)
                              if isinstance(n, EinsumNode) else n for n in program.nodes])


class EnableDirectReads(Transform):
    """``read_mode`` NN -> auto on every contraction: contract strided views without copying
    them first."""
    name = "enable-direct-reads"
    summary = "EinsumNode read_mode NN -> auto (contract views directly)"

    def match(self, program: Program) -> int:
        return sum(isinstance(n, EinsumNode) and n.read_mode == "NN" for n in program.nodes)

    def apply(self, program: Program) -> TransformResult:
        sites, nodes = 0, []
        for n in program.nodes:
            if isinstance(n, EinsumNode) and n.read_mode == "NN":
                n = replace(n, read_mode="auto")
                sites += 1
            nodes.append(n)
        return TransformResult(_rebuild(program, nodes), sites > 0, sites,
                               f"{sites} einsum(s) -> direct read")


class EnableFusedStore(Transform):
    """``fuse_out`` False -> True on every contraction: a permuted result may stay a view."""
    name = "enable-fused-store"
    summary = "EinsumNode fuse_out False -> True (permuted result kept as a view)"

    def match(self, program: Program) -> int:
        return sum(isinstance(n, EinsumNode) and not n.fuse_out for n in program.nodes)

    def apply(self, program: Program) -> TransformResult:
        sites, nodes = 0, []
        for n in program.nodes:
            if isinstance(n, EinsumNode) and not n.fuse_out:
                n = replace(n, fuse_out=True)
                sites += 1
            nodes.append(n)
        return TransformResult(_rebuild(program, nodes), sites > 0, sites,
                               f"{sites} einsum(s) -> fused store permitted")
