"""Dataflow view of a Program and the edit buffer every rewrite goes through.

A ``Program`` is an ordered list of steps over named tensors (ir.py).  Rewrites need three
questions answered about it — who binds a name, who reads it, and which steps form a
single-consumer chain — and one operation: drop a set of steps and put new ones in their place.
``Dataflow`` answers the questions from indices built once per program; ``ProgramEdit``
collects removals and insertions against the original step indices and builds the new
(re-validated) ``Program`` in one pass, so a rewrite never has to track shifting indices.
"""
from __future__ import annotations

from typing import Callable, Dict, Iterable, List, Optional, Tuple

from .ir import Node, Program, node_outputs

__all__ = ["Dataflow", "ProgramEdit"]


class Dataflow:
    """Producer and consumer indices of one program (immutable snapshot)."""

    def __init__(self, program: Program) -> None:
        self.program = program
        self.nodes: List[Node] = list(program.nodes)
        self._producer: Dict[str, int] = {}
        self._readers: Dict[str, List[int]] = {}
        for i, node in enumerate(self.nodes):
            for name in node.inputs:
                self._readers.setdefault(name, []).append(i)
            for name in node_outputs(node):
                self._producer[name] = i

    # ---- queries ---------------------------------------------------------------------------
    def producer(self, name: str) -> Optional[int]:
        """Index of the step that binds ``name`` (None for a program input or unknown name)."""
        return self._producer.get(name)

    def producer_node(self, name: str) -> Optional[Node]:
        i = self.producer(name)
        return None if i is None else self.nodes[i]

    def readers(self, name: str) -> List[int]:
        return list(self._readers.get(name, ()))

    def sole_reader(self, name: str) -> Optional[int]:
        r = self._readers.get(name, ())
        return r[0] if len(r) == 1 else None

    def binds(self, name: str) -> bool:
        return name in self._producer or name in self.program.inputs

    def chain(self, start: str, accept: Callable[[Node], bool]) -> List[int]:
        """Steps reached from ``start`` by following sole readers while ``accept`` holds: the
        single-consumer tail a fused kernel could absorb."""
        out: List[int] = []
        cur = start
        while True:
            i = self.sole_reader(cur)
            if i is None or not accept(self.nodes[i]):
                return out
            out.append(i)
            cur = node_outputs(self.nodes[i])[0]

    def find(self, pred: Callable[[Node], bool]) -> List[int]:
        return [i for i, n in enumerate(self.nodes) if pred(n)]

    def outputs_of(self, indices: Iterable[int]) -> List[str]:
        return [name for i in indices for name in node_outputs(self.nodes[i])]


class ProgramEdit:
    """Pending edits against one program's step indices.

    ``remove(i, ...)`` drops steps; ``insert(i, nodes)`` places ``nodes`` immediately before the
    step originally at index ``i`` (``len(program.nodes)`` appends).  ``build()`` applies them
    all at once; the result is a new ``Program`` with the same inputs and outputs, checked for
    use-before-def by its constructor."""

    def __init__(self, program: Program) -> None:
        self.program = program
        self._removed: set = set()
        self._inserts: List[Tuple[int, int, List[Node]]] = []

    def remove(self, *indices: int) -> "ProgramEdit":
        for i in indices:
            if not 0 <= i < len(self.program.nodes):
                raise IndexError(f"no step {i} to remove")
            self._removed.add(i)
        return self

    def remove_all(self, indices: Iterable[int]) -> "ProgramEdit":
        return self.remove(*indices)

    def insert(self, before: int, nodes: List[Node]) -> "ProgramEdit":
        self._inserts.append((before, len(self._inserts), list(nodes)))
        return self

    def replace(self, indices: Iterable[int], nodes: List[Node]) -> "ProgramEdit":
        """Drop ``indices`` and put ``nodes`` where the first of them stood."""
        idx = sorted(set(indices))
        if not idx:
            raise ValueError("replace needs at least one step")
        self.remove(*idx)
        return self.insert(idx[0], nodes)

    @property
    def removed(self) -> frozenset:
        return frozenset(self._removed)

    def build(self) -> Program:
        by_pos: Dict[int, List[Node]] = {}
        for pos, _, nodes in sorted(self._inserts):
            by_pos.setdefault(pos, []).extend(nodes)
        out: List[Node] = []
        for i, node in enumerate(self.program.nodes):
            out.extend(by_pos.pop(i, ()))
            if i not in self._removed:
                out.append(node)
        for pos in sorted(by_pos):
            out.extend(by_pos[pos])
        return Program(nodes=out, inputs=list(self.program.inputs),
                       outputs=list(self.program.outputs))
