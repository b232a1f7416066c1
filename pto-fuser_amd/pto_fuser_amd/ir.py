"""Program IR of the delta-rule compile stack (src/pto_fuser/ir.py:1-180).

A program is an ordered list of steps over named tensors.  Three compute node kinds —
``EinsumNode`` (one library contraction), ``OpaqueNode`` (a hand-written kernel the contraction
core cannot express, hosted by key) and ``VecGlueNode`` (an elementwise / mask step) — plus
``FusedNode`` (one HIP kernel standing in for a whole sub-chain, possibly with several outputs)
and ``TensorOp`` (host plumbing: views, reshapes, casts, slices, stacks, allocations).

The node fields and names follow the reference so that its builders, transforms and tests read
the same here; the executors behind them are this package's (staged torch/hipBLASLt, HIP-graph
replay, libptofuser_hip kernels).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, List, Optional

__all__ = ["TensorRef", "Node", "EinsumNode", "OpaqueNode", "VecGlueNode", "FusedNode",
           "TensorOp", "Program", "node_outputs"]


@dataclass(frozen=True)
class TensorRef:
    """A named handle into the execution environment (shape / dtype advisory)."""
    name: str
    shape: Optional[tuple] = None
    dtype: Optional[Any] = None

    def __str__(self) -> str:
        return self.name


class Node:
    """Base of every program step."""
    inputs: List[str]
    output: str


@dataclass
class EinsumNode(Node):
    """One two-operand contraction.  ``read_mode`` / ``fuse_out`` are lowering annotations
    (set by transforms, verified by the compile driver): ``read_mode="NN"`` makes both operands
    contiguous before the contraction (the always-valid baseline), ``"auto"`` contracts the
    views as they are; ``fuse_out=False`` makes the result contiguous, ``True`` lets a permuted
    result stay a view."""
    equation: str
    inputs: List[str]
    output: str
    out_dtype: Optional[Any] = None
    read_mode: str = "auto"
    fuse_out: bool = True
    epilogue: Optional[list] = None
    prologue: Optional[list] = None


@dataclass
class OpaqueNode(Node):
    """A hand-written kernel hosted by key from the opaque registry, which owns its contract
    (input dtype / layout adapters, output dtype)."""
    kernel: str
    inputs: List[str]
    output: str
    params: dict = field(default_factory=dict)


@dataclass
class VecGlueNode(Node):
    """Elementwise step computed in fp32 and cast to ``out_dtype``: tril | add | sub | mul |
    scale."""
    op: str
    inputs: List[str]
    output: str
    params: dict = field(default_factory=dict)
    out_dtype: Optional[Any] = None


@dataclass
class FusedNode(Node):
    """A sub-chain collapsed into one HIP kernel from the fused-kernel registry.  The only node
    with several outputs (the scan returns its snapshots and the final state)."""
    kernel: str
    inputs: List[str]
    outputs: List[str]
    params: dict = field(default_factory=dict)
    subsumes: List[str] = field(default_factory=list)

    @property
    def output(self) -> str:
        return self.outputs[0]


@dataclass
class TensorOp(Node):
    """Host plumbing without a kernel of its own: reshape | contiguous | transpose | permute |
    cast | slice | stack | zeros."""
    op: str
    inputs: List[str]
    output: str
    params: dict = field(default_factory=dict)


def node_outputs(node: Node) -> List[str]:
    """Names a step binds: a FusedNode's ``outputs``, otherwise its single ``output``."""
    outs = getattr(node, "outputs", None)
    return list(outs) if outs is not None else [node.output]


@dataclass
class Program:
    """Ordered steps plus declared inputs (bound at run time) and outputs (returned).
    Construction checks the dataflow: every name a step reads is an input or the output of an
    earlier step, and every declared output is produced."""
    nodes: List[Node]
    inputs: List[str]
    outputs: List[str]

    def __post_init__(self) -> None:
        known = set(self.inputs)
        for node in self.nodes:
            for name in node.inputs:
                if name not in known:
                    raise ValueError(f"step producing {node_outputs(node)[0]!r} reads {name!r} "
                                     f"before it is produced or bound as an input")
            known.update(node_outputs(node))
        missing = [o for o in self.outputs if o not in known]
        if missing:
            raise ValueError(f"declared outputs never produced: {missing}")
