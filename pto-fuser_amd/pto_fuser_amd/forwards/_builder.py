"""Small helper the Program builders share: appends typed steps and returns the bound name."""
from __future__ import annotations

from typing import List, Optional, Union

import torch

from ..ir import EinsumNode, Node, OpaqueNode, Program, TensorOp, VecGlueNode

Names = Union[str, List[str], None]


def _names(x: Names) -> List[str]:
    if x is None:
        return []
    return [x] if isinstance(x, str) else list(x)


class ProgramBuilder:
    def __init__(self, work: torch.dtype) -> None:
        self.work = work
        self.nodes: List[Node] = []

    def einsum(self, out: str, equation: str, a: str, b: str) -> str:
        self.nodes.append(EinsumNode(equation, [a, b], out, out_dtype=self.work))
        return out

    def glue(self, out: str, op: str, ins: Names, out_dtype: Optional[torch.dtype] = "work",
             **params) -> str:
        dt = self.work if out_dtype == "work" else out_dtype
        self.nodes.append(VecGlueNode(op, _names(ins), out, params=params, out_dtype=dt))
        return out

    def opaque(self, out: str, kernel: str, a: str) -> str:
        self.nodes.append(OpaqueNode(kernel, [a], out))
        return out

    def op(self, out: str, op: str, ins: Names = None, **params) -> str:
        self.nodes.append(TensorOp(op, _names(ins), out, params=params))
        return out

    def program(self, inputs: List[str], outputs: List[str]) -> Program:
        return Program(nodes=list(self.nodes), inputs=list(inputs), outputs=list(outputs))
