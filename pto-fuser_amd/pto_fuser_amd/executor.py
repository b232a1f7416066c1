"""Staged executor: runs a Program step by step on the current HIP stream.

The correctness floor every lowering is verified against (the reference's ``StagedExecutor``,
src/pto_fuser/executor.py:105-139).  Each node kind has one handler, and the elementwise glue and
host tensor ops are tables of small functions:

* ``EinsumNode``  — the contraction backend, fp32 ``torch.einsum`` on the device (hipBLASLt /
  rocBLAS GEMMs), the result cast to the node's ``out_dtype``.  Contracting in fp32 keeps the
  staged program a faithful reference for the fused kernels (the reference calls its pto-einsum
  library here).  The ``read_mode`` / ``fuse_out`` annotations are that library's layout hints
  and are not used by this backend.
* ``OpaqueNode``  — the opaque registry (the HIP triangular inverse).
* ``FusedNode``   — the fused-kernel registry (the HIP stage kernels); several outputs.
* ``VecGlueNode`` — elementwise in fp32, then cast; ``tril`` is a multiply by a cached 0/1 mask.
* ``TensorOp``    — views, copies, casts, stacks and allocations.
"""
from __future__ import annotations

from typing import Callable, Dict, List, Optional

import torch

from .fused import FusedKernelRegistry, shared_fused_registry
from .ir import EinsumNode, FusedNode, Node, OpaqueNode, Program, TensorOp, VecGlueNode
from .registry import OpaqueRegistry, default_registry

__all__ = ["StagedExecutor", "einsum_fp32", "GLUE_OPS", "TENSOR_OPS"]

Env = Dict[str, torch.Tensor]


def einsum_fp32(equation: str, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """The contraction backend: both operands widened to fp32."""
    return torch.einsum(equation, a.float(), b.float())


_MASKS: Dict[tuple, torch.Tensor] = {}


def _keep_lower(x: torch.Tensor, diagonal: int) -> torch.Tensor:
    key = (x.shape[-2], x.shape[-1], diagonal, x.device, x.dtype)
    mask = _MASKS.get(key)
    if mask is None:
        mask = torch.ones(x.shape[-2:], device=x.device, dtype=x.dtype).tril(diagonal)
        _MASKS[key] = mask
    return x * mask


GLUE_OPS: Dict[str, Callable[[List[torch.Tensor], dict], torch.Tensor]] = {
    "add": lambda xs, p: xs[0] + xs[1],
    "sub": lambda xs, p: xs[0] - xs[1],
    "mul": lambda xs, p: xs[0] * xs[1],
    "scale": lambda xs, p: xs[0] * p["scalar"],
    "tril": lambda xs, p: _keep_lower(xs[0], p.get("diagonal", 0)),
}


def _zeros(env: Env, node: TensorOp) -> torch.Tensor:
    p = node.params
    device = p.get("device") or (env[node.inputs[0]].device if node.inputs else None)
    return torch.zeros(p["shape"], dtype=p["dtype"], device=device)


TENSOR_OPS: Dict[str, Callable[[Env, TensorOp], torch.Tensor]] = {
    "reshape": lambda env, n: env[n.inputs[0]].reshape(n.params["shape"]),
    "contiguous": lambda env, n: env[n.inputs[0]].contiguous(),
    "transpose": lambda env, n: env[n.inputs[0]].transpose(*n.params["dims"]),
    "permute": lambda env, n: env[n.inputs[0]].permute(*n.params["dims"]).contiguous(),
    "cast": lambda env, n: env[n.inputs[0]].to(n.params["dtype"]),
    "slice": lambda env, n: env[n.inputs[0]].select(n.params["axis"], n.params["index"]),
    "stack": lambda env, n: torch.stack([env[x] for x in n.inputs], dim=n.params["dim"]),
    "zeros": _zeros,
}


def _as(t: torch.Tensor, dtype) -> torch.Tensor:
    return t if dtype is None or t.dtype == dtype else t.to(dtype)


class StagedExecutor:
    def __init__(self, registry: Optional[OpaqueRegistry] = None,
                 einsum_fn: Optional[Callable] = None,
                 fused: Optional[FusedKernelRegistry] = None) -> None:
        self.registry = registry or default_registry()
        self.fused = fused or shared_fused_registry()
        self.einsum = einsum_fn or einsum_fp32
        self._handlers: Dict[type, Callable[[Node, Env], Dict[str, torch.Tensor]]] = {
            EinsumNode: self._contract, OpaqueNode: self._opaque, FusedNode: self._fused,
            VecGlueNode: self._glue, TensorOp: self._tensor_op}

    def run(self, program: Program, bindings: Env, return_env: bool = False) -> Env:
        missing = [n for n in program.inputs if n not in bindings]
        if missing:
            raise ValueError(f"missing bindings for program inputs: {missing}")
        env: Env = dict(bindings)
        for node in program.nodes:
            env.update(self.step(node, env))
        return env if return_env else {name: env[name] for name in program.outputs}

    def step(self, node: Node, env: Env) -> Env:
        """Execute one node; returns the names it binds."""
        handler = self._handlers.get(type(node))
        if handler is None:
            raise TypeError(f"no handler for {type(node).__name__}")
        return handler(node, env)

    def _contract(self, node: EinsumNode, env: Env) -> Env:
        a, b = (env[n] for n in node.inputs)
        return {node.output: _as(self.einsum(node.equation, a, b), node.out_dtype)}

    def _opaque(self, node: OpaqueNode, env: Env) -> Env:
        return {node.output: self.registry.run(node.kernel, [env[n] for n in node.inputs],
                                               node.params)}

    def _fused(self, node: FusedNode, env: Env) -> Env:
        outs = self.fused.run(node.kernel, [env[n] for n in node.inputs], node.params)
        if len(outs) != len(node.outputs):
            raise RuntimeError(f"fused kernel {node.kernel!r} returned {len(outs)} tensors for "
                               f"{len(node.outputs)} outputs {node.outputs}")
        return dict(zip(node.outputs, outs))

    def _glue(self, node: VecGlueNode, env: Env) -> Env:
        fn = GLUE_OPS.get(node.op)
        if fn is None:
            raise ValueError(f"unknown glue op {node.op!r}")
        return {node.output: _as(fn([env[n].float() for n in node.inputs], node.params),
                                 node.out_dtype)}

    def _tensor_op(self, node: TensorOp, env: Env) -> Env:
        fn = TENSOR_OPS.get(node.op)
        if fn is None:
            raise ValueError(f"unknown tensor op {node.op!r}")
        return {node.output: fn(env, node)}
