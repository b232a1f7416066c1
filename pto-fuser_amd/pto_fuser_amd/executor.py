"""Staged executor: the always-valid baseline backend (src/pto_fuser/executor.py:1-181).

Runs a ``Program`` node by node over a name -> tensor environment on the current HIP stream.
The backends behind the node kinds on MI355X:

* ``EinsumNode``  — ``torch.einsum`` on the device in fp32 (hipBLASLt / rocBLAS GEMMs), the
  result cast to the node's ``out_dtype``.  The reference calls its pto-einsum library here;
  contracting in fp32 keeps the staged program a faithful reference for the fused kernels and
  keeps bf16 batched products with transposed operands out of the picture.
* ``OpaqueNode`` / ``FusedNode`` — the HIP kernels of libptofuser_hip.so via the registries.
* ``VecGlueNode`` — torch elementwise kernels in fp32 (tril as a cached 0/1 mask multiply).
* ``TensorOp``    — torch views / copies.

It is the correctness reference every other lowering is verified against.
"""
from __future__ import annotations

import contextlib
from typing import Callable, Dict, Optional

import torch

from .fused import FusedKernelRegistry, shared_fused_registry
from .ir import (EinsumNode, FusedNode, OpaqueNode, Program, TensorOp, VecGlueNode,
                 node_outputs)
from .registry import OpaqueRegistry, default_registry

__all__ = ["StagedExecutor", "library_modes", "torch_einsum"]

_MASKS: Dict[tuple, torch.Tensor] = {}


def _tril_mask(rows: int, cols: int, diagonal: int, device, dtype) -> torch.Tensor:
    """Cached {0,1} lower-triangular mask over the last two dims (kept = col <= row + diag)."""
    key = (rows, cols, diagonal, str(device), dtype)
    m = _MASKS.get(key)
    if m is None:
        r = torch.arange(rows, device=device).unsqueeze(1)
        c = torch.arange(cols, device=device).unsqueeze(0)
        m = (c <= r + diagonal).to(dtype)
        _MASKS[key] = m
    return m


_MODE = {"read_mode": "auto", "fuse_out": True}


@contextlib.contextmanager
def library_modes(read_mode: str = "auto", fuse_out: bool = True):
    """Lowering toggles for the contractions run inside the block (executor.py:54-79).
    ``read_mode="NN"`` contracts contiguous copies of both operands (the baseline), ``"auto"``
    the operands as they are; ``fuse_out=False`` returns a contiguous result."""
    if read_mode not in ("auto", "NN"):
        raise ValueError(f"read_mode must be 'auto' or 'NN', got {read_mode!r}")
    saved = dict(_MODE)
    _MODE.update(read_mode=read_mode, fuse_out=bool(fuse_out))
    try:
        yield
    finally:
        _MODE.clear()
        _MODE.update(saved)


def torch_einsum(equation: str, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """The contraction core: fp32 einsum honouring the active ``library_modes``."""
    a32, b32 = a.float(), b.float()
    if _MODE["read_mode"] == "NN":
        a32, b32 = a32.contiguous(), b32.contiguous()
    out = torch.einsum(equation, a32, b32)
    return out if _MODE["fuse_out"] else out.contiguous()


def _cast(t: torch.Tensor, dtype) -> torch.Tensor:
    return t if dtype is None or t.dtype == dtype else t.to(dtype)


class StagedExecutor:
    def __init__(self, registry: Optional[OpaqueRegistry] = None,
                 einsum_fn: Optional[Callable] = None,
                 fused: Optional[FusedKernelRegistry] = None) -> None:
        self.registry = registry or default_registry()
        self.fused = fused or shared_fused_registry()
        self._einsum = einsum_fn

    @property
    def einsum(self) -> Callable:
        if self._einsum is None:
            self._einsum = torch_einsum
        return self._einsum

    def run(self, program: Program, bindings: Dict[str, torch.Tensor],
            return_env: bool = False) -> Dict[str, torch.Tensor]:
        missing = [n for n in program.inputs if n not in bindings]
        if missing:
            raise ValueError(f"missing bindings for inputs: {missing}")
        env: Dict[str, torch.Tensor] = dict(bindings)
        for node in program.nodes:
            result = self._exec(node, env)
            if isinstance(result, dict):
                env.update(result)
            else:
                env[node.output] = result
        if return_env:
            return env
        return {name: env[name] for name in program.outputs}

    def _exec(self, node, env: Dict[str, torch.Tensor]):
        if isinstance(node, EinsumNode):
            a, b = (env[n] for n in node.inputs)
            with library_modes(node.read_mode, node.fuse_out):
                out = self.einsum(node.equation, a, b)
            return _cast(out, node.out_dtype)
        if isinstance(node, OpaqueNode):
            return self.registry.run(node.kernel, [env[n] for n in node.inputs], node.params)
        if isinstance(node, FusedNode):
            outs = self.fused.run(node.kernel, [env[n] for n in node.inputs], node.params)
            if len(outs) != len(node.outputs):
                raise RuntimeError(f"fused kernel {node.kernel!r} returned {len(outs)} tensors "
                                   f"for outputs {node.outputs}")
            return dict(zip(node.outputs, outs))
        if isinstance(node, VecGlueNode):
            return self._exec_glue(node, env)
        if isinstance(node, TensorOp):
            return self._exec_tensorop(node, env)
        raise TypeError(f"unknown node type: {type(node).__name__}")

    def _exec_glue(self, node: VecGlueNode, env) -> torch.Tensor:
        op, p = node.op, node.params
        ins = [env[n].float() for n in node.inputs]
        if op == "tril":
            x = ins[0]
            out = x * _tril_mask(x.shape[-2], x.shape[-1], p.get("diagonal", 0), x.device, x.dtype)
        elif op == "add":
            out = ins[0] + ins[1]
        elif op == "sub":
            out = ins[0] - ins[1]
        elif op == "mul":
            out = ins[0] * ins[1]
        elif op == "scale":
            out = ins[0] * p["scalar"]
        else:
            raise ValueError(f"unknown glue op {op!r}")
        return _cast(out, node.out_dtype)

    def _exec_tensorop(self, node: TensorOp, env) -> torch.Tensor:
        op, p = node.op, node.params
        if op == "zeros":
            ref = env[node.inputs[0]] if node.inputs else None
            device = p.get("device") or (ref.device if ref is not None else None)
            return torch.zeros(p["shape"], dtype=p["dtype"], device=device)
        x = env[node.inputs[0]]
        if op == "reshape":
            return x.reshape(p["shape"])
        if op == "contiguous":
            return x.contiguous()
        if op == "transpose":
            return x.transpose(*p["dims"])
        if op == "permute":
            return x.permute(*p["dims"]).contiguous()
        if op == "cast":
            return x.to(p["dtype"])
        if op == "slice":
            return x.select(p["axis"], p["index"])
        if op == "stack":
            return torch.stack([env[n] for n in node.inputs], dim=p["dim"])
        raise ValueError(f"unknown tensor op {op!r}")


def produced_names(program: Program):
    """Every name the program binds (inputs and step outputs), in order."""
    names = list(program.inputs)
    for n in program.nodes:
        names.extend(node_outputs(n))
    return names
