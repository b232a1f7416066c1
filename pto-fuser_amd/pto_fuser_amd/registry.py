"""Opaque-kernel registry: OpaqueNode key -> a hand-written kernel and its contract.

An ``OpaqueNode`` names a kernel the contraction backend cannot express (the reference's
``OpaqueRegistry``, src/pto_fuser/registry.py:52-90).  Each registration is an ``OpaqueKernel``:
a factory that builds the raw callable on first use, and a lowering that applies the pinned
contract (input dtype and layout adapters, output dtype) around the raw call.

The seed entry is ``tri_inv_rec_unroll``, the unit-lower triangular inverse ``(I + A)^-1`` of
the delta-rule forward, served by ``pf_tri_inv_exec``.  The reference's kernel (un-vendored
pto-kernels) inverts strictly-upper fp16 matrices, so its lowering narrows to fp16, transposes
and synchronises the device around the launch (registry.py:107-127).  ``pf_tri_inv_exec`` reads
the strictly-lower fp32 ``A`` as it is and launches on the current stream: the lowering is a
widening to fp32, nothing else, and the node is capturable into a HIP graph unchanged.

``capture_mode()`` marks a region as HIP-graph capture for lowerings that must behave
differently there (the reference drops its host synchronisations under it).  It counts nesting
depth, so inner regions never end an outer one; no lowering of this build needs it.
"""
from __future__ import annotations

import contextlib
from dataclasses import dataclass
from typing import Any, Callable, Dict, List, Optional

import torch

__all__ = ["OpaqueContract", "OpaqueKernel", "OpaqueRegistry", "capture_mode",
           "in_capture_mode", "default_registry"]

_capture_depth = 0


@contextlib.contextmanager
def capture_mode():
    global _capture_depth
    _capture_depth += 1
    try:
        yield
    finally:
        _capture_depth -= 1


def in_capture_mode() -> bool:
    return _capture_depth > 0


@dataclass(frozen=True)
class OpaqueContract:
    """Pinned interface of one opaque kernel: required input dtypes and the output dtype."""
    in_dtypes: List[Any]
    out_dtype: Any
    notes: str = ""


class OpaqueKernel:
    def __init__(self, key: str, factory: Callable[[], Callable], lowering: Callable,
                 contract: OpaqueContract) -> None:
        self.key, self.contract = key, contract
        self._factory, self._lowering = factory, lowering
        self._raw: Optional[Callable] = None

    def __call__(self, inputs: List[torch.Tensor], params: dict) -> torch.Tensor:
        if self._raw is None:
            self._raw = self._factory()
        return self._lowering(self._raw, inputs, params)


class OpaqueRegistry:
    def __init__(self) -> None:
        self._kernels: Dict[str, OpaqueKernel] = {}

    def register(self, key: str, *, factory: Callable, lowering: Callable,
                 contract: OpaqueContract) -> None:
        if key in self._kernels:
            raise ValueError(f"opaque kernel {key!r} is already registered")
        self._kernels[key] = OpaqueKernel(key, factory, lowering, contract)

    def keys(self) -> List[str]:
        return sorted(self._kernels)

    def _get(self, key: str) -> OpaqueKernel:
        try:
            return self._kernels[key]
        except KeyError:
            raise KeyError(f"no opaque kernel registered under {key!r} "
                           f"(known: {', '.join(self.keys()) or 'none'})") from None

    def contract(self, key: str) -> OpaqueContract:
        return self._get(key).contract

    def run(self, key: str, inputs: List[torch.Tensor], params: dict) -> torch.Tensor:
        return self._get(key)(inputs, params)


def _tri_inv_factory() -> Callable:
    from .ops import tri_inv
    return tri_inv


def _tri_inv_lowering(raw: Callable, inputs: List[torch.Tensor], params: dict) -> torch.Tensor:
    """(I + A)^-1 of the strictly-lower part of A [..., C, C]: widened to fp32 (never narrowed),
    flattened to [M, C, C]; fp32 out."""
    (A,) = inputs
    C = A.shape[-1]
    return raw(A.reshape(-1, C, C).float().contiguous())


def default_registry() -> OpaqueRegistry:
    reg = OpaqueRegistry()
    reg.register(
        "tri_inv_rec_unroll", factory=_tri_inv_factory, lowering=_tri_inv_lowering,
        contract=OpaqueContract(
            in_dtypes=[torch.float32], out_dtype=torch.float32,
            notes="strictly-lower A [M,C,C] -> (I+A)^-1 (unit lower), C in {16,32,48,64,128}; "
                  "pf_tri_inv_exec on the current stream"))
    return reg
