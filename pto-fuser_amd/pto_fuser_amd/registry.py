"""Opaque-kernel registry (src/pto_fuser/registry.py:1-140).

An ``OpaqueNode`` names a hand-written kernel the contraction core cannot express; the registry
maps the key to a factory (the raw callable, built once) and a lowering that applies the pinned
contract — dtype casts and layout adapters — before the launch.

The seed entry ``tri_inv_rec_unroll`` is the unit-lower triangular inverse ``(I + A)^-1`` of the
delta-rule forward, served by ``pf_tri_inv_exec`` of libptofuser_hip.so.  The reference's
kernel inverts strictly-upper fp16 matrices, so its lowering casts to fp16, transposes, builds
``-I`` and brackets the raw launch with two device synchronisations (registry.py:107-127).
Here the kernel reads the strictly-lower fp32 ``A`` directly and launches on the current torch
stream, so the lowering is a cast to fp32 and nothing else: no transposes, no host syncs, and
the call is capturable into a HIP graph as it stands.  ``capture_mode`` is kept with the
reference's semantics (a process-wide flag a lowering may consult while a graph is being
captured); none of the lowerings here needs it.
"""
from __future__ import annotations

import contextlib
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Optional

import torch

__all__ = ["OpaqueContract", "OpaqueRegistry", "capture_mode", "default_registry",
           "in_capture_mode"]

_CAPTURE_MODE = False


@contextlib.contextmanager
def capture_mode():
    """Mark a region as HIP-graph capture (nests; restored on exit or error)."""
    global _CAPTURE_MODE
    prev = _CAPTURE_MODE
    _CAPTURE_MODE = True
    try:
        yield
    finally:
        _CAPTURE_MODE = prev


def in_capture_mode() -> bool:
    return _CAPTURE_MODE


@dataclass
class OpaqueContract:
    """Pinned interface of one opaque kernel: required input dtypes and the output dtype."""
    in_dtypes: List[Any]
    out_dtype: Any
    notes: str = ""


@dataclass
class _Entry:
    factory: Callable[[], Callable]
    lowering: Callable
    contract: OpaqueContract
    _raw: Optional[Callable] = field(default=None, repr=False)

    def callable(self) -> Callable:
        if self._raw is None:
            self._raw = self.factory()
        return self._raw


class OpaqueRegistry:
    def __init__(self) -> None:
        self._entries: Dict[str, _Entry] = {}

    def register(self, key: str, *, factory: Callable, lowering: Callable,
                 contract: OpaqueContract) -> None:
        if key in self._entries:
            raise ValueError(f"opaque kernel {key!r} already registered")
        self._entries[key] = _Entry(factory, lowering, contract)

    def keys(self) -> List[str]:
        return list(self._entries)

    def contract(self, key: str) -> OpaqueContract:
        if key not in self._entries:
            raise KeyError(f"no opaque kernel registered under {key!r}")
        return self._entries[key].contract

    def run(self, key: str, inputs: List[torch.Tensor], params: dict) -> torch.Tensor:
        if key not in self._entries:
            raise KeyError(f"no opaque kernel registered under {key!r}")
        entry = self._entries[key]
        return entry.lowering(entry.callable(), inputs, params)


# --------------------------------------------------------------------------- #
#  tri_inv_rec_unroll -> pf_tri_inv_exec
# --------------------------------------------------------------------------- #
def _tri_inv_factory() -> Callable:
    from .ops import tri_inv
    return tri_inv


def _tri_inv_lowering(tri_inv: Callable, inputs: List[torch.Tensor], params: dict) -> torch.Tensor:
    """(I + A)^-1 of the strictly-lower part of A [M, C, C]; fp32 in, fp32 out (the cast is the
    contract: any incoming dtype is widened, never narrowed)."""
    (A,) = inputs
    if A.dim() != 3:
        A = A.reshape(-1, A.shape[-2], A.shape[-1])
    return tri_inv(A.float().contiguous())


def default_registry() -> OpaqueRegistry:
    reg = OpaqueRegistry()
    reg.register(
        "tri_inv_rec_unroll",
        factory=_tri_inv_factory,
        lowering=_tri_inv_lowering,
        contract=OpaqueContract(
            in_dtypes=[torch.float32], out_dtype=torch.float32,
            notes="strictly-lower A [M,C,C] -> (I+A)^-1 (unit lower); C in {16,32,48,64,128}; "
                  "pf_tri_inv_exec on the current stream"))
    return reg
