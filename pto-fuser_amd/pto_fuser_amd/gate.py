"""Correctness gates of the compile stack (src/pto_fuser/gate.py:1-69).

* frob gate — relative Frobenius norm of the difference, ``||got - ref|| / ||ref||``, under a
  tolerance;
* determinism gate — the candidate run twice on identical inputs must be bit-identical.

Every non-default lowering is kept only if it passes both against the staged lowering.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Dict, List

import torch

__all__ = ["frob_rel", "GateResult", "gate_frob_rel", "gate_outputs", "gate_determinism"]


def frob_rel(got: torch.Tensor, ref: torch.Tensor) -> float:
    g, r = got.double(), ref.double()
    return float((g - r).norm().item() / max(r.norm().item(), 1e-9))


@dataclass
class GateResult:
    name: str
    passed: bool
    detail: str

    def __str__(self) -> str:
        return f"[{'OK' if self.passed else 'FAIL'}] {self.name}: {self.detail}"


def gate_frob_rel(name: str, got: torch.Tensor, ref: torch.Tensor, tol: float) -> GateResult:
    rel = frob_rel(got, ref)
    amax = float((got.double() - ref.double()).abs().max().item()) if ref.numel() else 0.0
    return GateResult(name, rel < tol, f"frob_rel={rel:.3e} (tol {tol:.1e})  max_abs={amax:.3e}")


def gate_outputs(got: Dict[str, torch.Tensor], ref: Dict[str, torch.Tensor],
                 tol: float) -> List[GateResult]:
    """frob-gate every name present in both dicts."""
    return [gate_frob_rel(n, got[n], ref[n], tol) for n in ref if n in got]


def gate_determinism(run_fn: Callable[[], Dict[str, torch.Tensor]]) -> GateResult:
    """Run twice; every output must be bit-identical."""
    a = run_fn()
    b = run_fn()
    bad = []
    for name in a:
        if not torch.equal(a[name], b[name]):
            diff = float((a[name].double() - b[name].double()).abs().max().item())
            bad.append(f"{name}(Δ={diff:.3e})")
    passed = not bad
    return GateResult("determinism", passed,
                      "bit-identical across 2 runs" if passed else "NDET: " + ", ".join(bad))
