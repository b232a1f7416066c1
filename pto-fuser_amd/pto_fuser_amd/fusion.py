"""Staged-vs-fused decision for one stage (src/pto_fuser/fusion.py:1-109).

``decide`` runs both lowerings of a stage on identical inputs: the fused output is frob-gated
against the staged one, the fused run is checked bit-deterministic, both are timed back to back
with one trailing device synchronisation, and the fused lowering is kept only if it passes both
gates and is faster.
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Callable, Dict, List

import torch

from .gate import frob_rel, gate_determinism

__all__ = ["FusionDecision", "decide", "format_decisions"]

Outputs = Dict[str, torch.Tensor]
RunFn = Callable[[], Outputs]


@dataclass
class FusionDecision:
    stage: str
    kernel: str
    gated_ok: bool
    deterministic: bool
    faster: bool
    kept: bool
    t_staged_ms: float
    t_fused_ms: float
    frob: float
    detail: str

    @property
    def speedup(self) -> float:
        return self.t_staged_ms / self.t_fused_ms if self.t_fused_ms else float("nan")

    def __str__(self) -> str:
        verdict = "FUSE" if self.kept else "stage"
        flags = f"frob={self.frob:.1e} {'det' if self.deterministic else 'NDET'}"
        return (f"[{verdict}] {self.stage:<14} {self.kernel:<14} {flags:<18} "
                f"staged {self.t_staged_ms:7.3f}ms -> fused {self.t_fused_ms:7.3f}ms "
                f"({self.speedup:.2f}x)")


def _time(fn: RunFn, iters: int = 30, warmup: int = 5) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / iters * 1e3


def decide(stage: str, kernel: str, staged: RunFn, fused: RunFn, *, tol: float = 2e-2,
           iters: int = 30, warmup: int = 5) -> FusionDecision:
    ref = staged()
    got = fused()
    worst = max((frob_rel(got[n], ref[n]) for n in ref if n in got), default=float("inf"))
    det = gate_determinism(fused)
    t_staged = _time(staged, iters, warmup)
    t_fused = _time(fused, iters, warmup)
    gated_ok, faster = worst < tol, t_fused < t_staged
    kept = gated_ok and det.passed and faster
    detail = (f"frob_rel={worst:.2e} (tol {tol:.0e}); {det.detail}; "
              f"{'faster' if faster else 'not faster'}")
    return FusionDecision(stage, kernel, gated_ok, det.passed, faster, kept, t_staged, t_fused,
                          worst, detail)


def format_decisions(decisions: List[FusionDecision]) -> str:
    kept = sum(d.kept for d in decisions)
    return "\n".join([str(d) for d in decisions] +
                     [f"-- {kept}/{len(decisions)} stages fused (gated-green, deterministic, and "
                      f"faster than staged-captured)"])
