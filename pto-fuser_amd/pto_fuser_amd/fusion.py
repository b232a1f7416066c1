"""Staged-vs-fused decision for one stage (the reference's verification primitive,
src/pto_fuser/fusion.py:78-101).

``decide`` runs the staged and the fused lowering of one stage on the same inputs and keeps the
fused one only if (1) its outputs are within ``tol`` (relative Frobenius norm) of the staged
outputs, (2) two runs of it are bit-identical, and (3) it is faster.  A ``FusionDecision``
stores the measurements; every verdict is derived from them, so a decision cannot disagree with
its own numbers.  Timing brackets ``iters`` back-to-back calls with one pair of HIP events on the
current stream, after ``warmup`` calls.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Dict, List

import torch

from .gate import frob_rel, gate_determinism

__all__ = ["FusionDecision", "decide", "format_decisions"]

Outputs = Dict[str, torch.Tensor]


@dataclass(frozen=True)
class FusionDecision:
    stage: str
    kernel: str
    frob: float
    deterministic: bool
    t_staged_ms: float
    t_fused_ms: float
    tol: float = 2e-2

    @property
    def gated_ok(self) -> bool:
        return self.frob < self.tol

    @property
    def faster(self) -> bool:
        return self.t_fused_ms < self.t_staged_ms

    @property
    def kept(self) -> bool:
        return self.gated_ok and self.deterministic and self.faster

    @property
    def speedup(self) -> float:
        return self.t_staged_ms / self.t_fused_ms if self.t_fused_ms else float("nan")

    @property
    def detail(self) -> str:
        why = [w for ok, w in ((self.gated_ok, f"frob {self.frob:.1e} >= {self.tol:.0e}"),
                               (self.deterministic, "runs differ"),
                               (self.faster, "not faster")) if not ok]
        return "kept" if not why else "staged: " + ", ".join(why)

    def __str__(self) -> str:
        return (f"{'FUSE ' if self.kept else 'stage'} {self.stage:<14} {self.kernel:<20} "
                f"{self.t_staged_ms:8.3f} -> {self.t_fused_ms:8.3f} ms ({self.speedup:5.2f}x)  "
                f"frob {self.frob:.1e}  {self.detail}")


def _ms_per_call(fn: Callable[[], Outputs], iters: int, warmup: int) -> float:
    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    stop.record(stream)
    stop.synchronize()
    return start.elapsed_time(stop) / iters


def decide(stage: str, kernel: str, staged: Callable[[], Outputs], fused: Callable[[], Outputs],
           *, tol: float = 2e-2, iters: int = 30, warmup: int = 5) -> FusionDecision:
    ref, got = staged(), fused()
    frob = max((frob_rel(got[n], ref[n]) for n in ref if n in got), default=float("inf"))
    det = gate_determinism(fused).passed
    return FusionDecision(stage, kernel, frob, det, _ms_per_call(staged, iters, warmup),
                          _ms_per_call(fused, iters, warmup), tol)


def format_decisions(decisions: List[FusionDecision]) -> str:
    kept = sum(d.kept for d in decisions)
    return "\n".join([str(d) for d in decisions] +
                     [f"{kept}/{len(decisions)} stages fused (within tolerance, deterministic "
                      f"and faster than staged)"])
