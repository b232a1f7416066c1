"""Compile driver: propose, verify, keep or roll back.

``compile_program(program, features, bindings=..., verify=True)`` is the reference's entry point
(src/pto_fuser/compile.py:46-102): the policy proposes an ordered list of transforms, each is
applied to the best program so far, and a candidate survives only if it computes the same thing
as the canonical program and is faster.  Here the driver is a ``Compiler`` holding the best
program and, when verifying, a ``Verifier``:

* the verifier captures a program once as a HIP graph (graph.GraphReplayExecutor) and times
  ``iters`` replays after ``warmup``; the canonical program's outputs are the reference for every
  candidate;
* a candidate is kept when its worst relative Frobenius error over the outputs is under ``tol``,
  a second replay of its graph is bit-identical to the first, and its replay time beats the best
  program's.  A rejected candidate leaves the best program unchanged (rollback is simply not
  adopting it).

Without bindings, or with ``verify=False``, every matching transform is applied unverified: the
structural form the unit tests check.
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Dict, Optional

from .cost import Features
from .gate import frob_rel, gate_determinism
from .ir import Program
from .policy import PlannedTransform, Policy
from .report import CompilationReport, Measurement, TransformRecord
from .transform import canonicalize

__all__ = ["CompileResult", "Verifier", "Compiler", "compile_program"]


@dataclass
class CompileResult:
    program: Program
    report: CompilationReport


class Verifier:
    """Graph-captured runs of candidate programs against one set of bindings."""

    def __init__(self, bindings: Dict, tol: float, iters: int, warmup: int) -> None:
        self.bindings, self.tol, self.iters, self.warmup = bindings, tol, iters, warmup
        self.reference: Optional[Dict] = None

    def _capture(self, program: Program):
        from .graph import GraphReplayExecutor
        return GraphReplayExecutor().capture(program, self.bindings)

    def _time_ms(self, graph) -> float:
        import torch
        for _ in range(self.warmup):
            graph.replay(self.bindings, clone=False)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(self.iters):
            graph.replay(self.bindings, clone=False)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / self.iters * 1e3

    def baseline(self, program: Program) -> float:
        """Record the canonical outputs; return the canonical program's replay time."""
        graph = self._capture(program)
        self.reference = graph.replay(self.bindings)
        return self._time_ms(graph)

    def measure(self, program: Program, best_ms: float) -> Measurement:
        graph = self._capture(program)
        first = graph.replay(self.bindings)
        shared = [n for n in self.reference if n in first]
        frob = max((frob_rel(first[n], self.reference[n]) for n in shared), default=float("inf"))
        det = gate_determinism(lambda: graph.replay(self.bindings))
        return Measurement(frob, det.passed, best_ms, self._time_ms(graph))


class Compiler:
    """The best program so far and the records of every proposal."""

    def __init__(self, program: Program, verifier: Optional[Verifier]) -> None:
        self.best = program
        self.verifier = verifier
        self.best_ms = verifier.baseline(program) if verifier is not None else None

    def propose(self, planned: PlannedTransform) -> TransformRecord:
        t, pred = planned.transform, planned.prediction
        rec = TransformRecord(t.name, t.summary, pred.benefit, pred.rationale)
        if not t.match(self.best):
            rec.outcome, rec.note = "no-match", "site consumed by an earlier transform"
            return rec
        candidate = t.apply(self.best).program
        if self.verifier is None:
            rec.outcome, rec.note, self.best = "applied", "applied (unverified)", candidate
            return rec
        m = self.verifier.measure(candidate, self.best_ms)
        rec.measurement = m
        if m.frob < self.verifier.tol and m.deterministic and m.faster:
            rec.outcome, self.best, self.best_ms = "kept", candidate, m.t_cand_ms
        else:
            rec.outcome = "rejected"
        return rec


def compile_program(program: Program, features: Features, *, policy: Optional[Policy] = None,
                    bindings: Optional[Dict] = None, verify: bool = True, tol: float = 2e-2,
                    iters: int = 30, warmup: int = 5) -> CompileResult:
    policy = policy or Policy()
    canonical = canonicalize(program)
    verifier = (Verifier(bindings, tol, iters, warmup)
                if verify and bindings is not None else None)
    compiler = Compiler(canonical, verifier)
    records = [compiler.propose(p) for p in policy.pipeline(canonical, features)]
    return CompileResult(compiler.best, CompilationReport(features, records, verifier is not None))
