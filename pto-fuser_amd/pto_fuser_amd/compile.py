"""Compile driver: propose / verify / dispose (src/pto_fuser/compile.py:1-123).

``compile_program`` canonicalises the program, asks the policy for a pipeline, then tries each
proposed transform in turn.  With bindings and ``verify=True`` every candidate is captured into a
HIP graph and replayed on the device; it is kept only if its outputs are within ``tol`` (relative
Frobenius norm) of the *canonical* program's, a second replay of the same graph is bit-identical,
and it is faster than the best program so far.  Without bindings (or ``verify=False``) the
transforms are applied unverified — the structural form the unit tests check.
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Dict, Optional

from .cost import Features
from .gate import frob_rel, gate_determinism
from .ir import Program
from .policy import Policy
from .report import CompilationReport, TransformRecord
from .transform import canonicalize

__all__ = ["CompileResult", "compile_program"]


@dataclass
class CompileResult:
    program: Program
    report: CompilationReport


def compile_program(program: Program, features: Features, *, policy: Optional[Policy] = None,
                    bindings: Optional[Dict] = None, verify: bool = True, tol: float = 2e-2,
                    iters: int = 30, warmup: int = 5) -> CompileResult:
    policy = policy or Policy()
    canonical = canonicalize(program)
    plan = policy.pipeline(canonical, features)
    do_verify = verify and bindings is not None
    records = []
    prog = canonical
    if do_verify:
        ref_out, base_ms, _ = _run_and_time(canonical, bindings, iters, warmup)
    for planned in plan:
        t, pred = planned.transform, planned.prediction
        rec = TransformRecord(name=t.name, summary=t.summary, predicted_benefit=pred.benefit,
                              predicted_rationale=pred.rationale, matched=t.match(prog) > 0,
                              attempted=False, kept=False)
        if not rec.matched:
            rec.note = "no match after prior transforms"
            records.append(rec)
            continue
        cand = t.apply(prog).program
        rec.attempted = True
        if not do_verify:
            prog, rec.kept, rec.note = cand, True, "applied (unverified)"
            records.append(rec)
            continue
        got, cand_ms, replay = _run_and_time(cand, bindings, iters, warmup)
        worst = max((frob_rel(got[n], ref_out[n]) for n in ref_out if n in got),
                    default=float("inf"))
        det = gate_determinism(replay)
        faster = cand_ms < base_ms
        rec.kept = worst < tol and det.passed and faster
        rec.frob, rec.deterministic, rec.faster = worst, det.passed, faster
        rec.t_base_ms, rec.t_cand_ms = base_ms, cand_ms
        if rec.kept:
            prog, base_ms = cand, cand_ms
        records.append(rec)
    return CompileResult(prog, CompilationReport(features, records, do_verify))


def _run_and_time(program: Program, bindings: Dict, iters: int, warmup: int):
    """Capture ``program`` as one HIP graph; return (outputs, ms per replay, a function that
    replays the same graph once more) — the determinism gate re-runs this capture."""
    import torch
    from .graph import GraphReplayExecutor
    gr = GraphReplayExecutor().capture(program, bindings)
    out = None
    for _ in range(max(1, warmup)):
        out = gr.replay(bindings)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        gr.replay(bindings, clone=False)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / iters * 1e3
    return out, ms, (lambda: gr.replay(bindings))
