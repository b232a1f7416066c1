"""Compilation report: what the policy proposed, what the verifier measured, what was kept.

One ``TransformRecord`` per proposed transform.  A record starts from the cost model's
prediction and ends in one of four outcomes:

  no-match    an earlier transform already consumed the site
  applied     kept without verification (no bindings, or verify=False)
  kept        verified: within tolerance of the canonical program, bit-deterministic, faster
  rejected    verified and failed at least one of the three

The fields are the reference's report fields (src/pto_fuser/report.py), derived here from the
outcome and the measurement rather than set one by one.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

__all__ = ["Measurement", "TransformRecord", "CompilationReport"]


@dataclass(frozen=True)
class Measurement:
    """One verified candidate: worst frob_rel against the canonical outputs, whether two replays
    of its graph were bit-identical, and its replay time against the best program so far."""
    frob: float
    deterministic: bool
    t_base_ms: float
    t_cand_ms: float

    @property
    def faster(self) -> bool:
        return self.t_cand_ms < self.t_base_ms


@dataclass
class TransformRecord:
    name: str
    summary: str
    predicted_benefit: float
    predicted_rationale: str
    outcome: str = "pending"
    measurement: Optional[Measurement] = None
    note: str = ""

    # ---- the reference's flat fields, derived -------------------------------------------
    @property
    def matched(self) -> bool:
        return self.outcome != "no-match"

    @property
    def attempted(self) -> bool:
        return self.outcome in ("applied", "kept", "rejected")

    @property
    def kept(self) -> bool:
        return self.outcome in ("applied", "kept")

    @property
    def frob(self) -> Optional[float]:
        return None if self.measurement is None else self.measurement.frob

    @property
    def deterministic(self) -> Optional[bool]:
        return None if self.measurement is None else self.measurement.deterministic

    @property
    def faster(self) -> Optional[bool]:
        return None if self.measurement is None else self.measurement.faster

    @property
    def t_base_ms(self) -> Optional[float]:
        return None if self.measurement is None else self.measurement.t_base_ms

    @property
    def t_cand_ms(self) -> Optional[float]:
        return None if self.measurement is None else self.measurement.t_cand_ms

    @property
    def speedup(self) -> Optional[float]:
        m = self.measurement
        return None if m is None or not m.t_cand_ms else m.t_base_ms / m.t_cand_ms

    def row(self) -> List[str]:
        m = self.measurement
        measured = "" if m is None else (
            f"frob {m.frob:.1e}, {'deterministic' if m.deterministic else 'NOT deterministic'}, "
            f"{m.t_base_ms:.3f} -> {m.t_cand_ms:.3f} ms ({self.speedup:.2f}x)")
        return [self.outcome, self.name, f"{self.predicted_benefit:+.1f} us",
                measured or self.note]


@dataclass
class CompilationReport:
    features: object
    records: List[TransformRecord] = field(default_factory=list)
    verified: bool = False

    @property
    def kept(self) -> List[TransformRecord]:
        return [r for r in self.records if r.kept]

    def __str__(self) -> str:
        rows = [["outcome", "transform", "predicted", "measured / note"]]
        rows += [r.row() for r in self.records]
        widths = [max(len(r[i]) for r in rows) for i in range(3)]
        lines = [f"{len(self.kept)} of {len(self.records)} transforms kept "
                 f"({'verified on the device' if self.verified else 'unverified'})"]
        for r in rows:
            lines.append("  " + "  ".join(c.ljust(w) for c, w in zip(r[:3], widths)) + "  " + r[3])
        return "\n".join(lines)
