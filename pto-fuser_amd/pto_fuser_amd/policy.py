"""Policy: cost model + program -> ordered transform pipeline (src/pto_fuser/policy.py:1-86).

Instantiates the whole transform library for the program's dims, drops what does not match,
asks the cost model whether each is worth trying, and orders the survivors: structural fusions
first (they remove contractions), then the annotation levers over what remains.  It proposes;
the compile driver decides by measurement.

``Policy(whole_forward=True)`` also proposes, ahead of everything else, the whole-forward
rewrites of this build (the canonical GDN / KDA program -> its two-kernel fused forward); the
default pipeline is the reference's per-stage lowering.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

from .cost import CostModel, Features, Prediction
from .ir import Program
from .transform import EnableDirectReads, EnableFusedStore, Transform

__all__ = ["PlannedTransform", "Policy"]

# fusions before annotation levers; the chunk_o flash before the epilogue generator (if the flash
# is kept the generator only finds kkt, if it is dropped the generator fuses the score alone)
_ORDER = {
    "fuse-gdn-forward": -1, "fuse-kda-forward": -1,
    "lower-resident-scan": 0, "lower-perdim-scan": 0,
    "fuse-chunk-o-flash": 1, "fuse-perdim-chunk-o-flash": 1,
    "fuse-contraction-epilogue": 2, "batch-chunk-intra-score": 2,
    "enable-direct-reads": 3, "enable-fused-store": 4,
}


@dataclass
class PlannedTransform:
    transform: Transform
    prediction: Prediction

    @property
    def name(self) -> str:
        return self.transform.name


class Policy:
    def __init__(self, cost: Optional[CostModel] = None, whole_forward: bool = False) -> None:
        self.cost = cost or CostModel()
        self.whole_forward = whole_forward

    def candidates(self, feat: Features) -> List[Transform]:
        from .template import FuseChunkOFlash, FuseContractionEpilogue, FusePerDimChunkOFlash
        from .transforms import (BatchChunkIntraScore, FuseGdnForward, FuseKdaForward,
                                 LowerPerDimScan, LowerResidentScan)
        B, H, nc, C, D = feat.B, feat.H, feat.nc, feat.C, feat.D
        v2 = self.cost.predict("fuse-contraction-epilogue", feat).v2
        intra_v2 = self.cost.predict("batch-chunk-intra-score", feat).v2
        whole: List[Transform] = []
        if self.whole_forward:
            whole = [FuseGdnForward(B, H, nc, C, D, feat.dtype),
                     FuseKdaForward(B, H, nc, C, D, feat.dtype)]
        return whole + [
            LowerResidentScan(B, H, nc, C, D, feat.dtype),
            LowerPerDimScan(B, H, nc, C, D, feat.dtype),
            FuseChunkOFlash(B, H, nc, C, D),
            FusePerDimChunkOFlash(B, H, nc, C, D),
            FuseContractionEpilogue(B, H, nc, C, D, v2=v2),
            BatchChunkIntraScore(feat.N, nc, C, D, D, per_dim_gate=feat.per_dim_gate,
                                 v2=intra_v2 if feat.per_dim_gate else None),
            EnableDirectReads(),
            EnableFusedStore(),
        ]

    def pipeline(self, program: Program, feat: Features) -> List[PlannedTransform]:
        planned = []
        for t in self.candidates(feat):
            if t.match(program) == 0:
                continue
            pred = self.cost.predict(t.name, feat)
            if pred.worth_trying:
                planned.append(PlannedTransform(t, pred))
        planned.sort(key=lambda p: _ORDER.get(p.name, 99))
        return planned
