"""Policy: program + shape -> the ordered list of transforms the compile driver will try.

The policy instantiates the transform library for the forward's dims, keeps the transforms
that find a site in the program and that the cost model expects to pay, and orders them by
pipeline stage (``Transform.stage``):

  whole        the canonical forward -> the fused two-kernel forward (opt-in, this build only)
  structural   the unrolled scan -> the resident-state scan kernel
  fusion       the chunk_o score -> output chain -> one flash kernel
  epilogue     the remaining score contractions -> gated-score stage kernels (templates)
  annotation   contraction layout annotations

Within a stage the library's own order holds.  The order matters where two transforms compete
for one site: the chunk_o flash runs before the epilogue templates, so the score it consumes is
gone when the templates look (the reference's policy orders its transforms the same way,
src/pto_fuser/policy.py:27-32).  The policy proposes; the compile driver decides by measurement.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, List, Optional, Tuple

from .cost import CostModel, Features, Prediction
from .ir import Program
from .transform import EnableDirectReads, EnableFusedStore, Transform

__all__ = ["PlannedTransform", "Policy", "STAGES"]

STAGES: Tuple[str, ...] = ("whole", "structural", "fusion", "epilogue", "annotation")


@dataclass
class PlannedTransform:
    transform: Transform
    prediction: Prediction

    @property
    def name(self) -> str:
        return self.transform.name


def _library(f: Features, cost: CostModel, whole: bool) -> List[Transform]:
    from .template import FuseChunkOFlash, FuseContractionEpilogue, FusePerDimChunkOFlash
    from .transforms import FuseGdnForward, FuseKdaForward, LowerPerDimScan, LowerResidentScan
    dims = (f.B, f.H, f.nc, f.C, f.D)
    makers: List[Callable[[], Transform]] = []
    if whole:
        makers += [lambda: FuseGdnForward(*dims, f.dtype), lambda: FuseKdaForward(*dims, f.dtype)]
    makers += [
        lambda: LowerResidentScan(*dims, f.dtype),
        lambda: LowerPerDimScan(*dims, f.dtype),
        lambda: FuseChunkOFlash(*dims),
        lambda: FusePerDimChunkOFlash(*dims),
        lambda: FuseContractionEpilogue(
            *dims, v2=cost.predict("fuse-contraction-epilogue", f).v2),
        EnableDirectReads,
        EnableFusedStore,
    ]
    return [make() for make in makers]


class Policy:
    def __init__(self, cost: Optional[CostModel] = None, whole_forward: bool = False) -> None:
        self.cost = cost or CostModel()
        self.whole_forward = whole_forward

    def candidates(self, feat: Features) -> List[Transform]:
        return _library(feat, self.cost, self.whole_forward)

    def pipeline(self, program: Program, feat: Features) -> List[PlannedTransform]:
        ranked = []
        for pos, t in enumerate(self.candidates(feat)):
            if not t.match(program):
                continue
            pred = self.cost.predict(t.name, feat)
            if pred.worth_trying:
                ranked.append((STAGES.index(t.stage), pos, PlannedTransform(t, pred)))
        return [p for _, _, p in sorted(ranked, key=lambda r: r[:2])]
