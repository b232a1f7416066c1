"""Forward-shaped structural rewrites (src/pto_fuser/transforms/__init__.py): the resident-state
scans of GDN and KDA, the batched intra-chunk score of the chunked linear family, and (opt-in,
no reference counterpart) the whole-forward rewrites onto the fused GDN / KDA kernels."""
from .chunked import BatchChunkIntraScore
from .gdn import LowerResidentScan
from .kda import LowerPerDimScan
from .whole import FuseGdnForward, FuseKdaForward

__all__ = ["LowerResidentScan", "LowerPerDimScan", "BatchChunkIntraScore", "FuseGdnForward",
           "FuseKdaForward"]
