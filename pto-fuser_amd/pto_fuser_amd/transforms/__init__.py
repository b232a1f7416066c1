"""Forward-shaped structural rewrites (src/pto_fuser/transforms/__init__.py): the resident-state
scans of GDN and KDA and the batched intra-chunk score of the chunked linear family."""
from .chunked import BatchChunkIntraScore
from .gdn import LowerResidentScan
from .kda import LowerPerDimScan

__all__ = ["LowerResidentScan", "LowerPerDimScan", "BatchChunkIntraScore"]
