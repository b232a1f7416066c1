"""Forward-shaped structural rewrites: the resident-state scans of GDN and KDA
(src/pto_fuser/transforms/gdn.py, kda.py) and, opt-in with no reference counterpart, the
whole-forward rewrites onto the fused GDN / KDA kernels."""
from .gdn import LowerResidentScan
from .kda import LowerPerDimScan
from .whole import FuseGdnForward, FuseKdaForward

__all__ = ["LowerResidentScan", "LowerPerDimScan", "FuseGdnForward", "FuseKdaForward"]
