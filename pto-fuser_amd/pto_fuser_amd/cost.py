"""Cost model: the heuristic that ranks transforms before the verifier measures them
(src/pto_fuser/cost.py:1-139), re-seeded for MI355X (CDNA4).

The reference seeds its predictions from a measured NPU grid (launch/dispatch-bound at small head
count, bandwidth-bound at large).  Here every prediction is a first-principles estimate of the
time a rewrite saves per forward under HIP-graph replay, in microseconds:

    saved_us = saved_HBM_bytes / HBM_EFFECTIVE_BPS * 1e6 + saved_graph_nodes * GRAPH_NODE_US

with MI355X constants: 8 TB/s HBM3E, of which a streaming elementwise / small-GEMM kernel reaches
about 60 % (HBM_EFFECTIVE_BPS); about 1 µs of launch gap per kernel node inside a replayed graph
(GRAPH_NODE_US); 256 CUs (CU_COUNT).  The estimate ranks and prunes; the verifier's measurement
decides, and the compilation report shows both so the constants can be recalibrated.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

__all__ = ["Features", "Prediction", "CostModel", "HBM_PEAK_BPS", "HBM_EFFECTIVE_BPS",
           "GRAPH_NODE_US", "CU_COUNT"]

HBM_PEAK_BPS = 8.0e12
HBM_EFFECTIVE_BPS = 0.6 * HBM_PEAK_BPS
GRAPH_NODE_US = 1.0
CU_COUNT = 256


@dataclass(frozen=True)
class Features:
    """Shape / dtype signature of a chunked delta-rule forward (the transforms' options)."""
    B: int
    H: int
    nc: int
    C: int
    D: int
    dtype: torch.dtype = torch.bfloat16
    per_dim_gate: bool = False

    @property
    def T(self) -> int:
        return self.nc * self.C

    @property
    def M(self) -> int:
        """Chunk-parallel batch (one workgroup per chunk in the parallel stages)."""
        return self.B * self.H * self.nc

    @property
    def N(self) -> int:
        """Scan chains, one per (b, h)."""
        return self.B * self.H

    @property
    def esize(self) -> int:
        return 4 if self.dtype in (torch.float32, torch.float64) else 2

    @property
    def regime(self) -> str:
        """launch-bound: the chunk-parallel stages have fewer workgroups than the GPU has CUs, so
        launch gaps and latency dominate.  bandwidth-bound: even the sequential scan (one
        workgroup per chain and 32-column state slice) fills every CU.  crossover in between."""
        if self.M < CU_COUNT:
            return "launch-bound"
        if self.N * max(1, self.D // 32) >= CU_COUNT:
            return "bandwidth-bound"
        return "crossover"


@dataclass
class Prediction:
    """Predicted µs saved per forward (> 0 = expected win) plus the rationale; ``v2`` selects
    between a fused kernel's two registry keys."""
    benefit: float
    rationale: str
    v2: Optional[bool] = None

    @property
    def worth_trying(self) -> bool:
        return self.benefit > 0


def _us(nbytes: float, nodes: float) -> float:
    return nbytes / HBM_EFFECTIVE_BPS * 1e6 + nodes * GRAPH_NODE_US


class CostModel:
    """First-principles MI355X estimates over the transform library."""

    def predict(self, transform_name: str, f: Features) -> Prediction:
        e, C, D, M, N, nc = f.esize, f.C, f.D, f.M, f.N, f.nc
        v2 = C * D >= 4096
        if transform_name in ("lower-resident-scan", "lower-perdim-scan"):
            # staged: per chunk and chain ~10 kernels; the state S (D*D) is read/written ~10x
            # (two contractions, mul, add, the snapshot stack) and the C*D operands ~9x.
            # fused: S stays in registers; one snapshot write per chunk + 3 operand reads,
            # then one batched W·h contraction and a subtraction rebuild v_new.
            staged = N * nc * (10 * D * D * e + 9 * C * D * e)
            fused = N * nc * (D * D * e + 3 * C * D * e) + M * (3 * C * D * e + D * D * e)
            saved = _us(staged - fused, 10 * nc - 4)
            return Prediction(saved, f"S kept in registers: {nc} chunks x ~10 kernels and "
                                     f"{(staged - fused) / 1e6:.1f} MB of state traffic removed")
        if transform_name in ("fuse-gdn-forward", "fuse-kda-forward"):
            # staged: every stage through HBM (the kkt score, T, W/U, the per-chunk state and
            # v_new, the chunk_o score) and ~10 kernels per chunk for the unrolled scan;
            # fused: q, k, v, gates in, o out, plus the WY factors once through HBM.
            staged = N * nc * (10 * D * D * e + 9 * C * D * e) + M * (6 * C * C * 4 + 8 * C * D * e)
            fused = M * (3 * C * D * e + C * D * 4 + 4 * C * D * e + C * C * e)
            saved = _us(max(staged - fused, 0), 10 * nc + 20)
            return Prediction(saved, f"whole forward in 2 kernels: {(staged - fused) / 1e6:.1f} MB "
                                     f"of stage traffic and ~{10 * nc + 20} launches removed")
        if transform_name in ("fuse-chunk-o-flash", "fuse-perdim-chunk-o-flash"):
            # the [M,C,C] score is written in fp32, cast, masked/gated and re-read by the
            # second contraction in the staged form; the flash kernel keeps it in LDS.
            saved = _us(M * C * C * (4 + 4 + 3 * e + e), 3)
            return Prediction(saved, f"chunk_o score ({M * C * C * 4 / 1e6:.1f} MB fp32) never "
                                     f"leaves LDS; 4 kernels -> 1")
        if transform_name == "fuse-contraction-epilogue":
            saved = _us(M * C * C * (4 + 4 + 4 * e), 3)
            return Prediction(saved, "gate/mask epilogue applied in registers: one [M,C,C] "
                                     "score round trip and 3 kernels removed per site", v2=v2)
        if transform_name == "enable-direct-reads":
            return Prediction(0.5, "contract strided views directly (skips operand copies); "
                                   "layout-dependent, measured by the verifier")
        if transform_name == "enable-fused-store":
            return Prediction(0.25, "leave permuted contraction results as views")
        return Prediction(0.0, "unknown transform — no prediction")
