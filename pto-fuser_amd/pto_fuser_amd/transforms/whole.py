"""Whole-forward rewrites: a canonical GDN or KDA program -> the fused forward of this build.

The reference's compile stack stops at per-stage fused kernels (the resident scan, the gated
score, the chunk_o flash); its whole forward still runs as several kernels with HBM round trips
between them.  This build also has each forward as two kernels (``ops.gdn_chunk_forward``,
``ops.kda_chunk_forward``: a chunk-parallel kernel that forms the WY factors, then the scan with
the output fused in).  ``FuseGdnForward`` / ``FuseKdaForward`` hand the compile stack that option:
they replace every step of a program that computes the forward from the builder's inputs with one
``FusedNode`` (``gdn_forward`` / ``kda_forward``) reading qF, kF, vF, the fp32 cumulative gate
``g_native`` and ``beta_native``.

A program qualifies when it is the builder's forward (its family's coefficient among the inputs,
the opaque ``tri_inv_rec_unroll`` solve, the ``o_s`` scale step, output ``o`` only) and its shape
is one the fused kernels run (C = 64 or 128 — the kernels run 64-token chunks, and a 128-token
program regroups the same arithmetic — and D = 128).  The
scale is read from the ``o_s`` step, so the fused node computes the same function; the compile
driver still verifies it against the canonical program before keeping it.

These transforms are opt-in (``Policy(whole_forward=True)``): the default pipeline keeps the
reference's per-stage lowering so its compilation reports stay comparable.
"""
from __future__ import annotations

from typing import Optional

import torch

from ..ir import FusedNode, OpaqueNode, Program, VecGlueNode
from ..transform import Transform, TransformResult

__all__ = ["FuseGdnForward", "FuseKdaForward"]

_WHOLE_KERNELS = ("gdn_forward", "kda_forward")
_NATIVE = ("qF", "kF", "vF", "g_native", "beta_native")


class _WholeForward(Transform):
    family_input = ""
    kernel = ""
    stage = "whole"

    def __init__(self, B: int, H: int, nc: int, C: int, D: int,
                 work: torch.dtype = torch.bfloat16) -> None:
        self.B, self.H, self.nc, self.C, self.D = B, H, nc, C, D
        self.work = work

    def _shape_ok(self) -> bool:
        return self.C in (64, 128) and self.D == 128

    def _scale(self, program: Program) -> Optional[float]:
        """The output scale when ``program`` is the builder's forward of this family, else None."""
        if any(isinstance(n, FusedNode) and n.kernel in _WHOLE_KERNELS for n in program.nodes):
            return None
        if self.family_input not in program.inputs or not all(n in program.inputs
                                                              for n in _NATIVE):
            return None
        if list(program.outputs) != ["o"] or not self._shape_ok():
            return None
        if not any(isinstance(n, OpaqueNode) and n.kernel == "tri_inv_rec_unroll"
                   for n in program.nodes):
            return None
        for n in program.nodes:
            if isinstance(n, VecGlueNode) and n.output == "o_s" and n.op == "scale":
                return float(n.params["scalar"])
        return None

    def match(self, program: Program) -> int:
        return 1 if self._scale(program) is not None else 0

    def apply(self, program: Program) -> TransformResult:
        scale = self._scale(program)
        if scale is None:
            return TransformResult(program, False, 0, "not a canonical forward of this family")
        node = FusedNode(kernel=self.kernel, inputs=list(_NATIVE), outputs=["o"],
                         params={"B": self.B, "H": self.H, "nc": self.nc, "C": self.C,
                                 "D": self.D, "scale": scale},
                         subsumes=[f"{len(program.nodes)} staged steps (kkt, solve, WY, "
                                   f"{self.nc}-chunk scan, chunk_o)"])
        new = Program(nodes=[node], inputs=list(program.inputs), outputs=["o"])
        return TransformResult(new, True, 1,
                               f"{len(program.nodes)} steps -> {self.kernel} (2 kernels)")


class FuseGdnForward(_WholeForward):
    """GDN (scalar per-token decay): the program with ``coef_vcs`` -> ``gdn_forward``."""
    name = "fuse-gdn-forward"
    summary = "whole GDN program -> gdn_forward FusedNode (chunk-local + scan/output kernels)"
    family_input = "coef_vcs"
    kernel = "gdn_forward"


class FuseKdaForward(_WholeForward):
    """KDA (per-channel decay): the program with ``coef_krest`` -> ``kda_forward``; the fused
    KDA kernels take bf16 or fp32 operands."""
    name = "fuse-kda-forward"
    summary = "whole KDA program -> kda_forward FusedNode (chunk-local + scan/output kernels)"
    family_input = "coef_krest"
    kernel = "kda_forward"
