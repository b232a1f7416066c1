"""Resident-state scan rewrite of the GDN program (src/pto_fuser/transforms/gdn.py:1-103).

The canonical GDN program (``forwards.gdn.build_gdn_program``) unrolls the cross-chunk scan:
per chunk a W·S contraction, a residual, a decay multiply, a kᵀ·v contraction and an add, with
the state S written to HBM every chunk.  ``LowerResidentScan`` replaces that region with the
``chunk_h_scan`` FusedNode — the HIP scan keeps S in registers for the whole chain — plus one
batched ``W·h`` contraction that rebuilds ``v_new`` for the output stage.  The node names it
matches are the builder's documented contract.
"""
from __future__ import annotations

from typing import List, Tuple

import torch

from ..dataflow import Dataflow, ProgramEdit
from ..ir import EinsumNode, FusedNode, Node, Program, TensorOp, VecGlueNode
from ..transform import Transform


def has_fused(program: Program, kernel_prefix: str) -> bool:
    return any(isinstance(n, FusedNode) and n.kernel.startswith(kernel_prefix)
               for n in program.nodes)


class _ResidentScan(Transform):
    """Shared rewrite of the scalar (GDN) and per-channel (KDA) scans.  Subclasses name the
    program input that identifies their family, the per-chunk node names of their unrolled scan,
    the coefficient that scales k, and whether the decay is per channel."""

    family_input = ""
    k_coef = ""
    k_scaled = ""
    perdim = False
    per_chunk: Tuple[str, ...] = ()

    def __init__(self, B: int, H: int, nc: int, C: int, D: int,
                 work: torch.dtype = torch.bfloat16) -> None:
        self.B, self.H, self.nc, self.C, self.D = B, H, nc, C, D
        self.M = B * H * nc
        self.work = work

    stage = "structural"
    no_site_note = "no canonical scan region"

    def sites(self, flow: Dataflow) -> List[set]:
        """The unrolled scan's steps (one site): every step binding a name of the canonical
        scan region, found by the builder's documented names."""
        program = flow.program
        if has_fused(program, "chunk_h_scan") or self.family_input not in program.inputs:
            return []
        if not all(flow.producer(n) is not None for n in ("S0", "h_flat", "vn_flat")):
            return []
        names = {"S0", "h_bh", "h_flat", "vn_bh", "vn_flat"}
        for c in range(self.nc):
            names.update(p.format(c=c, c1=c + 1) for p in self.per_chunk)
        steps = {i for n in names if (i := flow.producer(n)) is not None}
        return [steps] if steps else []

    def rewrite(self, flow: Dataflow, steps: set, edit: ProgramEdit) -> str:
        B, H, nc, C, D, M = self.B, self.H, self.nc, self.C, self.D, self.M
        new: List[Node] = [VecGlueNode("mul", ["kb5", self.k_coef], self.k_scaled,
                                       out_dtype=self.work)]
        # [N, nc, C, D] (heads outer) -> token-major [B, nc, C, H, D], the scan's layout
        for nm, src in (("sw", "Wb"), ("su", "Ub"), ("sk", self.k_scaled)):
            new.append(TensorOp("reshape", [src], f"{nm}5", params={"shape": [B, H, nc, C, D]}))
            new.append(TensorOp("permute", [f"{nm}5"], nm, params={"dims": (0, 2, 3, 1, 4)}))
        new.append(TensorOp("reshape", ["coef_S"], "sdecay",
                            params={"shape": [B, H, nc, D] if self.perdim else [B, H, nc]}))
        params = {"B": B, "H": H, "nc": nc}
        if self.perdim:
            params["perdim_decay"] = True
        new.append(FusedNode(kernel="chunk_h_scan", inputs=["sw", "su", "sk", "sdecay"],
                             outputs=["h_out_k", "final_k"], params=params,
                             subsumes=[f"{nc} per-chunk W·S / kᵀ·v contraction pairs + glue"]))
        new.append(TensorOp("permute", ["h_out_k"], "h_bhn", params={"dims": (0, 2, 1, 3, 4)}))
        new.append(TensorOp("reshape", ["h_bhn"], "h_flat", params={"shape": [M, D, D]}))
        new.append(EinsumNode("nid,nde->nie", ["W_m", "h_flat"], "WS_all", out_dtype=self.work,
                              read_mode="NN", fuse_out=False))
        new.append(VecGlueNode("sub", ["U_m", "WS_all"], "vn_flat", out_dtype=self.work))
        edit.replace(steps, new)
        return f"scan of {nc} chunks -> chunk_h_scan (state in registers)"


class LowerResidentScan(_ResidentScan):
    """GDN: scalar decay e^{G_last} per chunk; k scaled by e^{G_last - G} (``coef_vcs``)."""
    name = "lower-resident-scan"
    summary = "unrolled chunk_h scan -> chunk_h_scan FusedNode (state in registers)"
    family_input = "coef_vcs"
    k_coef = "coef_vcs"
    k_scaled = "k_vcs"
    perdim = False
    per_chunk = ("Wc{c}_s", "Wc{c}", "WS{c}", "Uc{c}", "vn{c}", "vcs{c}", "vn2{c}", "kc{c}_s",
                 "kc{c}", "dS{c}", "sc{c}", "Sd{c}", "S{c1}")
