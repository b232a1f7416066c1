"""Batched intra-chunk score for the chunked linear family (src/pto_fuser/transforms/chunked.py).

The chunked linear-attention programs (vanilla LA, RetNet, Mamba-2 with a scalar gate; GLA with a
per-channel gate) compute the intra-chunk score ``A_c = tril(q_c·k_cᵀ)`` once per chunk inside
the unrolled scan: ``nc`` small contractions plus ``nc`` mask steps.  ``BatchChunkIntraScore``
replaces them with one launch over all ``N·nc`` chunks of an existing stage kernel — the gated
score (``gated_qk_native_v2``, scalar log-gate ``g_intra``) or the per-channel prologue score
(``qk_prologue[_v2]``, operands prescaled by ``P`` / ``invP``) — and slices the per-chunk scores
back out of the batched result.  The gate kind is a construction option: the IR cannot tell a
scalar from a per-channel gate.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

from ..ir import EinsumNode, FusedNode, Program, TensorOp, VecGlueNode
from ..transform import Transform, TransformResult


def select_prologue_kernel(C: int, d_k: int) -> str:
    """The reference picks its L2-ring prologue variant at C·d_k >= 4096; both keys run the same
    HIP kernel here, the choice only names the node."""
    return "qk_prologue_v2" if C * d_k >= 4096 else "qk_prologue"


def _only_consumer(program: Program, name: str) -> Optional[int]:
    hits = [i for i, n in enumerate(program.nodes) if name in n.inputs]
    return hits[0] if len(hits) == 1 else None


class BatchChunkIntraScore(Transform):
    name = "batch-chunk-intra-score"
    summary = "nc per-chunk tril(q·kᵀ) intra scores -> one batched gated / prologue kernel"

    def __init__(self, N: int, nc: int, C: int, d_k: int, d_v: int,
                 per_dim_gate: bool = False, v2: Optional[bool] = None) -> None:
        self.N, self.nc, self.C, self.d_k, self.d_v = N, nc, C, d_k, d_v
        self.per_dim_gate, self.v2 = per_dim_gate, v2

    def _sites(self, program: Program) -> List[Tuple[int, int, str]]:
        """(score einsum index, tril index, masked score name) for each chunk's
        ``nid,njd->nij -> tril -> nij,nje->nie`` chain."""
        out = []
        for i, n in enumerate(program.nodes):
            if not (isinstance(n, EinsumNode) and n.equation == "nid,njd->nij"):
                continue
            t = _only_consumer(program, n.output)
            if t is None:
                continue
            tn = program.nodes[t]
            if not (isinstance(tn, VecGlueNode) and tn.op == "tril"):
                continue
            o = _only_consumer(program, tn.output)
            if o is None:
                continue
            on = program.nodes[o]
            if isinstance(on, EinsumNode) and on.equation == "nij,nje->nie":
                out.append((i, t, tn.output))
        return out

    def match(self, program: Program) -> int:
        if any(isinstance(n, FusedNode) and n.output == "A_all" for n in program.nodes):
            return 0
        return 1 if self._sites(program) else 0

    def apply(self, program: Program) -> TransformResult:
        sites = self._sites(program)
        if not sites:
            return TransformResult(program, False, 0, "no per-chunk intra scores")
        nc, C = self.nc, self.C
        if self.per_dim_gate:
            if self.v2 is None:
                kernel = select_prologue_kernel(C, self.d_k)
            else:
                kernel = "qk_prologue_v2" if self.v2 else "qk_prologue"
            batched = FusedNode(kernel=kernel, inputs=["q", "k", "P", "invP"], outputs=["A_all"],
                                params={"nc": nc, "H": self.N, "C": C, "D": self.d_k},
                                subsumes=[s for _, _, s in sites])
        else:
            batched = FusedNode(kernel="gated_qk_native_v2",
                                inputs=["q", "k", "g_intra", "beta_intra"], outputs=["A_all"],
                                params={"nc": nc, "H": self.N, "C": C, "D": self.d_k,
                                        "causal": True},
                                subsumes=[s for _, _, s in sites])
        nodes = [batched, TensorOp("reshape", ["A_all"], "A_allr",
                                   params={"shape": (self.N, nc, C, C)})]
        drop = {i for i, _, _ in sites} | {t for _, t, _ in sites}
        chunk_of = {t: c for c, (_, t, _) in enumerate(sites)}
        for idx, node in enumerate(program.nodes):
            if idx in chunk_of:
                nodes.append(TensorOp("slice", ["A_allr"], node.output,
                                      params={"axis": 1, "index": chunk_of[idx]}))
            elif idx not in drop:
                nodes.append(node)
        prog = Program(nodes=nodes, inputs=list(program.inputs), outputs=list(program.outputs))
        return TransformResult(prog, True, 1, f"{len(sites)} per-chunk intra scores -> "
                                              f"{batched.kernel}")
