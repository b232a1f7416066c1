"""Stand-alone stage programs for the staged-vs-fused decision
(src/pto_fuser/forwards/fused_stages.py:1-163).

Each stage comes in two lowerings over the same inputs, so ``fusion.decide`` can gate and time
one against the other:

* ``chunk_h_scan`` — staged: the scan unrolled into per-chunk contractions and glue, S through
  HBM every chunk; fused: one ``chunk_h_scan`` node (S in registers).  Token-major operands
  w, u, k [B, nc, C, H, D], decay [B, H, nc].
* ``kkt_gated`` — fused only here (one node over the [1, T, H, D] token layout); its staged
  twin is the kkt region of the GDN program.

The reference fixes C = D = 128 (its prototype tile); here C and D are parameters (default 128).
"""
from __future__ import annotations

from typing import Dict

import torch

from ..ir import EinsumNode, FusedNode, Program, TensorOp, VecGlueNode

__all__ = ["make_scan_inputs", "build_scan_fused_program", "build_scan_staged_program",
           "make_kkt_inputs", "build_kkt_fused_program"]


def make_scan_inputs(B: int, H: int, nc: int, C: int = 128, D: int = 128, device="cpu",
                     dtype=torch.bfloat16, seed: int = 0) -> Dict[str, torch.Tensor]:
    """Token-major scan operands with contractive magnitudes (the reference's run_scan
    scales: w, k ~ 0.02·N, u ~ 0.05·N, decay ~ 0.7 + 0.2·U)."""
    gen = torch.Generator().manual_seed(seed)
    w = torch.randn(B, nc, C, H, D, generator=gen) * 0.02
    k = torch.randn(B, nc, C, H, D, generator=gen) * 0.02
    u = torch.randn(B, nc, C, H, D, generator=gen) * 0.05
    decay = 0.7 + 0.2 * torch.rand(B, H, nc, generator=gen)
    return {"w": w.to(dtype).to(device), "u": u.to(dtype).to(device),
            "k": k.to(dtype).to(device), "decay": decay.float().to(device)}


def build_scan_fused_program(B: int, H: int, nc: int) -> Program:
    node = FusedNode(kernel="chunk_h_scan", inputs=["w", "u", "k", "decay"],
                     outputs=["h_out", "final"], params={"B": B, "H": H, "nc": nc},
                     subsumes=["the nc per-chunk W·S / kᵀ·v contraction pairs + residual glue"])
    return Program(nodes=[node], inputs=["w", "u", "k", "decay"], outputs=["h_out", "final"])


def build_scan_staged_program(B: int, H: int, nc: int, C: int = 128, D: int = 128,
                              work=torch.bfloat16) -> Program:
    """The unrolled scan over the N = B·H chains; outputs in the fused node's layouts
    (h_out [B, nc, H, D, D], final [B, H, D, D])."""
    N = B * H
    nodes = []
    for name in ("w", "u", "k"):
        nodes.append(TensorOp("permute", [name], f"{name}_p", {"dims": (0, 3, 1, 2, 4)}))
        nodes.append(TensorOp("reshape", [f"{name}_p"], f"{name}_b", {"shape": (N, nc, C, D)}))
    nodes.append(TensorOp("reshape", ["decay"], "decay_b", {"shape": (N, nc)}))
    nodes.append(TensorOp("zeros", ["w_b"], "S0", {"shape": (N, D, D), "dtype": work}))
    snaps, S = [], "S0"
    for c in range(nc):
        snaps.append(S)
        for nm in ("w", "k", "u"):
            nodes.append(TensorOp("slice", [f"{nm}_b"], f"{nm}_c{c}", {"axis": 1, "index": c}))
        nodes.append(EinsumNode("ncd,nde->nce", [f"w_c{c}", S], f"WS{c}"))
        nodes.append(VecGlueNode("sub", [f"u_c{c}", f"WS{c}"], f"vc{c}", out_dtype=work))
        nodes.append(EinsumNode("ncd,nce->nde", [f"k_c{c}", f"vc{c}"], f"kv{c}"))
        nodes.append(TensorOp("slice", ["decay_b"], f"dec{c}", {"axis": 1, "index": c}))
        nodes.append(TensorOp("reshape", [f"dec{c}"], f"decr{c}", {"shape": (N, 1, 1)}))
        nodes.append(VecGlueNode("mul", [S, f"decr{c}"], f"Sdec{c}"))
        S = f"S{c + 1}"
        nodes.append(VecGlueNode("add", [f"Sdec{c}", f"kv{c}"], S, out_dtype=work))
    nodes.append(TensorOp("stack", snaps, "h_b", {"dim": 1}))
    nodes.append(TensorOp("reshape", ["h_b"], "h_bhn", {"shape": (B, H, nc, D, D)}))
    nodes.append(TensorOp("permute", ["h_bhn"], "h_out", {"dims": (0, 2, 1, 3, 4)}))
    nodes.append(TensorOp("reshape", [S], "final", {"shape": (B, H, D, D)}))
    return Program(nodes=nodes, inputs=["w", "u", "k", "decay"], outputs=["h_out", "final"])


def make_kkt_inputs(nc: int, H: int, C: int = 128, D: int = 128, device="cpu",
                    dtype=torch.bfloat16, seed: int = 0) -> Dict[str, torch.Tensor]:
    """Gated-kkt operands on the token layout: k [1, T, H, D] L2-normalised, g_sum [1, T, H]
    (logsigmoid(N) summed within each chunk), beta [1, T, H] ~ U(0,1)."""
    gen = torch.Generator().manual_seed(seed)
    T = nc * C
    k = torch.nn.functional.normalize(torch.randn(1, T, H, D, generator=gen), dim=-1)
    beta = torch.rand(1, T, H, generator=gen)
    g_in = torch.nn.functional.logsigmoid(torch.randn(1, T, H, generator=gen))
    g_sum = g_in.reshape(1, nc, C, H).cumsum(2).reshape(1, T, H)
    return {"k": k.to(dtype).to(device), "g_sum": g_sum.float().to(device),
            "beta": beta.float().to(device)}


def build_kkt_fused_program(nc: int, H: int) -> Program:
    node = FusedNode(kernel="kkt_gated", inputs=["k", "g_sum", "beta"], outputs=["L"],
                     params={"nc": nc, "H": H},
                     subsumes=["k·kᵀ einsum + gated/masked epilogue"])
    return Program(nodes=[node], inputs=["k", "g_sum", "beta"], outputs=["L"])
