"""The gated DeltaNet (GDN) forward as a canonical Program
(examples/attention/_gdn_full.py:37-50,103-235; src/pto_fuser/forwards/gdn.py:1-70).

``build_gdn_program`` emits the all-staged lowering: every stage its own contraction or glue
step, the cross-chunk scan unrolled over the chunks, the gates applied as host-computed
coefficient tensors (``prepare_gdn_bindings``).  It is the correctness floor the compile driver
verifies every rewrite against and the starting point the transforms match on — its node and
input names are that contract:

  kkt       A   = tril((kF·kFᵀ) ⊙ coefA, -1)                   Araw, Ag, A_t, A
  solve     T   = (I + A)⁻¹                                     T_raw (opaque), Tm
  wy        W, U = T·(kF ⊙ coef_kb), T·(vF ⊙ coef_vb)          kb, vb, W_m, U_m, Wb, Ub, kb5
  scan      per chunk c: vn_c = U_c − W_c·S;                    S0, Wc{c}, WS{c}, Uc{c}, vn{c},
            S ← e^{G_last}·S + kᵀ·(vn_c ⊙ e^{G_last−G})          vcs{c}, vn2{c}, kc{c}, dS{c},
                                                                sc{c}, Sd{c}, S{c+1}, h_flat, vn_flat
  chunk_o   o = scale·((qF·h) ⊙ coef_qg + ((qF·kFᵀ) ⊙ coef_o)·vn)  o_inter_m, o_inter, Aqk,
                                                                Aqk_g, Aqk_c, o_intra, o_sum, o_s, o

The direct fused path of this build (``ops.gdn_chunk_forward``) computes the same function in two
kernels; this Program exists for the compile stack.
"""
from __future__ import annotations

from typing import Dict, List

import torch

from ..ir import Program
from ._builder import ProgramBuilder

__all__ = ["make_gdn_inputs", "prepare_gdn_bindings", "build_gdn_program",
           "GDN_PROGRAM_INPUTS"]

GDN_PROGRAM_INPUTS = ["qF", "kF", "vF", "coefA", "coef_kb", "coef_vb", "coef_qg", "coef_o",
                      "coef_vcs", "coef_S", "g_native", "beta_native", "beta_native_ones"]


def make_gdn_inputs(B, H, nc, C, D, device="cpu", dtype=torch.bfloat16, seed: int = 0
                    ) -> Dict[str, torch.Tensor]:
    """Operands in the [B,H,nc,C,D] / [B,H,nc,C] layout with the reference example's
    distributions (_gdn_full.py:37-50): q, k L2-normalised N(0,1) rows, v ~ N(0,1),
    beta ~ U(0,1), g_in = logsigmoid(N(0,1)).  Drawn on the CPU from a seeded generator, then
    moved to ``device``."""
    gen = torch.Generator().manual_seed(seed)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(B, H, nc, C, D, generator=gen), dim=-1)
    k = nrm(torch.randn(B, H, nc, C, D, generator=gen), dim=-1)
    v = torch.randn(B, H, nc, C, D, generator=gen)
    beta = torch.rand(B, H, nc, C, generator=gen)
    g_in = torch.nn.functional.logsigmoid(torch.randn(B, H, nc, C, generator=gen))
    out = dict(q=q.to(dtype), k=k.to(dtype), v=v.to(dtype), beta=beta.to(dtype), g_in=g_in)
    return {n: t.to(device) for n, t in out.items()}


def _safe_exp(x: torch.Tensor) -> torch.Tensor:
    return torch.where(x <= 0, torch.exp(torch.clamp(x, max=0.0)), torch.zeros_like(x))


def prepare_gdn_bindings(q, k, v, beta, g_in, work=torch.bfloat16) -> Dict[str, torch.Tensor]:
    """Flatten the operands to the Program's batch layouts and compute the gate coefficients
    (_gdn_full.py:103-144).  M = B·H·nc (chunk-parallel stages), N = B·H (scan chains).
    Coefficients are computed in fp32 and stored in ``work``; ``g_native`` (the within-chunk
    cumulative log decay) and the native beta tensors stay fp32, the dtype the HIP stage kernels
    read."""
    B, H, nc, C, D = q.shape
    M, N = B * H * nc, B * H
    G = g_in.float().cumsum(dim=3)                               # [B,H,nc,C]
    Gi, Gj = G.unsqueeze(-1), G.unsqueeze(-2)
    bt = beta.float()
    G_last = G[..., -1:]
    rows = torch.arange(C, device=q.device)
    causal = (rows[:, None] >= rows[None, :]).float()

    def flat(t, *tail):
        return t.reshape(M, *tail).to(work).contiguous()

    def chains(t, *tail):
        return t.reshape(N, nc, *tail).to(work).contiguous()

    return {
        "qF": flat(q, C, D), "kF": flat(k, C, D), "vF": flat(v, C, D),
        "coefA": flat(_safe_exp(Gi - Gj) * bt.unsqueeze(-1), C, C),
        "coef_kb": flat((bt * torch.exp(G)).unsqueeze(-1), C, 1),
        "coef_vb": flat(bt.unsqueeze(-1), C, 1),
        "coef_qg": flat(torch.exp(G).unsqueeze(-1), C, 1),
        "coef_o": flat(torch.exp(torch.clamp(Gi - Gj, max=0.0)) * causal, C, C),
        "coef_vcs": chains(torch.exp(G_last.unsqueeze(-1) - Gi), C, 1),
        "coef_S": chains(torch.exp(G_last).unsqueeze(-1), 1, 1),
        "g_native": G.reshape(M, C).contiguous(),
        "beta_native": bt.reshape(M, C).contiguous(),
        "beta_native_ones": torch.ones(M, C, device=q.device, dtype=torch.float32),
    }


def build_gdn_program(B, H, nc, C, D, scale, work=torch.bfloat16) -> Program:
    """The canonical all-staged GDN forward; output ``o`` [B,H,nc,C,D] fp32."""
    M, N = B * H * nc, B * H
    p = ProgramBuilder(work)
    # kkt
    p.einsum("Araw", "nid,njd->nij", "kF", "kF")
    p.glue("Ag", "mul", ["Araw", "coefA"])
    p.glue("A_t", "tril", "Ag", diagonal=-1)
    p.op("A", "contiguous", "A_t")
    # (I + A)^-1
    p.opaque("T_raw", "tri_inv_rec_unroll", "A")
    p.op("Tm", "cast", "T_raw", dtype=work)
    # WY
    p.glue("kb", "mul", ["kF", "coef_kb"])
    p.glue("vb", "mul", ["vF", "coef_vb"])
    p.einsum("W_m", "nij,njd->nid", "Tm", "kb")
    p.einsum("U_m", "nij,njd->nid", "Tm", "vb")
    p.op("Wb", "reshape", "W_m", shape=[N, nc, C, D])
    p.op("Ub", "reshape", "U_m", shape=[N, nc, C, D])
    p.op("kb5", "reshape", "kF", shape=[N, nc, C, D])
    # scan, unrolled; S written back every chunk
    p.op("S0", "zeros", "Wb", shape=[N, D, D], dtype=work)
    snaps: List[str] = []
    vns: List[str] = []
    S = "S0"
    for c in range(nc):
        snaps.append(S)
        p.op(f"Wc{c}_s", "slice", "Wb", axis=1, index=c)
        p.op(f"Wc{c}", "contiguous", f"Wc{c}_s")
        p.einsum(f"WS{c}", "nid,nde->nie", f"Wc{c}", S)
        p.op(f"Uc{c}", "slice", "Ub", axis=1, index=c)
        vns.append(p.glue(f"vn{c}", "sub", [f"Uc{c}", f"WS{c}"]))
        p.op(f"vcs{c}", "slice", "coef_vcs", axis=1, index=c)
        p.glue(f"vn2{c}", "mul", [f"vn{c}", f"vcs{c}"])
        p.op(f"kc{c}_s", "slice", "kb5", axis=1, index=c)
        p.op(f"kc{c}", "contiguous", f"kc{c}_s")
        p.einsum(f"dS{c}", "nid,nie->nde", f"kc{c}", f"vn2{c}")
        p.op(f"sc{c}", "slice", "coef_S", axis=1, index=c)
        p.glue(f"Sd{c}", "mul", [S, f"sc{c}"])
        S = p.glue(f"S{c + 1}", "add", [f"Sd{c}", f"dS{c}"])
    p.op("h_bh", "stack", snaps, dim=1)
    p.op("h_flat", "reshape", "h_bh", shape=[M, D, D])
    p.op("vn_bh", "stack", vns, dim=1)
    p.op("vn_flat", "reshape", "vn_bh", shape=[M, C, D])
    # chunk_o
    p.einsum("o_inter_m", "nid,nde->nie", "qF", "h_flat")
    p.glue("o_inter", "mul", ["o_inter_m", "coef_qg"])
    p.einsum("Aqk", "nid,njd->nij", "qF", "kF")
    p.glue("Aqk_g", "mul", ["Aqk", "coef_o"])
    p.op("Aqk_c", "contiguous", "Aqk_g")
    p.einsum("o_intra", "nij,nje->nie", "Aqk_c", "vn_flat")
    p.glue("o_sum", "add", ["o_inter", "o_intra"], out_dtype=torch.float32)
    p.glue("o_s", "scale", "o_sum", out_dtype=torch.float32, scalar=scale)
    p.op("o", "reshape", "o_s", shape=[B, H, nc, C, D])
    return p.program(GDN_PROGRAM_INPUTS, ["o"])

