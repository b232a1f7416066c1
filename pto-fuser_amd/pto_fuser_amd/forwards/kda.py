"""The Kimi Delta Attention (KDA) forward as a canonical Program
(examples/attention/_kda_full.py:25-160).

KDA is GDN with a per-key-channel decay: the gate multiplies the contraction *operands*
(k ⊙ e^{G}, k ⊙ e^{−G}) instead of the score, and the scan decays state row d by e^{G_tot,d}.
Same equations and node vocabulary as ``forwards.gdn``; the input set differs (per-channel
coefficients), which is what keeps each family's transforms on their own program:

  kkt      A   = tril((kF ⊙ coef_ag)·(kF ⊙ coef_bg)ᵀ ⊙ coef_beta, -1)   a_op, b_op, Araw, Ag, A_t, A
  solve    T   = (I + A)⁻¹                                              T_raw, Tm
  wy       W, U = T·(kF ⊙ coef_wg), T·(vF ⊙ coef_ub)                    wk, vb, W_m, U_m
  scan     vn_c = U_c − W_c·S;  S ← coef_S,c ⊙ S + (k_c ⊙ coef_krest,c)ᵀ·vn_c
  chunk_o  o = scale·((qF ⊙ coef_ag)·h + tril((qF ⊙ coef_ag)·(kF ⊙ coef_bg)ᵀ)·vn)
"""
from __future__ import annotations

from typing import Dict, List

import torch

from ..ir import Program
from ._builder import ProgramBuilder

__all__ = ["make_kda_inputs", "prepare_kda_bindings", "build_kda_program", "KDA_PROGRAM_INPUTS"]

KDA_PROGRAM_INPUTS = ["qF", "kF", "vF", "coef_ag", "coef_bg", "coef_beta", "coef_wg", "coef_ub",
                      "coef_krest", "coef_S", "g_native", "beta_native"]


def make_kda_inputs(B, H, nc, C, D, device="cpu", dtype=torch.bfloat16, seed: int = 0
                    ) -> Dict[str, torch.Tensor]:
    """Operands with the reference example's distributions (_kda_full.py:25-39): q, k
    L2-normalised, v ~ N(0,1), beta = sigmoid(N(0,1)), per-channel g_in = −U(0,1)·0.05."""
    gen = torch.Generator().manual_seed(seed)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(B, H, nc, C, D, generator=gen), dim=-1)
    k = nrm(torch.randn(B, H, nc, C, D, generator=gen), dim=-1)
    v = torch.randn(B, H, nc, C, D, generator=gen)
    beta = torch.sigmoid(torch.randn(B, H, nc, C, generator=gen))
    g_in = -torch.rand(B, H, nc, C, D, generator=gen) * 0.05
    out = dict(q=q.to(dtype), k=k.to(dtype), v=v.to(dtype), beta=beta.to(dtype), g_in=g_in)
    return {n: t.to(device) for n, t in out.items()}


def prepare_kda_bindings(q, k, v, beta, g_in, work=torch.bfloat16) -> Dict[str, torch.Tensor]:
    """Per-channel gate coefficients (_kda_full.py:78-103), computed in fp32, stored in
    ``work``.  ``g_native`` (the within-chunk cumulative log decay, [M, C, D]) and
    ``beta_native`` ([M, C]) stay fp32: the staged program does not read them, the whole-forward
    rewrite hands them to the fused KDA kernels."""
    B, H, nc, C, D = q.shape
    M, N = B * H * nc, B * H
    G = g_in.float().cumsum(dim=3)                       # [B,H,nc,C,D]
    bt = beta.float().unsqueeze(-1)                      # [B,H,nc,C,1]
    G_tot = G[:, :, :, -1:, :]                           # [B,H,nc,1,D]

    def flat(t, *tail):
        return t.reshape(M, *tail).to(work).contiguous()

    def chains(t, *tail):
        return t.reshape(N, nc, *tail).to(work).contiguous()

    return {
        "qF": flat(q, C, D), "kF": flat(k, C, D), "vF": flat(v, C, D),
        "coef_ag": flat(torch.exp(G), C, D), "coef_bg": flat(torch.exp(-G), C, D),
        "coef_beta": flat(bt.expand(B, H, nc, C, 1), C, 1),
        "coef_wg": flat(torch.exp(G) * bt, C, D),
        "coef_ub": flat(bt.expand(B, H, nc, C, 1), C, 1),
        "coef_krest": chains(torch.exp(G_tot - G), C, D),
        "coef_S": chains(torch.exp(G_tot).reshape(B, H, nc, D, 1), D, 1),
        "g_native": G.reshape(M, C, D).contiguous(),
        "beta_native": beta.float().reshape(M, C).contiguous(),
    }


def build_kda_program(B, H, nc, C, D, scale, work=torch.bfloat16) -> Program:
    """The canonical all-staged KDA forward; output ``o`` [B,H,nc,C,D] fp32."""
    M, N = B * H * nc, B * H
    p = ProgramBuilder(work)
    p.glue("a_op", "mul", ["kF", "coef_ag"])
    p.glue("b_op", "mul", ["kF", "coef_bg"])
    p.einsum("Araw", "nid,njd->nij", "a_op", "b_op")
    p.glue("Ag", "mul", ["Araw", "coef_beta"])
    p.glue("A_t", "tril", "Ag", diagonal=-1)
    p.op("A", "contiguous", "A_t")
    p.opaque("T_raw", "tri_inv_rec_unroll", "A")
    p.op("Tm", "cast", "T_raw", dtype=work)
    p.glue("wk", "mul", ["kF", "coef_wg"])
    p.glue("vb", "mul", ["vF", "coef_ub"])
    p.einsum("W_m", "nij,njd->nid", "Tm", "wk")
    p.einsum("U_m", "nij,njd->nid", "Tm", "vb")
    p.op("Wb", "reshape", "W_m", shape=[N, nc, C, D])
    p.op("Ub", "reshape", "U_m", shape=[N, nc, C, D])
    p.op("kb5", "reshape", "kF", shape=[N, nc, C, D])
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
        p.op(f"kc{c}_s", "slice", "kb5", axis=1, index=c)
        p.op(f"kc{c}", "contiguous", f"kc{c}_s")
        p.op(f"krc{c}", "slice", "coef_krest", axis=1, index=c)
        p.glue(f"krest{c}", "mul", [f"kc{c}", f"krc{c}"])
        p.einsum(f"dS{c}", "nid,nie->nde", f"krest{c}", f"vn{c}")
        p.op(f"sc{c}", "slice", "coef_S", axis=1, index=c)
        p.glue(f"Sd{c}", "mul", [S, f"sc{c}"])
        S = p.glue(f"S{c + 1}", "add", [f"Sd{c}", f"dS{c}"])
    p.op("h_bh", "stack", snaps, dim=1)
    p.op("h_flat", "reshape", "h_bh", shape=[M, D, D])
    p.op("vn_bh", "stack", vns, dim=1)
    p.op("vn_flat", "reshape", "vn_bh", shape=[M, C, D])
    p.glue("q_eff", "mul", ["qF", "coef_ag"])
    p.einsum("o_inter", "nid,nde->nie", "q_eff", "h_flat")
    p.glue("k_eff", "mul", ["kF", "coef_bg"])
    p.einsum("Aqk", "nid,njd->nij", "q_eff", "k_eff")
    p.glue("Aqk_t", "tril", "Aqk", diagonal=0)
    p.op("Aqk_c", "contiguous", "Aqk_t")
    p.einsum("o_intra", "nij,nje->nie", "Aqk_c", "vn_flat")
    p.glue("o_sum", "add", ["o_inter", "o_intra"], out_dtype=torch.float32)
    p.glue("o_s", "scale", "o_sum", out_dtype=torch.float32, scalar=scale)
    p.op("o", "reshape", "o_s", shape=[B, H, nc, C, D])
    return p.program(KDA_PROGRAM_INPUTS, ["o"])
