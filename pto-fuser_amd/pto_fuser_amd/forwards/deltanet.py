"""The chunked DeltaNet forward as a Program (src/pto_fuser/forwards/deltanet.py:23-111).

DeltaNet is GDN without decay.  Unlike the GDN program this one exposes every intermediate the
reference's worked example returns — A, T, W, U, v_new, h_state (the pre-update state per chunk)
and o — so a staged run and the fused kernels can be compared stage by stage:

  1. kkt       A = tril((β·k)·kᵀ, -1)
  2. solve     T = (I + A)⁻¹                    (opaque)
  3. recompute W = T·(β·k), U = T·(β·v)
  4. scan      per chunk: v_new = U − W·S, S += kᵀ·v_new
  5. chunk_o   o = scale·(q·h_state + tril(q·kᵀ)·v_new)
"""
from __future__ import annotations

from typing import Dict, List

import torch

from ..ir import Program
from ._builder import ProgramBuilder

__all__ = ["build_deltanet_program", "make_inputs", "DELTANET_OUTPUTS"]

DELTANET_OUTPUTS = ["A", "T", "W", "U", "v_new", "h_state", "o"]


def build_deltanet_program(B: int, H: int, nc: int, C: int, D: int, scale: float,
                           work=torch.bfloat16) -> Program:
    """Inputs q, k, v [B,H,nc,C,D], beta [B,H,nc,C]; outputs A, T, W, U, v_new, h_state, o."""
    M, N = B * H * nc, B * H
    p = ProgramBuilder(work)
    p.op("beta_u", "reshape", "beta", shape=[B, H, nc, C, 1])
    p.glue("kb", "mul", ["beta_u", "k"])
    p.glue("vb", "mul", ["beta_u", "v"])
    p.op("k_h", "cast", "k", dtype=work)
    p.op("q_h", "cast", "q", dtype=work)
    for src, dst in (("kb", "kbF"), ("vb", "vbF"), ("k_h", "kF"), ("q_h", "qF")):
        p.op(dst + "_r", "reshape", src, shape=[M, C, D])
        p.op(dst, "contiguous", dst + "_r")
    p.einsum("Araw", "nid,njd->nij", "kbF", "kF")
    p.glue("A_t", "tril", "Araw", diagonal=-1)
    p.op("A", "contiguous", "A_t")
    p.opaque("T_raw", "tri_inv_rec_unroll", "A")
    p.op("T", "cast", "T_raw", dtype=work)
    p.einsum("W_m", "nij,njd->nid", "T", "kbF")
    p.op("W", "reshape", "W_m", shape=[B, H, nc, C, D])
    p.einsum("U_m", "nij,njd->nid", "T", "vbF")
    p.op("U", "reshape", "U_m", shape=[B, H, nc, C, D])
    p.op("Wb", "reshape", "W", shape=[N, nc, C, D])
    p.op("Ub", "reshape", "U", shape=[N, nc, C, D])
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
        p.einsum(f"dS{c}", "nid,nie->nde", f"kc{c}", f"vn{c}")
        S = p.glue(f"S{c + 1}", "add", [S, f"dS{c}"])
    p.op("h_bh", "stack", snaps, dim=1)
    p.op("h_state", "reshape", "h_bh", shape=[B, H, nc, D, D])
    p.op("vn_bh", "stack", vns, dim=1)
    p.op("v_new", "reshape", "vn_bh", shape=[B, H, nc, C, D])
    p.op("h_flat_r", "reshape", "h_bh", shape=[M, D, D])
    p.op("h_flat", "contiguous", "h_flat_r")
    p.op("vn_flat_r", "reshape", "vn_bh", shape=[M, C, D])
    p.op("vn_flat", "contiguous", "vn_flat_r")
    p.einsum("o_inter", "nid,nde->nie", "qF", "h_flat")
    p.einsum("Aqk_raw", "nid,njd->nij", "qF", "kF")
    p.glue("Aqk_t", "tril", "Aqk_raw", diagonal=0)
    p.op("Aqk", "contiguous", "Aqk_t")
    p.einsum("o_intra", "nij,nje->nie", "Aqk", "vn_flat")
    p.glue("o_sum", "add", ["o_inter", "o_intra"], out_dtype=torch.float32)
    p.glue("o_s", "scale", "o_sum", out_dtype=torch.float32, scalar=scale)
    p.op("o", "reshape", "o_s", shape=[B, H, nc, C, D])
    return p.program(["q", "k", "v", "beta"], DELTANET_OUTPUTS)


def make_inputs(B, H, nc, C, D, device="cpu", dtype=torch.bfloat16, seed: int = 0
                ) -> Dict[str, torch.Tensor]:
    """The reference example's DeltaNet operands (deltanet.py:102-111): q, k L2-normalised,
    v ~ 0.1·N(0,1), beta ~ 0.5·U(0,1); seeded CPU draws moved to ``device``."""
    gen = torch.Generator().manual_seed(seed)
    nrm = torch.nn.functional.normalize
    k = nrm(torch.randn(B, H, nc, C, D, generator=gen), dim=-1)
    q = nrm(torch.randn(B, H, nc, C, D, generator=gen), dim=-1)
    v = torch.randn(B, H, nc, C, D, generator=gen) * 0.1
    beta = torch.rand(B, H, nc, C, generator=gen) * 0.5
    out = dict(q=q.to(dtype), k=k.to(dtype), v=v.to(dtype), beta=beta.to(dtype))
    return {n: t.to(device) for n, t in out.items()}
