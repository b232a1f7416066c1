"""Seeded synthetic inputs for the delta-rule forwards (the model's a1 step).

The reference's ``make_gdn_inputs`` (examples/attention/_gdn_full.py:37-50) draws
beta ~ U(0,1) and g = logsigmoid(N(0,1)); the benchmark configurations of this build specify
other distributions, which these generators follow:

  q, k ~ N(0,1) then L2-normalised per token row; v ~ N(0,1); beta = sigmoid(N(0,1));
  g = -softplus(N(0,1)) * gate_scale (0.1 for GDN, a [.., dk] tensor with 0.05 for KDA,
  zero for DeltaNet); optional h0 ~ N(0, h0_std).

Everything is drawn on the CPU from one ``torch.Generator`` in the order q, k, v,
beta-logits, g-logits, h0, in float32; q/k/v are then rounded to ``dtype``.  The same seed gives
the same tensors on every machine, so the GPU run and the CPU oracle see identical values.
"""
from __future__ import annotations

from typing import Dict, Optional

import torch


def make_delta_inputs(B: int, H: int, T: int, DK: int = 128, DV: int = 128, *,
                      kind: str = "gdn", dtype: torch.dtype = torch.bfloat16, seed: int = 0,
                      gate_scale: Optional[float] = None, h0_std: Optional[float] = None,
                      device=None) -> Dict[str, torch.Tensor]:
    """kind: "gdn" (scalar per-token decay), "deltanet" (no decay, g = None) or "kda"
    (per-channel decay g [B,H,T,DK]).  Returns q, k, v (dtype), beta, g (float32 or None) and
    h0 (float32 or None), on ``device`` (CPU by default)."""
    if kind not in ("gdn", "deltanet", "kda"):
        raise ValueError(f"unknown kind {kind!r}")
    gen = torch.Generator().manual_seed(seed)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(B, H, T, DK, generator=gen), dim=-1)
    k = nrm(torch.randn(B, H, T, DK, generator=gen), dim=-1)
    v = torch.randn(B, H, T, DV, generator=gen)
    beta = torch.sigmoid(torch.randn(B, H, T, generator=gen))
    g = None
    if kind == "gdn":
        scale = 0.1 if gate_scale is None else gate_scale
        g = -torch.nn.functional.softplus(torch.randn(B, H, T, generator=gen)) * scale
    elif kind == "kda":
        scale = 0.05 if gate_scale is None else gate_scale
        g = -torch.nn.functional.softplus(torch.randn(B, H, T, DK, generator=gen)) * scale
    h0 = None
    if h0_std is not None:
        h0 = torch.randn(B, H, DK, DV, generator=gen) * h0_std
    out = dict(q=q.to(dtype), k=k.to(dtype), v=v.to(dtype), beta=beta.float(),
               g=None if g is None else g.float(), h0=h0)
    if device is not None:
        out = {n: (None if t is None else t.to(device)) for n, t in out.items()}
    return out


def as_oracle_inputs(inp: Dict[str, torch.Tensor]):
    """The same tensors as float64 numpy arrays (dtype-rounded values, upcast), for the oracle."""
    return {n: (None if t is None else t.detach().to("cpu", torch.float64).numpy())
            for n, t in inp.items()}
