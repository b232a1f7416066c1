"""Resident-state scan rewrite of the KDA program (src/pto_fuser/transforms/kda.py:1-86).

KDA's gate is per key channel, so its scan decays state row d by e^{G_tot,d} and scales k by
e^{G_tot - G} per channel (``coef_krest``).  Same rewrite as GDN's ``LowerResidentScan``, with
``chunk_h_scan`` in its per-channel form (``perdim_decay=True``, decay ``[B, H, nc, D]``).
"""
from __future__ import annotations

from .gdn import _ResidentScan


class LowerPerDimScan(_ResidentScan):
    name = "lower-perdim-scan"
    summary = "unrolled KDA scan -> chunk_h_scan FusedNode (state in registers, per-channel decay)"
    family_input = "coef_krest"
    k_coef = "coef_krest"
    k_scaled = "k_krest"
    perdim = True
    per_chunk = ("Wc{c}_s", "Wc{c}", "WS{c}", "Uc{c}", "vn{c}", "kc{c}_s", "kc{c}", "krc{c}",
                 "krest{c}", "dS{c}", "sc{c}", "Sd{c}", "S{c1}")
