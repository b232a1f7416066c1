"""A seeded random sweep of the fused forwards against the oracle: GDN, DeltaNet (g = None) and
KDA, bf16 and fp32 operands, chunk size 64 or 128, with and without h0, gate scales from none to
steep, B·H from 1 to 66 (so both scan instantiations, the XCD-aware and the plain chain mapping)
and chains of 1 to 24 chunks.  The cases are drawn once from a fixed seed, so every run and every
failure names the same shapes.  Bounds as in the other parity tests: bf16 inputs max abs err
<= 2e-2, fp32 max rel err <= 1e-4, on o and the final state.  Oracle:
examples/attention/_gdn_full.py:57-97, src/pto_fuser/forwards/deltanet.py:114-143,
examples/attention/_kda_full.py:42-76 (restated in oracle/gdn_oracle.py)."""
import random

import numpy as np
import pytest
import torch

from conftest import announce, record_error
from oracle.gdn_oracle import deltanet_reference, gdn_reference, kda_reference
from pto_fuser_amd import gdn_chunk_forward, kda_chunk_forward
from pto_fuser_amd.forwards import as_oracle_inputs, make_delta_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
FP32_TOL = 1e-4
BF16_TOL = 2e-2
GATE_SCALES = {"gdn": (None, 0.02, 0.3, 1.0), "kda": (None, 0.1, 0.5), "deltanet": (None,)}


def _cases(n: int = 24, seed: int = 2026):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        kind = ("gdn", "deltanet", "kda")[i % 3]
        dtype = "bf16" if rng.random() < 0.7 else "fp32"
        if rng.random() < 0.35:
            B, H = rng.choice([(4, 16), (3, 22), (2, 32), (8, 8), (1, 64), (5, 13)])
            nc = rng.randint(1, 6)
        else:
            B, H = rng.randint(1, 3), rng.randint(1, 9)
            nc = rng.randint(1, 24)
        C = rng.choice((64, 64, 128))
        if C == 128 and nc % 2:
            nc += 1
        h0 = rng.random() < 0.5
        gs = rng.choice(GATE_SCALES[kind])
        out.append((kind, dtype, B, H, 64 * nc, C, h0, gs, rng.randint(0, 10 ** 6)))
    return out


@pytest.mark.parametrize("kind,dtype,B,H,T,C,h0,gs,seed", _cases(),
                         ids=lambda v: str(v) if not isinstance(v, float) else f"gs{v}")
def test_fused_forward_random_sweep(kind, dtype, B, H, T, C, h0, gs, seed):
    case = f"sweep {kind} {dtype} B{B} H{H} T{T} C{C} h0={h0} gs={gs} seed={seed}"
    announce(case)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    inp = make_delta_inputs(B, H, T, kind=kind, dtype=tdt, seed=seed, gate_scale=gs,
                            h0_std=0.02 if h0 else None)
    d = {n: (None if t is None else t.to(DEV)) for n, t in inp.items()}
    fwd = kda_chunk_forward if kind == "kda" else gdn_chunk_forward
    o, h = fwd(d["q"], d["k"], d["v"], d["beta"], d["g"], h0=d["h0"], chunk_size=C)
    torch.cuda.synchronize()
    o, h = o.cpu().numpy(), h.cpu().numpy()
    x = as_oracle_inputs(inp)
    if kind == "kda":
        ro, rh = kda_reference(x["q"], x["k"], x["v"], x["beta"], x["g"], C=C, h0=x["h0"],
                               dtype=np.float64)
    elif kind == "gdn":
        ro, rh = gdn_reference(x["q"], x["k"], x["v"], x["beta"], x["g"], C=C, h0=x["h0"],
                               dtype=np.float64)
    else:
        ref = deltanet_reference(x["q"], x["k"], x["v"], x["beta"], C=C, h0=x["h0"],
                                 dtype=np.float64)
        ro, rh = ref["o"].reshape(o.shape), ref["final"]
    bf16 = dtype == "bf16"
    tol = f"max abs <= {BF16_TOL}" if bf16 else f"max rel <= {FP32_TOL}"
    for name, got, r in (("o", o, ro), ("h", h, rh)):
        assert np.isfinite(got).all(), (case, name)
        e = record_error(case, name, got, r, tol)
        assert (e["abs"] if bf16 else e["rel"]) <= (BF16_TOL if bf16 else FP32_TOL), (case, name, e)
