"""Write tests/golden/*.npz: tiny seeded inputs and the outputs of the published token-recurrent
rules (fp64), independent of the chunked oracle.  Run from the repository root:

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle.gdn_oracle import gdn_recurrent, kda_recurrent  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def _inputs(rng, B, H, T, D, kda=False):
    nrm = lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True)
    q = nrm(rng.standard_normal((B, H, T, D)))
    k = nrm(rng.standard_normal((B, H, T, D)))
    v = rng.standard_normal((B, H, T, D))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, H, T))))
    shape = (B, H, T, D) if kda else (B, H, T)
    g = -np.log1p(np.exp(rng.standard_normal(shape))) * (0.05 if kda else 0.1)
    h0 = rng.standard_normal((B, H, D, D)) * 0.02
    # inputs are stored as float32: round them first so the stored values are the exact inputs
    return tuple(np.asarray(x, np.float32).astype(np.float64) for x in (q, k, v, beta, g, h0))


def main():
    rng = np.random.default_rng(20261201)
    f32 = lambda **kw: {n: np.asarray(x, np.float32) for n, x in kw.items()}
    q, k, v, beta, g, h0 = _inputs(rng, 1, 1, 128, 128)
    o, hT = gdn_recurrent(q, k, v, beta, g, h0=h0)
    np.savez_compressed(os.path.join(HERE, "gdn_recurrent_B1H1T128D128.npz"),
                        **f32(q=q, k=k, v=v, beta=beta, g=g, h0=h0, o=o, h_final=hT))
    q, k, v, beta, g, h0 = _inputs(rng, 1, 1, 64, 32, kda=True)
    o, hT = kda_recurrent(q, k, v, beta, g, h0=h0)
    np.savez_compressed(os.path.join(HERE, "kda_recurrent_B1H1T64D32.npz"),
                        **f32(q=q, k=k, v=v, beta=beta, g=g, h0=h0, o=o, h_final=hT))


if __name__ == "__main__":
    main()
