"""GPU parity of the stage kernels behind the compile stack's fused nodes, through the C ABI.

gated qkᵀ (kkt_gated / gated_qk, native and token layouts, qk_prologue), chunk_o flash
(qkv_flash / qkvp_flash) and the resident-state scan (chunk_h_scan, scalar and per-channel decay)
against the oracle on the same dtype-rounded inputs.  Tolerances: fp32 operands max rel err
<= 1e-4; bf16 operands (fp32 accumulation, bf16 rounding of on-chip MFMA operands) max rel err
<= 1e-2 for the single-pass stages and <= 2e-2 for the scan (its state is re-rounded to bf16 as
an MFMA operand every chunk).  max rel = max|x - r| / max|r|.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle.gdn_oracle import (gated_qk_reference, kkt_reference, max_rel, qkv_flash_reference,
                               scan_reference)
from pto_fuser_amd.ops import chunk_scan, gated_qk, qkv_flash

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = {torch.float32: 1e-4, torch.bfloat16: 1e-2}


def _t(x, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype)


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


def _gates(rng, shape, C):
    """Within-chunk cumulative log decay (non-increasing along the chunk) and beta in (0, 1)."""
    g = np.cumsum(-np.log1p(np.exp(rng.standard_normal(shape))) * 0.1, axis=-1)
    beta = 1 / (1 + np.exp(-rng.standard_normal(shape)))
    return g.astype(np.float32), beta.astype(np.float32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("C,D", [(64, 128), (128, 128), (32, 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_gated_qk_native(dtype, C, D, causal):
    announce(f"gated_qk native C={C} D={D} causal={causal} {dtype}")
    rng = np.random.default_rng(C + D + causal)
    M = 40
    a = _t(rng.standard_normal((M, C, D)) * 0.2, dtype)
    b = _t(rng.standard_normal((M, C, D)) * 0.2, dtype)
    g, beta = _gates(rng, (M, C), C)
    L = gated_qk(a.to(DEV), b.to(DEV), _t(g).to(DEV), _t(beta).to(DEV), chunk_size=C,
                 causal=causal)
    torch.cuda.synchronize()
    ref = gated_qk_reference(_np(a), _np(b), g, beta, causal=causal, dtype=np.float64)
    assert L.shape == (M, C, C)
    assert max_rel(_np(L), ref) <= TOL[dtype], max_rel(_np(L), ref)
    # the masked entries are exact zeros
    keep = np.tril(np.ones((C, C)), 0 if causal else -1).astype(bool)
    assert np.all(_np(L)[:, ~keep] == 0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_kkt_token_layout(dtype):
    """kkt_gated on the [1, T, H, D] token layout: L [T, H, C] (fused_stages.py:140-156)."""
    C, D, H, nc = 64, 128, 3, 5
    announce(f"kkt token layout H={H} nc={nc} {dtype}")
    rng = np.random.default_rng(7)
    k = _t(rng.standard_normal((1, nc * C, H, D)) * 0.1, dtype)
    g = np.empty((1, nc * C, H), np.float32)
    beta = np.empty((1, nc * C, H), np.float32)
    for h in range(H):
        gg, bb = _gates(rng, (nc, C), C)
        g[0, :, h], beta[0, :, h] = gg.reshape(-1), bb.reshape(-1)
    L = gated_qk(k.to(DEV), k.to(DEV), _t(g).to(DEV), _t(beta).to(DEV), chunk_size=C, heads=H,
                 causal=False)
    torch.cuda.synchronize()
    ref = kkt_reference(_np(k), g, beta, nc, H, C, dtype=np.float64)
    assert L.shape == (nc * C, H, C)
    assert max_rel(_np(L), ref) <= TOL[dtype], max_rel(_np(L), ref)


def test_gated_qk_mask_beta_none_and_bf16_out():
    """An explicit [C, C] mask multiplies the score; no g / beta means a plain masked product;
    bf16 output rounds the fp32 result."""
    C, D, M = 64, 64, 8
    announce("gated_qk explicit mask, bf16 out")
    rng = np.random.default_rng(11)
    a = rng.standard_normal((M, C, D)).astype(np.float32) * 0.3
    b = rng.standard_normal((M, C, D)).astype(np.float32) * 0.3
    mask = (rng.random((C, C)) < 0.5).astype(np.float32) * 0.5
    L = gated_qk(_t(a).to(DEV), _t(b).to(DEV), chunk_size=C, mask=_t(mask).to(DEV),
                 out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    ref = np.einsum("mid,mjd->mij", a.astype(np.float64), b.astype(np.float64)) * mask
    assert L.dtype == torch.bfloat16
    assert max_rel(_np(L), ref) <= 8e-3, max_rel(_np(L), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_qk_prologue_per_channel(dtype):
    """qk_prologue: causal((q ⊙ P)(k ⊙ P⁻¹)ᵀ) with P = exp(G) per channel."""
    C, D, M = 64, 128, 16
    announce(f"qk_prologue {dtype}")
    rng = np.random.default_rng(12)
    q = _t(rng.standard_normal((M, C, D)) * 0.1, dtype)
    k = _t(rng.standard_normal((M, C, D)) * 0.1, dtype)
    G = np.cumsum(-np.log1p(np.exp(rng.standard_normal((M, C, D)))) * 0.05, axis=1).astype(np.float32)
    P, invP = np.exp(G), np.exp(-G)
    L = gated_qk(q.to(DEV), k.to(DEV), chunk_size=C, causal=True, a_scale=_t(P).to(DEV),
                 b_scale=_t(invP).to(DEV))
    torch.cuda.synchronize()
    qd, kd = _np(q) * P, _np(k) * invP
    ref = np.tril(np.einsum("mid,mjd->mij", qd, kd))
    assert max_rel(_np(L), ref) <= TOL[dtype], max_rel(_np(L), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("C,D", [(64, 128), (128, 128), (32, 64)])
def test_qkv_flash(dtype, C, D):
    announce(f"qkv_flash C={C} D={D} {dtype}")
    rng = np.random.default_rng(100 + C + D)
    M = 24
    q = _t(rng.standard_normal((M, C, D)) * 0.1, dtype)
    k = _t(rng.standard_normal((M, C, D)) * 0.1, dtype)
    v = _t(rng.standard_normal((M, C, D)), dtype)
    g, _ = _gates(rng, (M, C), C)
    o = qkv_flash(q.to(DEV), k.to(DEV), v.to(DEV), _t(g).to(DEV), chunk_size=C)
    torch.cuda.synchronize()
    ref = qkv_flash_reference(_np(q), _np(k), _np(v), g, dtype=np.float64)
    assert o.shape == (M, C, D) and o.dtype == torch.float32
    assert max_rel(_np(o), ref) <= TOL[dtype], max_rel(_np(o), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_qkvp_flash_per_channel(dtype):
    C, D, M = 64, 128, 16
    announce(f"qkvp_flash {dtype}")
    rng = np.random.default_rng(21)
    q = _t(rng.standard_normal((M, C, D)) * 0.1, dtype)
    k = _t(rng.standard_normal((M, C, D)) * 0.1, dtype)
    v = _t(rng.standard_normal((M, C, D)), dtype)
    G = np.cumsum(-np.log1p(np.exp(rng.standard_normal((M, C, D)))) * 0.05, axis=1).astype(np.float32)
    ag, bg = np.exp(G), np.exp(-G)
    o = qkv_flash(q.to(DEV), k.to(DEV), v.to(DEV), chunk_size=C, q_scale=_t(ag).to(DEV),
                  k_scale=_t(bg).to(DEV))
    torch.cuda.synchronize()
    ref = np.tril(np.einsum("mid,mjd->mij", _np(q) * ag, _np(k) * bg)) @ _np(v)
    assert max_rel(_np(o), ref) <= TOL[dtype], max_rel(_np(o), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("perdim", [False, True])
@pytest.mark.parametrize("C,D", [(64, 128), (128, 128), (32, 64)])
def test_chunk_scan(dtype, perdim, C, D):
    B, H, nc = 2, 3, 5
    announce(f"chunk_scan C={C} D={D} perdim={perdim} {dtype}")
    rng = np.random.default_rng(300 + C + D + perdim)
    w = _t(rng.standard_normal((B, nc, C, H, D)) * 0.02, dtype)
    u = _t(rng.standard_normal((B, nc, C, H, D)) * 0.5, dtype)
    k = _t(rng.standard_normal((B, nc, C, H, D)) * 0.05, dtype)
    dshape = (B, H, nc, D) if perdim else (B, H, nc)
    decay = np.exp(-rng.random(dshape) * 0.5).astype(np.float32)
    h0 = (rng.standard_normal((B, H, D, D)) * 0.1).astype(np.float32)
    h_out, final = chunk_scan(w.to(DEV), u.to(DEV), k.to(DEV), _t(decay).to(DEV), _t(h0).to(DEV))
    torch.cuda.synchronize()
    ref_h, ref_f = scan_reference(_np(w), _np(u), _np(k), decay, h0=h0, dtype=np.float64)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert max_rel(_np(h_out), ref_h) <= tol, max_rel(_np(h_out), ref_h)
    assert max_rel(_np(final), ref_f) <= tol, max_rel(_np(final), ref_f)


def test_chunk_scan_zero_start_bf16_out():
    """No h0 (the reference's zero start) and bf16 snapshots; the first snapshot is exactly 0."""
    B, nc, C, H, D = 1, 3, 64, 2, 128
    announce("chunk_scan h0=None bf16 out")
    rng = np.random.default_rng(5)
    w, u, k = (rng.standard_normal((B, nc, C, H, D)).astype(np.float32) * s for s in (0.02, 0.5, 0.05))
    decay = np.exp(-rng.random((B, H, nc))).astype(np.float32)
    h_out, final = chunk_scan(_t(w).to(DEV), _t(u).to(DEV), _t(k).to(DEV), _t(decay).to(DEV),
                              out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    ref_h, ref_f = scan_reference(w, u, k, decay, dtype=np.float64)
    assert h_out.dtype == torch.bfloat16 and np.all(_np(h_out)[:, 0] == 0)
    assert max_rel(_np(h_out), ref_h) <= 8e-3
    assert max_rel(_np(final), ref_f) <= 1e-4
