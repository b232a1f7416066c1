"""CPU oracle for the chunked delta-rule forward (DeltaNet / GDN / KDA) — TEST INFRASTRUCTURE.

This module is the checker, never the product: only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg may import it.  The HIP path in ``pto-fuser_amd``
never calls into it and fails loudly if its extension is missing.

It restates, in numpy, the reference's fp32 golden functions for the path:

  * ``gdn_reference``        examples/attention/_gdn_full.py:57-97   (plus h0 and the final state)
  * ``deltanet_reference``   src/pto_fuser/forwards/deltanet.py:114-143 (plus h0 and the final state)
  * ``kda_reference``        examples/attention/_kda_full.py:42-76   (plus h0 and the final state)
  * ``scan_reference``       src/pto_fuser/forwards/fused_stages.py:46-62
  * ``kkt_reference``        src/pto_fuser/forwards/fused_stages.py:140-156
  * ``gated_qk_reference``   src/pto_fuser/kernels/kkt_fused.h:154-185 (the epilogue formula)
  * ``qkv_flash_reference``  tests/test_fusion_npu.py:152-156 (chunk_o flash semantics)
  * ``tri_inv_reference``    examples/attention/_gdn_full.py:76-78 (solve_triangular(I+A, I))
  * ``prepare_gdn_coefficients`` examples/attention/_gdn_full.py:103-144

and adds two published token-recurrent rules that pin them (not restatements of the
reference; they are the mathematics the chunked form must reproduce):

  * ``gdn_recurrent``  gated delta rule  S_t = a_t (I - b_t k_t k_t^T) S_{t-1} + b_t k_t v_t^T,
                       o_t = scale * q_t^T S_t           (Yang, Kautz & Hatamizadeh, ICLR 2025)
  * ``kda_recurrent``  S_t = (I - b_t k_t k_t^T) Diag(a_t) S_{t-1} + b_t k_t v_t^T

Layout: q, k [B,H,T,dk]; v [B,H,T,dv]; beta [B,H,T]; g [B,H,T] per-token log-decay (GDN) or
[B,H,T,dk] (KDA), *not* cumulatively summed — the oracle does the within-chunk cumsum like the
reference (_gdn_full.py:63).  h0 [B,H,dk,dv] or None.  Every function takes ``dtype``
(float32 mirrors the reference's fp32 torch; float64 is used to pin).

Pinning status (each function is checked in tests/test_oracle.py):
  gdn_reference       — vs gdn_recurrent (fp64), chunk-size invariance, state passing, beta=0
                        closed form, linearity in v, loop == batched.
  deltanet_reference  — equals gdn_reference at g=0; vs recurrent; intermediates satisfy
                        T(I+A)=I, W=T(beta k), U=T(beta v).
  kda_reference       — vs kda_recurrent (fp64); equals gdn_reference when g is constant over dk.
  scan_reference      — vs a direct unrolled restatement + decay=0/u=0 closed forms.
  kkt_reference / gated_qk_reference — vs brute-force triple loop; G=0,beta=1 -> strict-lower(KK^T).
  tri_inv_reference   — T(I+A)=I, Neumann series sum_k (-A)^k (fp64), C=2 closed form, scipy.
  qkv_flash_reference — vs brute-force loop at small C.
  prepare_gdn_coefficients — the staged coefficient decomposition reproduces gdn_reference.
No function is left "parity unpinned".
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "bf16_round", "within_chunk_cumsum", "safe_exp",
    "tri_inv_reference", "gated_qk_reference", "kkt_reference", "qkv_flash_reference",
    "gdn_reference", "deltanet_reference", "kda_reference", "scan_reference",
    "gdn_recurrent", "kda_recurrent", "prepare_gdn_coefficients", "chunk_intermediates",
    "max_abs", "max_rel", "frob_rel",
]


# --------------------------------------------------------------------------- #
#  small helpers
# --------------------------------------------------------------------------- #
def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), returned as float32.

    Used to build the dtype-rounded inputs the fp32 oracle consumes, so the measured error of
    a bf16 kernel is its arithmetic, not input quantisation."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).copy()
    nan = np.isnan(a)
    out[nan] = np.nan
    return out


def within_chunk_cumsum(g: np.ndarray, C: int) -> np.ndarray:
    """Cumulative sum of the per-token log-decay inside each chunk of C tokens, along axis 2.

    _gdn_full.py:63 (``g_sum = gf.cumsum(dim=3)`` over the [B,H,nc,C] layout); for KDA the
    same cumsum runs per channel (_kda_full.py:189)."""
    B, H, T = g.shape[:3]
    assert T % C == 0, f"T={T} is not a multiple of the chunk size C={C}"
    nc = T // C
    tail = g.shape[3:]
    gs = g.reshape(B, H, nc, C, *tail).cumsum(axis=3)
    return gs.reshape(B, H, T, *tail)


def safe_exp(x: np.ndarray) -> np.ndarray:
    """exp(x) where x <= 0, else 0 — _gdn_full.py:53-54."""
    return np.where(x <= 0, np.exp(np.minimum(x, 0)), np.zeros_like(x))


def max_abs(got, ref) -> float:
    return float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))))


def max_rel(got, ref) -> float:
    """max|x - r| / max|r| — the "max rel err" the tolerances are stated in."""
    r = np.asarray(ref, np.float64)
    return max_abs(got, ref) / max(float(np.max(np.abs(r))), 1e-30)


def frob_rel(got, ref) -> float:
    """||x - r||_F / ||r||_F — src/pto_fuser/gate.py:25-27."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    return float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-9))


# --------------------------------------------------------------------------- #
#  chunk-local stages
# --------------------------------------------------------------------------- #
def tri_inv_reference(A: np.ndarray, dtype=np.float64) -> np.ndarray:
    """(I + A)^-1 for strictly-lower A [..., C, C] by forward substitution.

    The reference solves ``solve_triangular(I + A, I, upper=False, unitriangular=True)``
    (_gdn_full.py:76-78, deltanet.py:123-124); the opaque kernel it replaces returns the same
    lower unit-triangular inverse in fp32 (registry.py:107-127).  Row i of T is
    e_i - sum_{j<i} A[i, j] T[j, :]."""
    A = np.asarray(A, dtype=dtype)
    C = A.shape[-1]
    T = np.zeros_like(A)
    T[..., 0, 0] = 1.0
    for i in range(1, C):
        # only the strictly-lower part of A participates (upper part is ignored, as tril does)
        T[..., i, :] = -np.einsum("...j,...jc->...c", A[..., i, :i], T[..., :i, :])
        T[..., i, i] = 1.0
    return T


def gated_qk_reference(a, b, g_sum, beta, causal: bool, dtype=np.float32) -> np.ndarray:
    """L = (a b^T) * exp(min(g_i + log beta_i - g_j, 0)) * mask, per [C, *] block.

    The gated-matmul epilogue of kkt_fused.h:154-185 (shared by the kkt stage, with a = b = k,
    real beta and a strict-lower mask, and by chunk_o's score, with beta = 1 and a causal mask
    including the diagonal; fused.py:190-282).  a, b [..., C, D]; g_sum, beta [..., C]."""
    a = np.asarray(a, dtype)
    b = np.asarray(b, dtype)
    g = np.asarray(g_sum, dtype)
    bt = np.asarray(beta, dtype)
    C = a.shape[-2]
    qk = a @ np.swapaxes(b, -1, -2)
    with np.errstate(divide="ignore"):
        gv = g + np.log(bt)
    diff = gv[..., :, None] - g[..., None, :]
    coeff = np.exp(np.minimum(diff, 0))
    rows = np.arange(C)
    mask = (rows[:, None] >= rows[None, :]) if causal else (rows[:, None] > rows[None, :])
    return (qk * coeff * mask).astype(dtype)


def kkt_reference(k, g_sum, beta, nc: int, H: int, C: int, dtype=np.float32) -> np.ndarray:
    """Gated kkt in the mega layout — fused_stages.py:140-156.

    k [1, T, H, D], g_sum [1, T, H] (already cumsummed within chunks), beta [1, T, H] ->
    L [T, H, C] with L[c*C + i, h, j] = (k_i . k_j) exp(min(g_i + log b_i - g_j, 0)) [i > j]."""
    D = k.shape[-1]
    kc = np.asarray(k, dtype).reshape(nc, C, H, D).transpose(0, 2, 1, 3)    # [nc,H,C,D]
    gs = np.asarray(g_sum, dtype).reshape(nc, C, H).transpose(0, 2, 1)      # [nc,H,C]
    bs = np.asarray(beta, dtype).reshape(nc, C, H).transpose(0, 2, 1)
    L = gated_qk_reference(kc, kc, gs, bs, causal=False, dtype=dtype)       # [nc,H,C,C]
    return L.transpose(0, 2, 1, 3).reshape(nc * C, H, C)


def qkv_flash_reference(q, k, v, g_sum, dtype=np.float32) -> np.ndarray:
    """chunk_o intra half in one pass: o = (causal(q k^T) * exp(min(g_i - g_j, 0))) v.

    The semantics of qkv_flash_native (fused.py:353-395), as the reference's own test states
    them (tests/test_fusion_npu.py:152-156).  q, k [M, C, D]; v [M, C, DV]; g_sum [M, C]."""
    ones = np.ones_like(np.asarray(g_sum, dtype))
    P = gated_qk_reference(q, k, g_sum, ones, causal=True, dtype=dtype)
    return (P @ np.asarray(v, dtype)).astype(dtype)


def chunk_intermediates(k, v, beta, G, dtype=np.float64):
    """A, T, W, U for one batch of chunks (the kkt -> solve -> wy stages, _gdn_full.py:73-82).

    k [..., C, dk], v [..., C, dv], beta [..., C], G [..., C] (within-chunk cumsum)."""
    k = np.asarray(k, dtype)
    v = np.asarray(v, dtype)
    bt = np.asarray(beta, dtype)
    G = np.asarray(G, dtype)
    C = k.shape[-2]
    A = np.tril((k @ np.swapaxes(k, -1, -2)) * safe_exp(G[..., :, None] - G[..., None, :])
                * bt[..., :, None], -1)
    T = tri_inv_reference(A, dtype=dtype)
    kb = k * (bt * np.exp(G))[..., None]
    vb = v * bt[..., None]
    return A, T, T @ kb, T @ vb


# --------------------------------------------------------------------------- #
#  full forwards
# --------------------------------------------------------------------------- #
def _prep(q, k, v, beta, dtype):
    return (np.asarray(q, dtype), np.asarray(k, dtype), np.asarray(v, dtype),
            np.asarray(beta, dtype))


def gdn_reference(q, k, v, beta, g, scale=None, C: int = 64, h0=None, dtype=np.float32,
                  loop: bool = False, return_snapshots: bool = False):
    """Gated DeltaNet chunked forward — examples/attention/_gdn_full.py:57-97.

    Returns ``(o [B,H,T,dv], h_final [B,H,dk,dv])``; ``return_snapshots`` also returns the
    pre-update states h_c [B,H,nc,dk,dv] and v_new [B,H,T,dv].  Differences from the
    reference, both additions: an initial state ``h0`` (the reference hard-wires S = 0 at
    :67) and the final state (the reference drops the S after its last chunk, :87).

    ``loop=True`` runs the reference's b, h, c triple loop (the CPU-baseline shape);
    ``loop=False`` runs the same per-chunk arithmetic batched over all (b, h) at once."""
    q, k, v, beta = _prep(q, k, v, beta, dtype)
    B, H, T, dk = q.shape
    dv = v.shape[-1]
    nc = T // C
    scale = dk ** -0.5 if scale is None else scale
    G = within_chunk_cumsum(np.asarray(g, dtype), C).reshape(B, H, nc, C)
    qc, kc = q.reshape(B, H, nc, C, dk), k.reshape(B, H, nc, C, dk)
    vc_in, bc = v.reshape(B, H, nc, C, dv), beta.reshape(B, H, nc, C)
    rows = np.arange(C)
    causal = (rows[:, None] >= rows[None, :]).astype(dtype)
    S0 = np.zeros((B, H, dk, dv), dtype) if h0 is None else np.array(h0, dtype)

    def step(S, qi, ki, vi, bi, gi):
        """One chunk: returns (o_c, S_next, v_new_c) for state S (any leading batch)."""
        A = np.tril((ki @ np.swapaxes(ki, -1, -2)) * safe_exp(gi[..., :, None] - gi[..., None, :])
                    * bi[..., :, None], -1)
        Tm = tri_inv_reference(A, dtype=dtype)
        kb = ki * (bi * np.exp(gi))[..., None]
        vb = vi * bi[..., None]
        W, U = Tm @ kb, Tm @ vb
        vn = U - W @ S
        gl = gi[..., -1:]
        S_next = (np.exp(gl)[..., None] * S
                  + np.swapaxes(ki, -1, -2) @ (vn * np.exp(gl - gi)[..., None]))
        inter = (qi @ S) * np.exp(gi)[..., None]
        gate = np.exp(np.minimum(gi[..., :, None] - gi[..., None, :], 0))
        o = inter + ((qi @ np.swapaxes(ki, -1, -2)) * gate * causal) @ vn
        return o, S_next, vn

    o = np.zeros((B, H, nc, C, dv), dtype)
    vnew = np.zeros((B, H, nc, C, dv), dtype)
    snaps = np.zeros((B, H, nc, dk, dv), dtype) if return_snapshots else None
    hf = np.zeros((B, H, dk, dv), dtype)
    if loop:
        for b in range(B):
            for h in range(H):
                S = S0[b, h].copy()
                for c in range(nc):
                    if snaps is not None:
                        snaps[b, h, c] = S
                    o[b, h, c], S, vnew[b, h, c] = step(S, qc[b, h, c], kc[b, h, c],
                                                        vc_in[b, h, c], bc[b, h, c], G[b, h, c])
                hf[b, h] = S
    else:
        S = S0.copy()
        for c in range(nc):
            if snaps is not None:
                snaps[:, :, c] = S
            o[:, :, c], S, vnew[:, :, c] = step(S, qc[:, :, c], kc[:, :, c], vc_in[:, :, c],
                                                bc[:, :, c], G[:, :, c])
        hf = S
    o = (o * dtype(scale)).reshape(B, H, T, dv)
    if return_snapshots:
        return o, hf, snaps, vnew.reshape(B, H, T, dv)
    return o, hf


def deltanet_reference(q, k, v, beta, scale=None, C: int = 64, h0=None, dtype=np.float32):
    """Ungated DeltaNet chunked forward — src/pto_fuser/forwards/deltanet.py:114-143.

    Returns the reference's seven outputs in its layouts (A, T [M,C,C]; W, U, v_new
    [B,H,nc,C,D]; h_state [B,H,nc,D,D]; o [B,H,nc,C,D]) plus ``final`` [B,H,D,D] (the state
    after the last chunk, which the reference drops) — with q, k, v given as [B,H,T,D]."""
    q, k, v, beta = _prep(q, k, v, beta, dtype)
    B, H, T, D = q.shape
    dv = v.shape[-1]
    nc = T // C
    scale = D ** -0.5 if scale is None else scale
    qF = q.reshape(B * H * nc, C, D)
    kF = k.reshape(B * H * nc, C, D)
    kbF = kF * beta.reshape(B * H * nc, C, 1)                 # kb = beta[...,None] * k  (:117)
    vbF = v.reshape(B * H * nc, C, dv) * beta.reshape(B * H * nc, C, 1)
    A = np.tril(kbF @ np.swapaxes(kF, -1, -2), -1)             # (:121-122)
    Tm = tri_inv_reference(A, dtype=dtype)                     # (:123-124)
    W = (Tm @ kbF).reshape(B, H, nc, C, D)
    U = (Tm @ vbF).reshape(B, H, nc, C, dv)
    kf5 = k.reshape(B, H, nc, C, D)
    h_state = np.zeros((B, H, nc, D, dv), dtype)
    v_new = np.zeros((B, H, nc, C, dv), dtype)
    S = np.zeros((B, H, D, dv), dtype) if h0 is None else np.array(h0, dtype)
    for c in range(nc):                                         # (:130-137), batched over b,h
        h_state[:, :, c] = S
        vn = U[:, :, c] - W[:, :, c] @ S
        v_new[:, :, c] = vn
        S = S + np.swapaxes(kf5[:, :, c], -1, -2) @ vn
    o_inter = qF @ h_state.reshape(-1, D, dv)
    Aqk = np.tril(qF @ np.swapaxes(kF, -1, -2), 0)
    o_intra = Aqk @ v_new.reshape(-1, C, dv)
    o = (o_inter + o_intra) * dtype(scale)
    return dict(A=A, T=Tm, W=W, U=U, h_state=h_state, v_new=v_new,
                o=o.reshape(B, H, nc, C, dv), final=S)


def kda_reference(q, k, v, beta, g, scale=None, C: int = 64, h0=None, dtype=np.float32):
    """KDA (per-channel decay) chunked forward — examples/attention/_kda_full.py:42-76.

    g [B,H,T,dk] per-token per-channel log-decay (cumsummed within chunks here, :189).
    Returns ``(o [B,H,T,dv], h_final [B,H,dk,dv])``; h0 and the final state are additions."""
    q, k, v, beta = _prep(q, k, v, beta, dtype)
    B, H, T, dk = q.shape
    dv = v.shape[-1]
    nc = T // C
    scale = dk ** -0.5 if scale is None else scale
    G = within_chunk_cumsum(np.asarray(g, dtype), C).reshape(B, H, nc, C, dk)
    qc, kc = q.reshape(B, H, nc, C, dk), k.reshape(B, H, nc, C, dk)
    vc_in, bc = v.reshape(B, H, nc, C, dv), beta.reshape(B, H, nc, C)
    rows = np.arange(C)
    causal = (rows[:, None] >= rows[None, :]).astype(dtype)
    S = np.zeros((B, H, dk, dv), dtype) if h0 is None else np.array(h0, dtype)
    o = np.zeros((B, H, nc, C, dv), dtype)
    for c in range(nc):
        gc, kk, qq, vv, bb = G[:, :, c], kc[:, :, c], qc[:, :, c], vc_in[:, :, c], bc[:, :, c]
        a_op = kk * np.exp(gc)
        b_op = kk * np.exp(-gc)
        A = np.tril((a_op @ np.swapaxes(b_op, -1, -2)) * bb[..., :, None], -1)
        Tm = tri_inv_reference(A, dtype=dtype)
        W = Tm @ (kk * np.exp(gc) * bb[..., None])
        U = Tm @ (vv * bb[..., None])
        vcorr = U - W @ S
        g_tot = gc[..., -1, :]                                    # [B,H,dk]
        k_rest = kk * np.exp(g_tot[..., None, :] - gc)
        q_eff = qq * np.exp(gc)
        k_eff = kk * np.exp(-gc)
        o[:, :, c] = q_eff @ S + ((q_eff @ np.swapaxes(k_eff, -1, -2)) * causal) @ vcorr
        S = np.exp(g_tot)[..., :, None] * S + np.swapaxes(k_rest, -1, -2) @ vcorr
    return (o * dtype(scale)).reshape(B, H, T, dv), S


def scan_reference(w, u, k, decay, h0=None, dtype=np.float32):
    """The simplified chunk_h recurrence — src/pto_fuser/forwards/fused_stages.py:46-62.

    w, u, k in the token-major [B, nc, C, H, D] layout, decay [B, H, nc] (scalar per chunk) or
    [B, H, nc, D] (per-dim row decay, scan_fused.h:143-180).  Per chunk: h_out[c] = S;
    S = decay * S + k^T (u - w S).  Returns ``(h_out [B,nc,H,D,D], final [B,H,D,D])``.
    (h0 is an addition; the reference starts from zero.)"""
    w = np.asarray(w, dtype)
    u = np.asarray(u, dtype)
    k = np.asarray(k, dtype)
    dec = np.asarray(decay, dtype)
    B, nc, C, H, D = w.shape
    Dv = u.shape[-1]
    h_out = np.zeros((B, nc, H, D, Dv), dtype)
    S = np.zeros((B, H, D, Dv), dtype) if h0 is None else np.array(h0, dtype)
    for c in range(nc):
        h_out[:, c] = S
        wc = w[:, c].transpose(0, 2, 1, 3)                         # [B,H,C,D]
        uc = u[:, c].transpose(0, 2, 1, 3)
        kc = k[:, c].transpose(0, 2, 1, 3)
        vc = uc - wc @ S
        d = dec[:, :, c]
        d = d[..., None, None] if d.ndim == 2 else d[..., :, None]
        S = d * S + np.swapaxes(kc, -1, -2) @ vc
    return h_out, S


def prepare_gdn_coefficients(g, beta, C: int, dtype=np.float32) -> dict:
    """The host gate coefficients of prepare_gdn_bindings — _gdn_full.py:103-144.

    g, beta [B,H,T] -> coefA [M,C,C], coef_kb/coef_vb/coef_qg [M,C,1], coef_o [M,C,C],
    coef_vcs [N,nc,C,1], coef_S [N,nc,1,1], g_native [M,C] (M = B*H*nc, N = B*H)."""
    g = np.asarray(g, dtype)
    bt = np.asarray(beta, dtype)
    B, H, T = g.shape
    nc = T // C
    M = B * H * nc
    gs = within_chunk_cumsum(g, C).reshape(B, H, nc, C)
    bt = bt.reshape(B, H, nc, C)
    gi, gj = gs[..., :, None], gs[..., None, :]
    gl = gs[..., -1:]
    rows = np.arange(C)
    causal = (rows[:, None] >= rows[None, :]).astype(dtype)
    return dict(
        coefA=(safe_exp(gi - gj) * bt[..., :, None]).reshape(M, C, C),
        coef_kb=(bt * np.exp(gs)).reshape(M, C, 1),
        coef_vb=bt.reshape(M, C, 1),
        coef_qg=np.exp(gs).reshape(M, C, 1),
        coef_o=(np.exp(np.minimum(gi - gj, 0)) * causal).reshape(M, C, C),
        coef_vcs=np.exp(gl[..., None] - gi).reshape(B * H, nc, C, 1),
        coef_S=np.exp(gl).reshape(B * H, nc, 1, 1),
        g_native=gs.reshape(M, C),
        beta_native=bt.reshape(M, C),
    )


# --------------------------------------------------------------------------- #
#  token-recurrent pins (published rules, not reference restatements)
# --------------------------------------------------------------------------- #
def gdn_recurrent(q, k, v, beta, g, scale=None, h0=None, dtype=np.float64):
    """Gated delta rule, one token at a time: S_t = e^{g_t}(I - b_t k_t k_t^T) S_{t-1}
    + b_t k_t v_t^T, o_t = scale q_t^T S_t.  g [B,H,T] per-token log-decay (g = 0 gives
    DeltaNet).  Returns (o, S_T)."""
    q, k, v, beta = _prep(q, k, v, beta, dtype)
    g = np.asarray(g, dtype)
    B, H, T, dk = q.shape
    dv = v.shape[-1]
    scale = dk ** -0.5 if scale is None else scale
    S = np.zeros((B, H, dk, dv), dtype) if h0 is None else np.array(h0, dtype)
    o = np.zeros((B, H, T, dv), dtype)
    for t in range(T):
        kt, vt, bt = k[:, :, t], v[:, :, t], beta[:, :, t]
        S = np.exp(g[:, :, t])[..., None, None] * S
        kS = np.einsum("bhd,bhde->bhe", kt, S)
        S = S + bt[..., None, None] * kt[..., :, None] * (vt - kS)[..., None, :]
        o[:, :, t] = np.einsum("bhd,bhde->bhe", q[:, :, t], S)
    return o * scale, S


def kda_recurrent(q, k, v, beta, g, scale=None, h0=None, dtype=np.float64):
    """Per-channel gated delta rule: S_t = (I - b_t k_t k_t^T) Diag(e^{g_t}) S_{t-1}
    + b_t k_t v_t^T, o_t = scale q_t^T S_t.  g [B,H,T,dk].  Returns (o, S_T)."""
    q, k, v, beta = _prep(q, k, v, beta, dtype)
    g = np.asarray(g, dtype)
    B, H, T, dk = q.shape
    dv = v.shape[-1]
    scale = dk ** -0.5 if scale is None else scale
    S = np.zeros((B, H, dk, dv), dtype) if h0 is None else np.array(h0, dtype)
    o = np.zeros((B, H, T, dv), dtype)
    for t in range(T):
        kt, vt, bt = k[:, :, t], v[:, :, t], beta[:, :, t]
        S = np.exp(g[:, :, t])[..., :, None] * S
        kS = np.einsum("bhd,bhde->bhe", kt, S)
        S = S + bt[..., None, None] * kt[..., :, None] * (vt - kS)[..., None, :]
        o[:, :, t] = np.einsum("bhd,bhde->bhe", q[:, :, t], S)
    return o * scale, S
