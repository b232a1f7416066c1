"""Pins of the CPU oracle (no GPU).

Every oracle function is checked against something that is not a retyping of its own formula:
the published token-recurrent rules (fp64), closed forms, invariants that a dropped term, a wrong
sign or a transposed operand would break, brute-force loops on tiny inputs, library routines
(scipy / numpy BLAS), and agreement between independent restatements (e.g. the standalone scan
stage driven exactly as the reference's resident-scan lowering drives it must reproduce the full
forward's per-chunk states).  The reference ships no golden vectors for this path; the committed
fixtures under tests/golden/ come from the recurrent rules (make_golden.py).
"""
import os

import numpy as np
import pytest
import scipy.linalg

from oracle.gdn_oracle import (bf16_round, chunk_intermediates, deltanet_reference,
                               frob_rel, gated_qk_reference, gdn_recurrent, gdn_reference,
                               kda_recurrent, kda_reference, kkt_reference, max_abs, max_rel,
                               prepare_gdn_coefficients, qkv_flash_reference, safe_exp,
                               scan_reference, tri_inv_reference, within_chunk_cumsum)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _nrm(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def _inputs(seed, B, H, T, D, Dv=None, kda=False, h0=True):
    rng = np.random.default_rng(seed)
    Dv = D if Dv is None else Dv
    q = _nrm(rng.standard_normal((B, H, T, D)))
    k = _nrm(rng.standard_normal((B, H, T, D)))
    v = rng.standard_normal((B, H, T, Dv))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, H, T))))
    g = -np.log1p(np.exp(rng.standard_normal((B, H, T, D) if kda else (B, H, T)))) * 0.1
    h = rng.standard_normal((B, H, D, Dv)) * 0.05 if h0 else None
    return q, k, v, beta, g, h


# --------------------------------------------------------------------------- #
#  full forwards vs the published recurrent rules
# --------------------------------------------------------------------------- #
@pytest.mark.parametrize("C", [16, 32, 64])
def test_gdn_chunked_equals_recurrent(C):
    q, k, v, beta, g, h0 = _inputs(1, 2, 2, 128, 32, 24)
    o, hT = gdn_reference(q, k, v, beta, g, C=C, h0=h0, dtype=np.float64)
    o_r, h_r = gdn_recurrent(q, k, v, beta, g, h0=h0)
    assert max_abs(o, o_r) < 1e-12 and max_abs(hT, h_r) < 1e-12


def test_gdn_golden_fixture():
    z = np.load(os.path.join(GOLDEN, "gdn_recurrent_B1H1T128D128.npz"))
    x = {n: z[n].astype(np.float64) for n in z.files}
    o, hT = gdn_reference(x["q"], x["k"], x["v"], x["beta"], x["g"], C=64, h0=x["h0"],
                          dtype=np.float64)
    assert max_rel(o, x["o"]) < 1e-6 and max_rel(hT, x["h_final"]) < 1e-6


def test_kda_chunked_equals_recurrent_and_golden():
    q, k, v, beta, g, h0 = _inputs(2, 1, 2, 96, 16, 16, kda=True)
    o, hT = kda_reference(q, k, v, beta, g, C=32, h0=h0, dtype=np.float64)
    o_r, h_r = kda_recurrent(q, k, v, beta, g, h0=h0)
    assert max_abs(o, o_r) < 1e-12 and max_abs(hT, h_r) < 1e-12
    z = np.load(os.path.join(GOLDEN, "kda_recurrent_B1H1T64D32.npz"))
    x = {n: z[n].astype(np.float64) for n in z.files}
    o, hT = kda_reference(x["q"], x["k"], x["v"], x["beta"], x["g"], C=16, h0=x["h0"],
                          dtype=np.float64)
    assert max_rel(o, x["o"]) < 1e-6 and max_rel(hT, x["h_final"]) < 1e-6


def test_deltanet_is_gdn_without_decay_and_recurrent():
    q, k, v, beta, g, h0 = _inputs(3, 1, 3, 64, 16)
    d = deltanet_reference(q, k, v, beta, C=16, h0=h0, dtype=np.float64)
    o_g, h_g = gdn_reference(q, k, v, beta, np.zeros_like(g), C=16, h0=h0, dtype=np.float64)
    o_r, h_r = gdn_recurrent(q, k, v, beta, np.zeros_like(g), h0=h0)
    assert max_abs(d["o"].reshape(o_g.shape), o_g) < 1e-12
    assert max_abs(d["final"], h_r) < 1e-12 and max_abs(o_g, o_r) < 1e-12
    # the staged intermediates obey their defining identities
    nc, C = 4, 16
    M = 3 * nc
    I = np.eye(C)
    assert max_abs(d["T"] @ (I + d["A"]), np.broadcast_to(I, (M, C, C))) < 1e-12
    kb = (k * beta[..., None]).reshape(M, C, -1)
    assert max_abs(d["W"].reshape(M, C, -1), d["T"] @ kb) < 1e-12
    assert max_abs(d["h_state"][:, :, 0], h0) == 0.0


def test_kda_with_channel_constant_gate_is_gdn():
    q, k, v, beta, g, h0 = _inputs(4, 1, 2, 64, 16)
    o_k, h_k = kda_reference(q, k, v, beta, np.repeat(g[..., None], 16, -1), C=32, h0=h0,
                             dtype=np.float64)
    o_g, h_g = gdn_reference(q, k, v, beta, g, C=32, h0=h0, dtype=np.float64)
    assert max_abs(o_k, o_g) < 1e-12 and max_abs(h_k, h_g) < 1e-12


# --------------------------------------------------------------------------- #
#  invariants of the GDN forward
# --------------------------------------------------------------------------- #
def test_gdn_chunk_size_invariance():
    q, k, v, beta, g, h0 = _inputs(5, 1, 2, 128, 16)
    outs = [gdn_reference(q, k, v, beta, g, C=C, h0=h0, dtype=np.float64) for C in (16, 32, 64)]
    for o, h in outs[1:]:
        assert max_abs(o, outs[0][0]) < 1e-12 and max_abs(h, outs[0][1]) < 1e-12


def test_gdn_state_passing():
    """[0,T) in one call == [0,T/2) then [T/2,T) started from the first half's final state."""
    q, k, v, beta, g, h0 = _inputs(6, 2, 2, 128, 16)
    o, hT = gdn_reference(q, k, v, beta, g, C=32, h0=h0, dtype=np.float64)
    s = slice(0, 64)
    e = slice(64, 128)
    o1, h1 = gdn_reference(q[:, :, s], k[:, :, s], v[:, :, s], beta[:, :, s], g[:, :, s], C=32,
                           h0=h0, dtype=np.float64)
    o2, h2 = gdn_reference(q[:, :, e], k[:, :, e], v[:, :, e], beta[:, :, e], g[:, :, e], C=32,
                           h0=h1, dtype=np.float64)
    assert max_abs(np.concatenate([o1, o2], 2), o) < 1e-12 and max_abs(h2, hT) < 1e-12


def test_gdn_beta_zero_closed_form():
    """beta = 0: the state only decays, S_c = e^{sum g before chunk c} h0, o = scale (q e^G) S_c."""
    q, k, v, beta, g, h0 = _inputs(7, 1, 2, 64, 16)
    C = 16
    o, hT = gdn_reference(q, k, v, np.zeros_like(beta), g, C=C, h0=h0, dtype=np.float64)
    G = within_chunk_cumsum(g, C)
    total = g.sum(-1)
    assert max_abs(hT, np.exp(total)[..., None, None] * h0) < 1e-12
    before = np.concatenate([np.zeros_like(g[..., :1]), np.cumsum(g, -1)[..., :-1]], -1)
    start = before.reshape(1, 2, 4, C)[..., 0]                   # decay up to each chunk start
    Sc = np.exp(start)[..., None, None] * h0[:, :, None]         # [B,H,nc,D,D]
    qc = (q * np.exp(G)[..., None]).reshape(1, 2, 4, C, 16)
    o_ref = np.einsum("bhncd,bhnde->bhnce", qc, Sc).reshape(o.shape) * 16 ** -0.5
    assert max_abs(o, o_ref) < 1e-12


def test_gdn_linear_in_v():
    q, k, v, beta, g, _ = _inputs(8, 1, 2, 64, 16)
    v2 = np.random.default_rng(80).standard_normal(v.shape)
    o1, h1 = gdn_reference(q, k, v, beta, g, C=16, dtype=np.float64)
    o2, h2 = gdn_reference(q, k, v2, beta, g, C=16, dtype=np.float64)
    o3, h3 = gdn_reference(q, k, 2 * v - 3 * v2, beta, g, C=16, dtype=np.float64)
    assert max_abs(o3, 2 * o1 - 3 * o2) < 1e-12 and max_abs(h3, 2 * h1 - 3 * h2) < 1e-12


def test_gdn_loop_equals_batched_fp32():
    q, k, v, beta, g, h0 = _inputs(9, 2, 2, 128, 32)
    a = gdn_reference(q, k, v, beta, g, C=64, h0=h0, dtype=np.float32, loop=True)
    b = gdn_reference(q, k, v, beta, g, C=64, h0=h0, dtype=np.float32, loop=False)
    assert max_abs(a[0], b[0]) < 1e-5 and max_abs(a[1], b[1]) < 1e-5


def test_fp32_oracle_close_to_fp64():
    q, k, v, beta, g, h0 = _inputs(10, 1, 2, 256, 128)
    o32, h32 = gdn_reference(q, k, v, beta, g, C=64, h0=h0, dtype=np.float32)
    o64, h64 = gdn_reference(q, k, v, beta, g, C=64, h0=h0, dtype=np.float64)
    assert max_rel(o32, o64) < 1e-5 and max_rel(h32, h64) < 1e-5


# --------------------------------------------------------------------------- #
#  chunk-local stages
# --------------------------------------------------------------------------- #
def test_tri_inv_identities():
    rng = np.random.default_rng(11)
    C = 64
    A = np.tril(rng.standard_normal((8, C, C)) * 0.05, -1)
    T = tri_inv_reference(A)
    I = np.eye(C)
    assert max_abs(T @ (I + A), np.broadcast_to(I, A.shape)) < 1e-12
    assert np.all(np.triu(T, 1) == 0) and np.all(np.diagonal(T, axis1=1, axis2=2) == 1)
    # A strictly lower is nilpotent: (I + A)^-1 = sum_{p < C} (-A)^p exactly
    neu = np.broadcast_to(I, A.shape).copy()
    P = neu.copy()
    for _ in range(1, C):
        P = P @ (-A)
        neu = neu + P
    assert max_abs(T, neu) < 1e-12
    for m in range(2):
        ref = scipy.linalg.solve_triangular(I + A[m], I, lower=True, unit_diagonal=True)
        assert max_abs(T[m], ref) < 1e-12
    # C = 2 closed form and "upper triangle ignored"
    a = 0.37
    T2 = tri_inv_reference(np.array([[[9.0, 9.0], [a, 9.0]]]))
    assert np.allclose(T2[0], [[1.0, 0.0], [-a, 1.0]], atol=0, rtol=0)


def test_kkt_brute_force_and_special_cases():
    rng = np.random.default_rng(12)
    nc, H, C, D = 2, 3, 8, 5
    k = rng.standard_normal((1, nc * C, H, D))
    beta = rng.uniform(0.1, 1.0, (1, nc * C, H))
    g = -rng.uniform(0.0, 0.3, (1, nc * C, H))
    g_sum = within_chunk_cumsum(g.transpose(0, 2, 1), C).transpose(0, 2, 1)
    L = kkt_reference(k, g_sum, beta, nc, H, C, dtype=np.float64)
    for c in range(nc):
        for h in range(H):
            for i in range(C):
                for j in range(C):
                    ti, tj = c * C + i, c * C + j
                    want = 0.0
                    if i > j:
                        dot = sum(k[0, ti, h, d] * k[0, tj, h, d] for d in range(D))
                        want = dot * np.exp(min(g_sum[0, ti, h] + np.log(beta[0, ti, h])
                                                - g_sum[0, tj, h], 0.0))
                    assert abs(L[ti, h, j] - want) < 1e-12
    # G = 0, beta = 1: strictly_lower(K K^T)
    L1 = kkt_reference(k, np.zeros_like(beta), np.ones_like(beta), nc, H, C, dtype=np.float64)
    kc = k.reshape(nc, C, H, D).transpose(0, 2, 1, 3)
    ref = np.tril(kc @ kc.transpose(0, 1, 3, 2), -1).transpose(0, 2, 1, 3).reshape(nc * C, H, C)
    assert max_abs(L1, ref) < 1e-12


def test_gated_qk_clamped_equals_canonical_in_domain_only():
    """The fused kernels' exp(min(G_i + log b_i - G_j, 0)) equals the canonical b_i safe_exp(G_i -
    G_j) when b <= 1 and G is non-increasing; with b > 1 they differ (the clamp caps at 1)."""
    rng = np.random.default_rng(13)
    C, D = 16, 8
    k = rng.standard_normal((3, C, D))
    G = np.cumsum(-rng.uniform(0, 0.2, (3, C)), -1)
    b = rng.uniform(0.05, 1.0, (3, C))
    clamped = gated_qk_reference(k, k, G, b, causal=False, dtype=np.float64)
    canon = np.tril((k @ k.transpose(0, 2, 1)) * safe_exp(G[..., :, None] - G[..., None, :])
                    * b[..., :, None], -1)
    assert max_abs(clamped, canon) < 1e-12
    big = gated_qk_reference(k, k, G, b * 3.0, causal=False, dtype=np.float64)
    canon3 = canon * 3.0
    assert max_abs(big, canon3) > 1e-3


def test_chunk_intermediates_wy_identities():
    rng = np.random.default_rng(14)
    k = _nrm(rng.standard_normal((4, 16, 8)))
    v = rng.standard_normal((4, 16, 6))
    b = rng.uniform(0, 1, (4, 16))
    G = np.cumsum(-rng.uniform(0, 0.2, (4, 16)), -1)
    A, T, W, U = chunk_intermediates(k, v, b, G)
    # (I + A) W = beta k e^G and (I + A) U = beta v  (the WY equations the solve enforces)
    I = np.eye(16)
    assert max_abs((I + A) @ W, k * (b * np.exp(G))[..., None]) < 1e-12
    assert max_abs((I + A) @ U, v * b[..., None]) < 1e-12


def test_qkv_flash_brute_force():
    rng = np.random.default_rng(15)
    M, C, D, DV = 2, 8, 4, 3
    q, k = rng.standard_normal((M, C, D)), rng.standard_normal((M, C, D))
    v = rng.standard_normal((M, C, DV))
    g = rng.standard_normal((M, C)) * 0.2
    o = qkv_flash_reference(q, k, v, g, dtype=np.float64)
    for m in range(M):
        for i in range(C):
            for e in range(DV):
                want = sum(float(q[m, i] @ k[m, j]) * np.exp(min(g[m, i] - g[m, j], 0.0)) * v[m, j, e]
                           for j in range(i + 1))
                assert abs(o[m, i, e] - want) < 1e-12


def test_scan_stage_reproduces_forward_snapshots():
    """scan_reference fed the way LowerResidentScan feeds chunk_h_scan (transforms/gdn.py:69-102:
    w = W, u = U, k scaled by e^{G_last - G}, decay = e^{G_last}, token-major layout) returns the
    full forward's pre-update states and final state."""
    q, k, v, beta, g, h0 = _inputs(16, 2, 3, 96, 8)
    C = 32
    o, hT, snaps, _ = gdn_reference(q, k, v, beta, g, C=C, h0=h0, dtype=np.float64,
                                    return_snapshots=True)
    B, H, T, D = q.shape
    nc = T // C
    G = within_chunk_cumsum(g, C).reshape(B, H, nc, C)
    _, _, W, U = chunk_intermediates(k.reshape(B, H, nc, C, D), v.reshape(B, H, nc, C, D),
                                     beta.reshape(B, H, nc, C), G)
    kvcs = k.reshape(B, H, nc, C, D) * np.exp(G[..., -1:] - G)[..., None]
    tm = lambda x: x.transpose(0, 2, 3, 1, 4)                    # [B,H,nc,C,D] -> [B,nc,C,H,D]
    h_out, final = scan_reference(tm(W), tm(U), tm(kvcs), np.exp(G[..., -1]), h0=h0,
                                  dtype=np.float64)
    assert max_abs(h_out.transpose(0, 2, 1, 3, 4), snaps) < 1e-12
    assert max_abs(final, hT) < 1e-12
    # decay = 0, one chunk, zero start: final = k^T u exactly
    w1, u1, k1 = (np.random.default_rng(160 + i).standard_normal((1, 1, 4, 2, 3)) for i in range(3))
    _, f1 = scan_reference(w1, u1, k1, np.zeros((1, 2, 1)), dtype=np.float64)
    assert max_abs(f1, np.einsum("bchd,bche->bhde", k1[:, 0], u1[:, 0])) < 1e-12


def test_coefficient_decomposition_reproduces_forward():
    """prepare_gdn_coefficients' host coefficients, used as _gdn_full.py:190-233 uses them (mul
    glue around plain contractions), reproduce gdn_reference."""
    q, k, v, beta, g, _ = _inputs(17, 1, 2, 64, 8)
    C = 16
    B, H, T, D = q.shape
    nc, M, N = T // C, B * H * (T // C), B * H
    cf = prepare_gdn_coefficients(g, beta, C, dtype=np.float64)
    qF, kF, vF = (x.reshape(M, C, D) for x in (q, k, v))
    A = np.tril((kF @ kF.transpose(0, 2, 1)) * cf["coefA"], -1)
    Tm = tri_inv_reference(A)
    W = Tm @ (kF * cf["coef_kb"])
    U = Tm @ (vF * cf["coef_vb"])
    Wb, Ub, kb5 = W.reshape(N, nc, C, D), U.reshape(N, nc, C, D), kF.reshape(N, nc, C, D)
    S = np.zeros((N, D, D))
    hs, vns = [], []
    for c in range(nc):
        hs.append(S)
        vn = Ub[:, c] - Wb[:, c] @ S
        vns.append(vn)
        S = S * cf["coef_S"][:, c] + kb5[:, c].transpose(0, 2, 1) @ (vn * cf["coef_vcs"][:, c])
    h_flat = np.stack(hs, 1).reshape(M, D, D)
    vn_flat = np.stack(vns, 1).reshape(M, C, D)
    o = ((qF @ h_flat) * cf["coef_qg"] + ((qF @ kF.transpose(0, 2, 1)) * cf["coef_o"]) @ vn_flat)
    o = (o * D ** -0.5).reshape(B, H, T, D)
    o_ref, _ = gdn_reference(q, k, v, beta, g, C=C, dtype=np.float64)
    assert max_abs(o, o_ref) < 1e-12


# --------------------------------------------------------------------------- #
#  helpers
# --------------------------------------------------------------------------- #
def test_bf16_round_matches_torch():
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(18).standard_normal(10000).astype(np.float32) * 7
    x[:4] = [0.0, -0.0, 1e-38, 3.0e38]
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(bf16_round(x), ref)


def test_error_metrics():
    r = np.array([1.0, -2.0, 4.0])
    x = r + np.array([0.0, 0.5, 0.0])
    assert max_abs(x, r) == 0.5 and max_rel(x, r) == 0.125
    assert abs(frob_rel(x, r) - 0.5 / np.sqrt(21.0)) < 1e-15


def test_scan_per_channel_decay_brute_force():
    """scan_reference with a per-channel decay vector: S <- diag(d) S + k^T (u - w S), checked
    element by element in plain loops, and equal to the scalar form when d is constant."""
    rng = np.random.default_rng(171)
    B, nc, C, H, D = 1, 2, 3, 2, 4
    w, u, k = (rng.standard_normal((B, nc, C, H, D)) for _ in range(3))
    dec = rng.random((B, H, nc, D))
    h0 = rng.standard_normal((B, H, D, D))
    h_out, final = scan_reference(w, u, k, dec, h0=h0, dtype=np.float64)
    for h in range(H):
        S = [[h0[0, h, i, j] for j in range(D)] for i in range(D)]
        for c in range(nc):
            for i in range(D):
                for j in range(D):
                    assert abs(h_out[0, c, h, i, j] - S[i][j]) < 1e-12
            vc = [[u[0, c, t, h, j] - sum(w[0, c, t, h, d] * S[d][j] for d in range(D))
                   for j in range(D)] for t in range(C)]
            S = [[dec[0, h, c, i] * S[i][j] + sum(k[0, c, t, h, i] * vc[t][j] for t in range(C))
                  for j in range(D)] for i in range(D)]
        assert max_abs(final[0, h], np.array(S)) < 1e-12
    const = np.repeat(dec[..., :1], D, axis=-1)
    hs, fs = scan_reference(w, u, k, const[..., 0], h0=h0, dtype=np.float64)
    hp, fp = scan_reference(w, u, k, const, h0=h0, dtype=np.float64)
    assert max_abs(hs, hp) < 1e-12 and max_abs(fs, fp) < 1e-12
