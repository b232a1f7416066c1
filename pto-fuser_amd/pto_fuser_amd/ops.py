"""Torch-facing operators over the C-ABI library (device memory and streams come from PyTorch).

* :func:`gdn_chunk_forward` — the fused gated delta-rule chunked forward (GDN; DeltaNet when
  ``g is None``): o and the final state h.  Math of gdn_reference
  (examples/attention/_gdn_full.py:57-97) plus an initial state.
* :func:`kda_chunk_forward` — the fused KDA forward (per-channel decay): o and the final state.
  Math of kda_reference (examples/attention/_kda_full.py:42-76) plus an initial state.
* :func:`kkt_inverse` — the standalone gated kkt + (I + A)^-1 stage (fused.py:482-499 followed
  by registry.py:107-127).
* :func:`tri_inv` — the opaque unit-lower inverse (registry.py:107-127).

Every operator validates shapes, dtypes, devices and contiguity on the host and raises
``ValueError`` before launching; a kernel-side failure raises :class:`HipKernelError`.  There
is no CPU fallback: on a machine without the HIP library or a GPU these raise.
"""
from __future__ import annotations

import weakref
from typing import Dict, Optional, Tuple

import torch

from . import _hip

SUPPORTED_C = (64, 128)   # the fused forwards run 64-token chunks; 128 regroups the same chunks
SUPPORTED_D = (128,)


def _dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return _hip.PF_DTYPE_F32
    if dtype == torch.bfloat16:
        return _hip.PF_DTYPE_BF16
    raise ValueError(f"unsupported operand dtype {dtype} (float32 or bfloat16)")


def _require(t: Optional[torch.Tensor], name: str, shape, dtype, device) -> None:
    if t is None:
        return
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a tensor")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if t.dtype != dtype:
        raise ValueError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


class GdnWorkspace:
    """Persistent per-shape workspace of the fused forward (pf_gdn_setup / pf_gdn_teardown):
    the T, P and G intermediates between the chunk-local and the scan kernels.  Allocated once,
    reused by every call with the same shape — the persistent-runner discipline of
    fused.py:93-115."""

    def __init__(self, B, H, T, C, DK, DV, dtype_code, device) -> None:
        lib = _hip.load()
        with torch.cuda.device(device):
            handle = lib.pf_gdn_setup(B, H, T, C, DK, DV, dtype_code)
        if not handle:
            raise _hip.HipKernelError("pf_gdn_setup", _hip.PF_ERR_ALLOC,
                                      "workspace allocation failed or shape unsupported")
        self.handle = handle
        self.bytes = lib.pf_gdn_workspace_bytes(B, H, T, C, DK, DV, dtype_code)
        self._finalizer = weakref.finalize(self, lib.pf_gdn_teardown, handle)

    def close(self) -> None:
        self._finalizer()


_WORKSPACES: Dict[tuple, object] = {}


def _stream_key(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _cached_workspace(key: tuple, make):
    """The workspace cached under ``key`` (shape, device and the current stream), created on
    first use.  One per stream: forwards of the same shape enqueued on two streams would
    otherwise overwrite each other's intermediates.  Creating one allocates device memory, which
    a HIP graph capture must not record: under capture a missing workspace raises (run the call
    once on the capture stream before capturing, as graph.GraphReplayExecutor's warmup does)."""
    ws = _WORKSPACES.get(key)
    if ws is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("no workspace for this shape on the capturing stream: run the "
                               "forward once on that stream before capturing it")
        ws = make()
        _WORKSPACES[key] = ws
    return ws


def gdn_workspace(B, H, T, C, DK, DV, dtype: torch.dtype, device) -> GdnWorkspace:
    code = _dtype_code(dtype)
    key = ("gdn", B, H, T, C, DK, DV, code, str(device), _stream_key(device))
    return _cached_workspace(key, lambda: GdnWorkspace(B, H, T, C, DK, DV, code, device))


class KdaWorkspace:
    """Persistent per-shape workspace of the fused KDA forward (pf_kda_setup / pf_kda_teardown):
    the gated operands, the WY factors, the score and the chunk decays between its two
    kernels."""

    def __init__(self, B, H, T, C, DK, DV, dtype_code, device) -> None:
        lib = _hip.load()
        with torch.cuda.device(device):
            handle = lib.pf_kda_setup(B, H, T, C, DK, DV, dtype_code)
        if not handle:
            raise _hip.HipKernelError("pf_kda_setup", _hip.PF_ERR_ALLOC,
                                      "workspace allocation failed or shape unsupported")
        self.handle = handle
        self.bytes = lib.pf_kda_workspace_bytes(B, H, T, C, DK, DV, dtype_code)
        self._finalizer = weakref.finalize(self, lib.pf_kda_teardown, handle)

    def close(self) -> None:
        self._finalizer()


def kda_workspace(B, H, T, C, DK, DV, dtype: torch.dtype, device) -> KdaWorkspace:
    code = _dtype_code(dtype)
    key = ("kda", B, H, T, C, DK, DV, code, str(device), _stream_key(device))
    return _cached_workspace(key, lambda: KdaWorkspace(B, H, T, C, DK, DV, code, device))


def release_workspaces() -> None:
    for ws in _WORKSPACES.values():
        ws.close()
    _WORKSPACES.clear()


def gdn_chunk_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                      g: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                      h0: Optional[torch.Tensor] = None, chunk_size: int = 64,
                      output_final_state: bool = True,
                      out: Optional[torch.Tensor] = None,
                      final_out: Optional[torch.Tensor] = None,
                      workspace: Optional[GdnWorkspace] = None,
                      ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Fused chunked gated delta-rule forward on the current HIP stream.

    q, k [B,H,T,DK] and v [B,H,T,DV] in float32 or bfloat16; beta, g [B,H,T] float32 (g is the
    per-token log decay, summed within chunks by the kernel; None = DeltaNet); h0 [B,H,DK,DV]
    float32 or None.  Returns (o [B,H,T,DV] float32 scaled by ``scale`` (default DK^-1/2),
    h_final [B,H,DK,DV] float32 or None).  chunk_size 64 or 128: both run the 64-token kernels
    (the result does not depend on the chunk size); T must be a multiple of it."""
    if q.dim() != 4:
        raise ValueError(f"q must be [B,H,T,DK], got shape {tuple(q.shape)}")
    B, H, T, DK = q.shape
    DV = v.shape[-1]
    C = int(chunk_size)
    if C not in SUPPORTED_C or DK not in SUPPORTED_D or DV not in SUPPORTED_D:
        raise ValueError(f"unsupported shape C={C} DK={DK} DV={DV} "
                         f"(C in {SUPPORTED_C}, DK/DV in {SUPPORTED_D})")
    if T % C:
        raise ValueError(f"T={T} must be a multiple of the chunk size {C}")
    dev = q.device
    if dev.type != "cuda":
        raise ValueError(f"q must be on a HIP device, got {dev}")
    code = _dtype_code(q.dtype)
    _require(q, "q", (B, H, T, DK), q.dtype, dev)
    _require(k, "k", (B, H, T, DK), q.dtype, dev)
    _require(v, "v", (B, H, T, DV), q.dtype, dev)
    _require(beta, "beta", (B, H, T), torch.float32, dev)
    _require(g, "g", (B, H, T), torch.float32, dev)
    _require(h0, "h0", (B, H, DK, DV), torch.float32, dev)
    o = out if out is not None else torch.empty(B, H, T, DV, device=dev, dtype=torch.float32)
    _require(o, "out", (B, H, T, DV), torch.float32, dev)
    hf = None
    if output_final_state:
        hf = final_out if final_out is not None else torch.empty(B, H, DK, DV, device=dev,
                                                                 dtype=torch.float32)
        _require(hf, "final_out", (B, H, DK, DV), torch.float32, dev)
    ws = workspace or gdn_workspace(B, H, T, C, DK, DV, q.dtype, dev)
    sc = float(DK ** -0.5 if scale is None else scale)
    lib = _hip.load()
    st = lib.pf_gdn_exec(_hip.ptr(q), _hip.ptr(k), _hip.ptr(v), _hip.ptr(beta), _hip.ptr(g),
                         _hip.ptr(h0), _hip.ptr(o), _hip.ptr(hf), B, H, T, C, DK, DV, code, sc,
                         ws.handle, _hip.current_stream_handle(dev))
    _hip.check("pf_gdn_exec", st)
    return o, hf


def kkt_inverse(k: torch.Tensor, g: Optional[torch.Tensor], beta: torch.Tensor,
                chunk_size: int = 64, g_is_cumsum: bool = False, return_A: bool = False):
    """Gated kkt + unit-lower inverse over all chunks.

    k [M*C, DK] (or any shape flattening to it) float32/bfloat16; g, beta [M*C] float32.
    Returns T = (I + A)^-1 [M, C, C] float32 (and A [M, C, C] float32 if ``return_A``)."""
    C = int(chunk_size)
    DK = k.shape[-1]
    if C != 64 or DK not in SUPPORTED_D:     # T is the per-chunk inverse: its size is C
        raise ValueError(f"unsupported shape C={C} DK={DK} (C = 64, DK in {SUPPORTED_D})")
    n = k.numel() // DK
    if n % C:
        raise ValueError(f"token count {n} is not a multiple of C={C}")
    M = n // C
    dev = k.device
    if dev.type != "cuda":
        raise ValueError(f"k must be on a HIP device, got {dev}")
    code = _dtype_code(k.dtype)
    if not k.is_contiguous():
        raise ValueError("k must be contiguous")
    _require(beta.reshape(-1) if beta.is_contiguous() else beta, "beta", (n,), torch.float32, dev)
    if g is not None:
        _require(g.reshape(-1) if g.is_contiguous() else g, "g", (n,), torch.float32, dev)
    Tm = torch.empty(M, C, C, device=dev, dtype=torch.float32)
    A = torch.empty(M, C, C, device=dev, dtype=torch.float32) if return_A else None
    st = _hip.load().pf_kkt_inv_exec(_hip.ptr(k), _hip.ptr(g), _hip.ptr(beta), _hip.ptr(A),
                                     _hip.ptr(Tm), M, C, DK, code, int(bool(g_is_cumsum)),
                                     _hip.current_stream_handle(dev))
    _hip.check("pf_kkt_inv_exec", st)
    return (Tm, A) if return_A else Tm


STAGE_C = (16, 32, 64, 128)
TRI_INV_C = (16, 32, 48, 64, 128)
STAGE_D = (64, 128)


def _stage_shape(C: int, D: int, dtype: torch.dtype) -> None:
    if C not in STAGE_C or D not in STAGE_D or (dtype == torch.bfloat16 and C < 32):
        raise ValueError(f"unsupported stage shape C={C} D={D} {dtype} (C in {STAGE_C}, "
                         f"D in {STAGE_D}; bfloat16 needs C >= 32)")


def _on_device(t: torch.Tensor, name: str) -> torch.device:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a tensor on a HIP device")
    return t.device


def gated_qk(a: torch.Tensor, b: torch.Tensor, g: Optional[torch.Tensor] = None,
             beta: Optional[torch.Tensor] = None, *, chunk_size: int, heads: int = 1,
             causal: bool = True, mask: Optional[torch.Tensor] = None,
             a_scale: Optional[torch.Tensor] = None, b_scale: Optional[torch.Tensor] = None,
             out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Gated a bᵀ per chunk: L_ij = (a'_i·b'_j)·exp(min(g_i + log β_i − g_j, 0))·mask_ij.

    ``heads = 1``: a, b are the native batch [M, C, D] (any shape flattening to it), g/β [M, C];
    L is [M, C, C].  ``heads = H``: a, b are the token layout [nc*C, H, D] (= [1, T, H, D]),
    g/β [nc*C, H], L is [nc*C, H, C] — the two layouts of kkt_fused_lib.cpp's callers
    (fused.py:200-290).  ``mask`` [C, C] float32 overrides ``causal`` (True: i ≥ j, False: i > j).
    ``a_scale``/``b_scale`` (float32, a's/b's shape) multiply the operands first: the per-channel
    prologue of qk_prologue (fused.py:293-340).  g, β, mask, scales may be None."""
    dev = _on_device(a, "a")
    C, H, D = int(chunk_size), int(heads), a.shape[-1]
    code = _dtype_code(a.dtype)
    _stage_shape(C, D, a.dtype)
    n = a.numel() // D
    if n % (C * H):
        raise ValueError(f"{n} rows do not split into chunks of {C} tokens x {H} heads")
    nc = n // (C * H)
    for name, t in (("a", a), ("b", b)):
        _require(t.reshape(n, D) if t.is_contiguous() else t, name, (n, D), a.dtype, dev)
    for name, t in (("a_scale", a_scale), ("b_scale", b_scale)):
        if t is not None:
            _require(t.reshape(n, D) if t.is_contiguous() else t, name, (n, D), torch.float32, dev)
    for name, t in (("g", g), ("beta", beta)):
        if t is not None:
            _require(t.reshape(n) if t.is_contiguous() else t, name, (n,), torch.float32, dev)
    _require(mask, "mask", (C, C), torch.float32, dev)
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"out_dtype must be float32 or bfloat16, got {out_dtype}")
    L = torch.empty((nc, C, C) if H == 1 else (nc * C, H, C), device=dev, dtype=out_dtype)
    st = _hip.load().pf_gated_qk_exec(
        _hip.ptr(a), _hip.ptr(b), _hip.ptr(a_scale), _hip.ptr(b_scale), _hip.ptr(g),
        _hip.ptr(beta), _hip.ptr(mask), _hip.ptr(L), nc, H, C, D, code, int(bool(causal)),
        _dtype_code(out_dtype), _hip.current_stream_handle(dev))
    _hip.check("pf_gated_qk_exec", st)
    return L


def qkv_flash(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: Optional[torch.Tensor] = None,
              beta: Optional[torch.Tensor] = None, *, chunk_size: int,
              q_scale: Optional[torch.Tensor] = None,
              k_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """chunk_o flash, one launch: o = causal_incl((q'k'ᵀ)·exp(min(g_i + log β_i − g_j, 0)))·v.

    q, k, v [M, C, D] (any shape flattening to it), float32 or bfloat16; g, β [M, C] float32 or
    None; q_scale/k_scale [M, C, D] float32 or None (the per-channel qkvp form).  Returns o
    [M, C, D] float32 (qkv_fused.h:62-175 semantics)."""
    dev = _on_device(q, "q")
    C, D = int(chunk_size), q.shape[-1]
    code = _dtype_code(q.dtype)
    _stage_shape(C, D, q.dtype)
    n = q.numel() // D
    if n % C:
        raise ValueError(f"{n} rows do not split into chunks of {C}")
    M = n // C
    for name, t in (("q", q), ("k", k), ("v", v)):
        _require(t.reshape(n, D) if t.is_contiguous() else t, name, (n, D), q.dtype, dev)
    for name, t in (("q_scale", q_scale), ("k_scale", k_scale)):
        if t is not None:
            _require(t.reshape(n, D) if t.is_contiguous() else t, name, (n, D), torch.float32, dev)
    for name, t in (("g", g), ("beta", beta)):
        if t is not None:
            _require(t.reshape(n) if t.is_contiguous() else t, name, (n,), torch.float32, dev)
    o = torch.empty(M, C, D, device=dev, dtype=torch.float32)
    st = _hip.load().pf_qkv_flash_exec(
        _hip.ptr(q), _hip.ptr(k), _hip.ptr(v), _hip.ptr(q_scale), _hip.ptr(k_scale), _hip.ptr(g),
        _hip.ptr(beta), _hip.ptr(o), M, C, D, code, _hip.current_stream_handle(dev))
    _hip.check("pf_qkv_flash_exec", st)
    return o


def chunk_scan(w: torch.Tensor, u: torch.Tensor, k: torch.Tensor, decay: torch.Tensor,
               h0: Optional[torch.Tensor] = None, out_dtype: torch.dtype = torch.float32,
               output_final_state: bool = True):
    """Resident-state chunk recurrence (chunk_h_scan, scan_fused.h:198-262).

    w, u, k [B, nc, C, H, D] float32/bfloat16 (token-major); decay [B, H, nc] (scalar per chunk) or
    [B, H, nc, D] (per key channel: row d of S scales by decay[..., d]) float32; h0 [B, H, D, D]
    float32 or None.  Returns (h_out [B, nc, H, D, D] in ``out_dtype`` — the state *before* each
    chunk — and the final state [B, H, D, D] float32 or None)."""
    dev = _on_device(w, "w")
    if w.dim() != 5:
        raise ValueError(f"w must be [B, nc, C, H, D], got {tuple(w.shape)}")
    B, nc, C, H, D = w.shape
    code = _dtype_code(w.dtype)
    _stage_shape(C, D, w.dtype)
    for name, t in (("w", w), ("u", u), ("k", k)):
        _require(t, name, (B, nc, C, H, D), w.dtype, dev)
    if decay.dim() == 3:
        perdim = 0
        _require(decay, "decay", (B, H, nc), torch.float32, dev)
    else:
        perdim = 1
        _require(decay, "decay", (B, H, nc, D), torch.float32, dev)
    _require(h0, "h0", (B, H, D, D), torch.float32, dev)
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"out_dtype must be float32 or bfloat16, got {out_dtype}")
    h_out = torch.empty(B, nc, H, D, D, device=dev, dtype=out_dtype)
    final = torch.empty(B, H, D, D, device=dev, dtype=torch.float32) if output_final_state else None
    st = _hip.load().pf_scan_exec(
        _hip.ptr(w), _hip.ptr(u), _hip.ptr(k), _hip.ptr(decay), _hip.ptr(h0), _hip.ptr(h_out),
        _hip.ptr(final), B, H, nc, C, D, code, perdim, _dtype_code(out_dtype),
        _hip.current_stream_handle(dev))
    _hip.check("pf_scan_exec", st)
    return h_out, final


def tri_inv(A: torch.Tensor) -> torch.Tensor:
    """(I + A)^-1 of strictly-lower A [M, C, C] float32 (upper part ignored), C in TRI_INV_C."""
    if A.dim() != 3 or A.shape[1] != A.shape[2]:
        raise ValueError(f"A must be [M, C, C], got {tuple(A.shape)}")
    M, C, _ = A.shape
    if C not in TRI_INV_C:
        raise ValueError(f"tri_inv supports C in {TRI_INV_C}, got {C}")
    if A.dtype != torch.float32 or A.device.type != "cuda" or not A.is_contiguous():
        raise ValueError("A must be a contiguous float32 tensor on a HIP device")
    out = torch.empty_like(A)
    st = _hip.load().pf_tri_inv_exec(_hip.ptr(A), _hip.ptr(out), M, C,
                                     _hip.current_stream_handle(A.device))
    _hip.check("pf_tri_inv_exec", st)
    return out


def kda_chunk_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                      g: torch.Tensor, scale: Optional[float] = None,
                      h0: Optional[torch.Tensor] = None, chunk_size: int = 64,
                      output_final_state: bool = True,
                      out: Optional[torch.Tensor] = None,
                      final_out: Optional[torch.Tensor] = None,
                      workspace: Optional[KdaWorkspace] = None,
                      ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Fused chunked KDA forward (per-channel decay) on the current HIP stream.

    q, k [B,H,T,DK] and v [B,H,T,DV] bfloat16 or float32 (one dtype); beta [B,H,T] float32;
    g [B,H,T,DK] float32 (the per-token, per-channel log decay, summed within chunks by the
    kernel); h0 [B,H,DK,DV] float32 or None.  Returns (o [B,H,T,DV] float32 scaled by ``scale``
    (default DK^-1/2), h_final [B,H,DK,DV] float32 or None).  chunk_size 64 or 128 (both run
    64-token chunks)."""
    if q.dim() != 4:
        raise ValueError(f"q must be [B,H,T,DK], got shape {tuple(q.shape)}")
    B, H, T, DK = q.shape
    DV = v.shape[-1]
    C = int(chunk_size)
    if C not in SUPPORTED_C or DK not in SUPPORTED_D or DV not in SUPPORTED_D:
        raise ValueError(f"unsupported shape C={C} DK={DK} DV={DV} "
                         f"(C in {SUPPORTED_C}, DK/DV in {SUPPORTED_D})")
    if q.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"the fused KDA forward takes bfloat16 or float32 operands, got {q.dtype}")
    if T % C:
        raise ValueError(f"T={T} must be a multiple of the chunk size {C}")
    dev = q.device
    if dev.type != "cuda":
        raise ValueError(f"q must be on a HIP device, got {dev}")
    _require(q, "q", (B, H, T, DK), q.dtype, dev)
    _require(k, "k", (B, H, T, DK), q.dtype, dev)
    _require(v, "v", (B, H, T, DV), q.dtype, dev)
    _require(beta, "beta", (B, H, T), torch.float32, dev)
    if g is None:
        raise ValueError("g (the per-channel log decay [B,H,T,DK]) is required")
    _require(g, "g", (B, H, T, DK), torch.float32, dev)
    _require(h0, "h0", (B, H, DK, DV), torch.float32, dev)
    o = out if out is not None else torch.empty(B, H, T, DV, device=dev, dtype=torch.float32)
    _require(o, "out", (B, H, T, DV), torch.float32, dev)
    hf = None
    if output_final_state:
        hf = final_out if final_out is not None else torch.empty(B, H, DK, DV, device=dev,
                                                                 dtype=torch.float32)
        _require(hf, "final_out", (B, H, DK, DV), torch.float32, dev)
    ws = workspace or kda_workspace(B, H, T, C, DK, DV, q.dtype, dev)
    sc = float(DK ** -0.5 if scale is None else scale)
    lib = _hip.load()
    st = lib.pf_kda_exec(_hip.ptr(q), _hip.ptr(k), _hip.ptr(v), _hip.ptr(beta), _hip.ptr(g),
                         _hip.ptr(h0), _hip.ptr(o), _hip.ptr(hf), B, H, T, C, DK, DV,
                         _dtype_code(q.dtype), sc, ws.handle, _hip.current_stream_handle(dev))
    _hip.check("pf_kda_exec", st)
    return o, hf
