"""Torch-facing operators over the C-ABI library (device memory and streams come from PyTorch).

* :func:`gdn_chunk_forward` — the fused gated delta-rule chunked forward (GDN; DeltaNet when
  ``g is None``): o and the final state h.  Math of gdn_reference
  (examples/attention/_gdn_full.py:57-97) plus an initial state.
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

SUPPORTED_C = (64,)
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
        self.key = (B, H, T, C, DK, DV, dtype_code, str(device))
        self.bytes = lib.pf_gdn_workspace_bytes(B, H, T, C, DK, DV, dtype_code)
        self._finalizer = weakref.finalize(self, lib.pf_gdn_teardown, handle)

    def close(self) -> None:
        self._finalizer()


_WORKSPACES: Dict[tuple, GdnWorkspace] = {}


def gdn_workspace(B, H, T, C, DK, DV, dtype: torch.dtype, device) -> GdnWorkspace:
    code = _dtype_code(dtype)
    key = (B, H, T, C, DK, DV, code, str(device))
    ws = _WORKSPACES.get(key)
    if ws is None:
        ws = GdnWorkspace(B, H, T, C, DK, DV, code, device)
        _WORKSPACES[key] = ws
    return ws


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
    h_final [B,H,DK,DV] float32 or None)."""
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
    if C not in SUPPORTED_C or DK not in SUPPORTED_D:
        raise ValueError(f"unsupported shape C={C} DK={DK}")
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


def tri_inv(A: torch.Tensor) -> torch.Tensor:
    """(I + A)^-1 of strictly-lower A [M, C, C] float32 (upper part ignored), C in 16..64."""
    if A.dim() != 3 or A.shape[1] != A.shape[2]:
        raise ValueError(f"A must be [M, C, C], got {tuple(A.shape)}")
    M, C, _ = A.shape
    if C not in (16, 32, 48, 64):
        raise ValueError(f"tri_inv supports C in (16, 32, 48, 64), got {C}")
    if A.dtype != torch.float32 or A.device.type != "cuda" or not A.is_contiguous():
        raise ValueError("A must be a contiguous float32 tensor on a HIP device")
    out = torch.empty_like(A)
    st = _hip.load().pf_tri_inv_exec(_hip.ptr(A), _hip.ptr(out), M, C,
                                     _hip.current_stream_handle(A.device))
    _hip.check("pf_tri_inv_exec", st)
    return out
