"""CPU stand-ins for the HIP kernels, for host-side tests only.

The product registries launch libptofuser_hip.so and refuse CPU tensors.  To check on the CPU
that the Program builders compute the delta-rule forward and that every rewrite wires its fused
node correctly (layouts, permutes, names), these registries serve the same keys and contracts
with the oracle's restatements (fp64 numpy) in place of the kernels.  Never imported by the
package."""
from __future__ import annotations

import numpy as np
import torch

from oracle.gdn_oracle import gated_qk_reference, scan_reference, tri_inv_reference
from pto_fuser_amd.fused import FusedContract, FusedKernelRegistry, _Recipe
from pto_fuser_amd.registry import OpaqueContract, OpaqueRegistry


def _np(t):
    return t.detach().double().cpu().numpy()


def _t(x, like):
    return torch.from_numpy(np.ascontiguousarray(x)).to(like.dtype if like.is_floating_point()
                                                       else torch.float32)


def _native(params, a):
    M = int(params["nc"]) * int(params["H"])
    D = int(params.get("D", a.shape[-1]))
    C = int(params.get("C", a.numel() // (M * D)))
    return M, C, D


def _scan(inputs, params):
    w, u, k, decay = inputs
    B, H, nc = params["B"], params["H"], params["nc"]
    D = w.shape[-1]
    C = w.numel() // (B * nc * H * D)
    shape = (B, nc, C, H, D)
    d = _np(decay).reshape((B, H, nc, D) if params.get("perdim_decay") else (B, H, nc))
    h_out, final = scan_reference(_np(w).reshape(shape), _np(u).reshape(shape),
                                  _np(k).reshape(shape), d, dtype=np.float64)
    return [_t(h_out, w), _t(final, w)]


def _gated(a, b, g, beta, params, causal, scales=None):
    M, C, D = _native(params, a)
    A, Bm = _np(a).reshape(M, C, D), _np(b).reshape(M, C, D)
    if scales is not None:
        A, Bm = A * _np(scales[0]).reshape(M, C, D), Bm * _np(scales[1]).reshape(M, C, D)
    G = np.zeros((M, C)) if g is None else _np(g).reshape(M, C)
    bt = np.ones((M, C)) if beta is None else _np(beta).reshape(M, C)
    return gated_qk_reference(A, Bm, G, bt, causal=causal, dtype=np.float64)


def _kkt_native(inputs, params):
    k, g, beta = inputs
    return [_t(_gated(k, k, g, beta, params, False), k)]


def _qk_native(inputs, params):
    a, b, g, beta = inputs
    return [_t(_gated(a, b, g, beta, params, params.get("causal", True)), a)]


def _prologue(inputs, params):
    q, k, P, invP = inputs
    return [_t(_gated(q, k, None, None, params, True, (P, invP)), q)]


def _flash(inputs, params):
    q, k, v, g, beta = inputs
    M, C, D = _native(params, q)
    L = _gated(q, k, g, beta, params, True)
    return [torch.from_numpy(L @ _np(v).reshape(M, C, D)).float()]


def _flash_perdim(inputs, params):
    q, k, v, ag, bg = inputs
    M, C, D = _native(params, q)
    L = _gated(q, k, None, None, params, True, (ag, bg))
    return [torch.from_numpy(L @ _np(v).reshape(M, C, D)).float()]


def _cpu(fn, *slots) -> _Recipe:
    """A library-free recipe (empty src_file): the launch ignores lib and ws."""
    return _Recipe(src_dir="", src_file="", defines=lambda p: dict(p), setup_sym="",
                   teardown_sym="", bind=lambda lib: None,
                   launch=lambda lib, ws, inputs, params: fn(inputs, params),
                   contract=FusedContract(list(slots), [], [], torch.float32, "CPU stand-in"))


def cpu_fused_registry() -> FusedKernelRegistry:
    reg = FusedKernelRegistry()
    reg.register("chunk_h_scan", _cpu(_scan, "w", "u", "k", "decay"))
    for s in ("", "_v2"):
        reg.register("kkt_gated_native" + s, _cpu(_kkt_native, "k", "g", "b"))
        reg.register("gated_qk_native" + s, _cpu(_qk_native, "a", "b", "g", "b"))
        reg.register("qk_prologue" + s, _cpu(_prologue, "q", "k", "P", "iP"))
        reg.register("qkv_flash_native" + s, _cpu(_flash, "q", "k", "v", "g", "b"))
        reg.register("qkvp_flash_native" + s, _cpu(_flash_perdim, "q", "k", "v", "a", "b"))
    return reg


def cpu_opaque_registry() -> OpaqueRegistry:
    reg = OpaqueRegistry()
    reg.register("tri_inv_rec_unroll", factory=lambda: None,
                 lowering=lambda raw, ins, p: torch.from_numpy(
                     tri_inv_reference(np.tril(_np(ins[0]), -1))).float(),
                 contract=OpaqueContract([torch.float32], torch.float32, "CPU stand-in"))
    return reg
