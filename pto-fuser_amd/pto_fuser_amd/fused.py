"""Fused-kernel registry: the FusedNode backend.

A ``FusedNode`` names one HIP kernel of libptofuser_hip.so that stands in for a staged
sub-chain.  The registry maps the key to a recipe and builds, per shape key, a ``FusedKernel``:
the loaded library, the workspace its setup symbol returns, and the launch adapter (operand
layout and dtype, output allocation).  Launches go on the current torch stream with no host
synchronisation and no allocation inside the library, so a fused node is capturable into a HIP
graph.

Recipes have the fields of the reference's recipe (src/pto_fuser/fused.py:119-127: src_dir,
src_file, defines, setup_sym, teardown_sym, bind, launch(lib, ws, inputs, params), contract), so
a recipe written for either registry loads in both.  Loading differs: the reference compiles
``src_file`` with bisheng into one ``.so`` per ``-D`` set (fused.py:58-77); this registry loads a
prebuilt ``.so`` as it lies (this build's library is compiled once and dispatches shapes at run
time), and a recipe with an empty ``src_file`` launches without a library.

Keys and contracts are the reference's, so its programs and transforms name the same kernels:

  chunk_h_scan                      pf_scan_exec       resident-state recurrence
  kkt_gated, gated_qk               pf_gated_qk_exec   token layout [1, T, H, D]
  kkt_gated_native[_v2],
  gated_qk_native[_v2]              pf_gated_qk_exec   native batch [M, C, D]
  qk_prologue[_v2]                  pf_gated_qk_exec   per-channel operand prescale
  qkv_flash_native[_v2]             pf_qkv_flash_exec  chunk_o score -> output
  qkvp_flash_native[_v2]            pf_qkv_flash_exec  per-channel chunk_o flash
  gdn_forward                       pf_gdn_exec        the whole GDN forward (two kernels)
  kda_forward                       pf_kda_exec        the whole KDA forward (two kernels)

The last two have no counterpart among the reference's keys: they are the fused forwards of
this build (``ops.gdn_chunk_forward`` / ``ops.kda_chunk_forward``) offered to the compile stack.
Their workspaces are the ops module's cached per-stream ones.

Differences from the reference, all deliberate:

* The ``_v2`` keys (the reference's FFTS-interleave / L2-ring variants, which exist to stop its
  intermediate scores round-tripping HBM) run the same kernels as the plain keys: the HIP kernels
  never write the score to HBM in the first place.
* Operand dtype: bf16 (the MI355X MFMA type) or fp32 instead of fp16.  An fp16 operand is
  converted to bf16; fp32 operands run the fp32 MFMA path.  Gates are fp32.
* The scan accepts any C in {16, 32, 64, 128} and D in {64, 128} (the reference is fixed to
  C = D = 128) and returns the final state.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Any, Callable, Dict, List, Optional, Tuple

import torch

from . import _build, _hip, ops

__all__ = ["FusedContract", "FusedKernel", "FusedKernelRegistry", "default_fused_registry",
           "shared_fused_registry"]


@dataclass
class FusedContract:
    """The pinned interface of one fused kernel."""
    in_slots: List[str]
    in_dtypes: List[Any]
    out_names: List[str]
    out_dtype: Any
    notes: str = ""


@dataclass
class _Recipe:
    src_dir: str
    src_file: str                                 # prebuilt .so, or "" for a library-free launch
    defines: Callable[[dict], Dict[str, int]]     # params -> shape key (the kernel cache key)
    setup_sym: str                                # workspace constructor ("" = none)
    teardown_sym: str                             # workspace destructor ("" = none)
    bind: Callable[[Any], None]                   # argtypes / restypes on the loaded library
    launch: Callable                              # (lib, ws, inputs, params) -> [outputs]
    contract: FusedContract


class FusedKernel:
    """One recipe at one shape key: the library, its workspace and the launch adapter."""

    def __init__(self, lib: Any, launch: Callable, setup_sym: str, teardown_sym: str) -> None:
        self._lib, self._launch, self._teardown = lib, launch, teardown_sym
        self._ws = ctypes.c_void_p(getattr(lib, setup_sym)()) if lib is not None and setup_sym \
            else ctypes.c_void_p(0)

    def run(self, inputs: List[torch.Tensor], params: dict) -> List[torch.Tensor]:
        return self._launch(self._lib, self._ws, inputs, params)

    def close(self) -> None:
        if self._ws and self._teardown and self._lib is not None:
            getattr(self._lib, self._teardown)(self._ws)
        self._ws = ctypes.c_void_p(0)


class FusedKernelRegistry:
    def __init__(self) -> None:
        self._recipes: Dict[str, _Recipe] = {}
        self._cache: Dict[Tuple, FusedKernel] = {}
        self._libs: Dict[str, Any] = {}

    def register(self, key: str, recipe: _Recipe) -> None:
        if key in self._recipes:
            raise ValueError(f"fused kernel {key!r} is already registered")
        self._recipes[key] = recipe

    def keys(self) -> List[str]:
        return sorted(self._recipes)

    def _recipe(self, key: str) -> _Recipe:
        try:
            return self._recipes[key]
        except KeyError:
            raise KeyError(f"no fused kernel registered under {key!r}") from None

    def contract(self, key: str) -> FusedContract:
        return self._recipe(key).contract

    def recipe(self, key: str) -> _Recipe:
        return self._recipe(key)

    def _library(self, r: _Recipe):
        """The loaded library of a recipe, bound once per file (None for a library-free one)."""
        if not r.src_file:
            return None
        path = os.path.join(r.src_dir, r.src_file)
        if path not in self._libs:
            if not path.endswith(".so"):
                raise RuntimeError(f"{path}: this registry loads prebuilt shared libraries only "
                                   f"(build the kernel library first)")
            own = os.path.abspath(path) == os.path.abspath(_hip.lib_path())
            lib = _hip.load() if own else ctypes.CDLL(path)
            r.bind(lib)
            self._libs[path] = lib
        return self._libs[path]

    def kernel(self, key: str, params: dict) -> FusedKernel:
        r = self._recipe(key)
        ck = (key, tuple(sorted(r.defines(params).items())))
        if ck not in self._cache:
            self._cache[ck] = FusedKernel(self._library(r), r.launch, r.setup_sym,
                                            r.teardown_sym)
        return self._cache[ck]

    def run(self, key: str, inputs: List[torch.Tensor], params: dict) -> List[torch.Tensor]:
        return self.kernel(key, params).run(inputs, params)

    def close(self) -> None:
        for k in self._cache.values():
            k.close()
        self._cache.clear()


# --------------------------------------------------------------------------- #
#  operand adapters
# --------------------------------------------------------------------------- #
def _operand_dtype(*ts: torch.Tensor) -> torch.dtype:
    """fp32 if any operand is fp32 or wider, else bf16."""
    return torch.float32 if any(t.dtype in (torch.float32, torch.float64) for t in ts) \
        else torch.bfloat16


def _op(t: torch.Tensor, dtype: torch.dtype, shape=None) -> torch.Tensor:
    t = t.to(dtype) if t.dtype != dtype else t
    if shape is not None:
        t = t.reshape(shape)
    return t.contiguous()


def _f32(t: Optional[torch.Tensor], shape=None) -> Optional[torch.Tensor]:
    if t is None:
        return None
    return _op(t, torch.float32, shape)


def _native_dims(a: torch.Tensor, params: dict) -> Tuple[int, int, int]:
    """(M, C, D) of a native [M, C, D] operand from the node params (M = nc * H)."""
    M = int(params["nc"]) * int(params["H"])
    D = int(params.get("D", a.shape[-1]))
    C = int(params.get("C", a.numel() // (M * D)))
    if M * C * D != a.numel():
        raise ValueError(f"operand of {a.numel()} elements is not [M={M}, C={C}, D={D}]")
    return M, C, D


# --------------------------------------------------------------------------- #
#  chunk_h_scan
# --------------------------------------------------------------------------- #
def _scan_launch(inputs, params) -> List[torch.Tensor]:
    w, u, k, decay = inputs          # [B,nc,C,H,D] x3; decay [B,H,nc] or [B,H,nc,D]
    B, H, nc = int(params["B"]), int(params["H"]), int(params["nc"])
    dt = _operand_dtype(w, u, k)
    D = w.shape[-1]
    C = w.numel() // (B * nc * H * D)
    shape = (B, nc, C, H, D)
    dshape = (B, H, nc, D) if params.get("perdim_decay") else (B, H, nc)
    h_out, final = ops.chunk_scan(_op(w, dt, shape), _op(u, dt, shape), _op(k, dt, shape),
                                  _f32(decay, dshape), out_dtype=dt)
    return [h_out, final.to(dt)]


# --------------------------------------------------------------------------- #
#  gated a·bᵀ (kkt / chunk_o score / per-channel prologue)
# --------------------------------------------------------------------------- #
def _gated_token_layout(a, b, g_sum, beta, params, causal) -> List[torch.Tensor]:
    """Token layout: a, b [1, T, H, D]; g_sum, beta [1, T, H] -> L [T, H, C]."""
    nc, H = int(params["nc"]), int(params["H"])
    D = a.shape[-1]
    T = a.numel() // (H * D)
    C = T // nc
    dt = _operand_dtype(a, b)
    L = ops.gated_qk(_op(a, dt, (T, H, D)), _op(b, dt, (T, H, D)), _f32(g_sum, (T, H)),
                     _f32(beta, (T, H)), chunk_size=C, heads=H, causal=causal, out_dtype=dt)
    return [L]


def _kkt_launch(inputs, params):
    k, g_sum, beta = inputs
    return _gated_token_layout(k, k, g_sum, beta, params, causal=False)


def _gated_qk_launch(inputs, params):
    a, b, g_sum, beta = inputs
    return _gated_token_layout(a, b, g_sum, beta, params, causal=params.get("causal", True))


def _gated_native(a, b, g, beta, params, causal) -> List[torch.Tensor]:
    """Native layout: a, b [M, C, D]; g, beta [M, C] -> L [M, C, C]."""
    M, C, D = _native_dims(a, params)
    dt = _operand_dtype(a, b)
    L = ops.gated_qk(_op(a, dt, (M, C, D)), _op(b, dt, (M, C, D)), _f32(g, (M, C)),
                     _f32(beta, (M, C)), chunk_size=C, causal=causal, out_dtype=dt)
    return [L]


def _kkt_native_launch(inputs, params):
    k, g_native, beta_native = inputs
    return _gated_native(k, k, g_native, beta_native, params, causal=False)


def _gated_qk_native_launch(inputs, params):
    a, b, g_native, beta_native = inputs
    return _gated_native(a, b, g_native, beta_native, params, causal=params.get("causal", True))


def _prologue_launch(inputs, params):
    """L = tril((q ⊙ P)(k ⊙ invP)ᵀ), causal incl. the diagonal (prologue_fused.h:37-107)."""
    q, k, P, invP = inputs
    M, C, D = _native_dims(q, params)
    dt = _operand_dtype(q, k)
    L = ops.gated_qk(_op(q, dt, (M, C, D)), _op(k, dt, (M, C, D)), chunk_size=C, causal=True,
                     a_scale=_f32(P, (M, C, D)), b_scale=_f32(invP, (M, C, D)), out_dtype=dt)
    return [L]


# --------------------------------------------------------------------------- #
#  chunk_o flash
# --------------------------------------------------------------------------- #
def _flash_dims(q, v, params):
    M, C, D = _native_dims(q, params)
    DV = int(params.get("DV", D))
    if DV != D or v.numel() != M * C * DV:
        raise ValueError(f"chunk_o flash needs v of shape [M, C, D] with DV == D (got DV={DV})")
    return M, C, D


def _qkv_launch(inputs, params):
    """o = causal((q·kᵀ)·exp(min(g_i + log β_i − g_j, 0)))·v, fp32 (qkv_fused.h:62-175)."""
    q, k, v, g_native, beta_native = inputs
    M, C, D = _flash_dims(q, v, params)
    dt = _operand_dtype(q, k, v)
    o = ops.qkv_flash(_op(q, dt, (M, C, D)), _op(k, dt, (M, C, D)), _op(v, dt, (M, C, D)),
                      _f32(g_native, (M, C)), _f32(beta_native, (M, C)), chunk_size=C)
    return [o]


def _qkvp_launch(inputs, params):
    """o = tril((q ⊙ coef_ag)·(k ⊙ coef_bg)ᵀ)·v, fp32 (qkv_prologue_fused.h:99-187)."""
    q, k, v, coef_ag, coef_bg = inputs
    M, C, D = _flash_dims(q, v, params)
    dt = _operand_dtype(q, k, v)
    o = ops.qkv_flash(_op(q, dt, (M, C, D)), _op(k, dt, (M, C, D)), _op(v, dt, (M, C, D)),
                      chunk_size=C, q_scale=_f32(coef_ag, (M, C, D)),
                      k_scale=_f32(coef_bg, (M, C, D)))
    return [o]


# --------------------------------------------------------------------------- #
#  whole forwards
# --------------------------------------------------------------------------- #
def _per_token_gate(G: torch.Tensor) -> torch.Tensor:
    """The within-chunk cumulative log decay G [M, C(, D)] back to the per-token gate g the fused
    forwards take (they accumulate g inside each chunk themselves): g_0 = G_0,
    g_i = G_i - G_(i-1)."""
    G = G.float()
    return torch.diff(G, dim=1, prepend=torch.zeros_like(G[:, :1]))


def _whole_dims(q: torch.Tensor, params: dict) -> Tuple[int, int, int, int, int]:
    B, H, nc = int(params["B"]), int(params["H"]), int(params["nc"])
    C, D = int(params["C"]), int(params["D"])
    if q.numel() != B * H * nc * C * D:
        raise ValueError(f"operand of {q.numel()} elements is not [B*H*nc={B * H * nc}, C={C}, "
                         f"D={D}]")
    return B, H, nc, C, D


def _gdn_forward_launch(inputs, params) -> List[torch.Tensor]:
    """o [B,H,nc,C,D] fp32 = the GDN forward of qF, kF, vF [M,C,D] with the cumulative gate
    g_native [M,C] and beta_native [M,C] (_gdn_full.py:103-235), through pf_gdn_exec."""
    q, k, v, g_native, beta_native = inputs
    B, H, nc, C, D = _whole_dims(q, params)
    T = nc * C
    dt = _operand_dtype(q, k, v)
    o, _ = ops.gdn_chunk_forward(_op(q, dt, (B, H, T, D)), _op(k, dt, (B, H, T, D)),
                                 _op(v, dt, (B, H, T, D)), _f32(beta_native, (B, H, T)),
                                 _per_token_gate(g_native.reshape(-1, C)).reshape(B, H, T),
                                 scale=float(params["scale"]), chunk_size=C,
                                 output_final_state=False)
    return [o.reshape(B, H, nc, C, D)]


def _kda_forward_launch(inputs, params) -> List[torch.Tensor]:
    """o [B,H,nc,C,D] fp32 = the KDA forward of qF, kF, vF [M,C,D] (bf16, or fp32 end to end)
    with the per-channel cumulative gate g_native [M,C,D] and beta_native [M,C]
    (_kda_full.py:42-160), through pf_kda_exec."""
    q, k, v, g_native, beta_native = inputs
    B, H, nc, C, D = _whole_dims(q, params)
    T = nc * C
    dt = _operand_dtype(q, k, v)
    o, _ = ops.kda_chunk_forward(_op(q, dt, (B, H, T, D)), _op(k, dt, (B, H, T, D)),
                                 _op(v, dt, (B, H, T, D)), _f32(beta_native, (B, H, T)),
                                 _per_token_gate(g_native.reshape(-1, C, D)).reshape(B, H, T, D),
                                 scale=float(params["scale"]), chunk_size=C,
                                 output_final_state=False)
    return [o.reshape(B, H, nc, C, D)]


# --------------------------------------------------------------------------- #
#  the default registry
# --------------------------------------------------------------------------- #
def _shape_key(*names):
    return lambda p: {n: p[n] for n in names if n in p}


def _bound(lib) -> None:
    """The in-tree library is bound by its loader (_hip.load binds every entry point)."""


def _adapt(fn: Callable) -> Callable:
    """A launch adapter in the recipe convention: the ops module holds the library and the
    workspaces, so the adapter needs only the operands."""
    return lambda lib, ws, inputs, params: fn(inputs, params)


_BF, _F32 = torch.bfloat16, torch.float32


def _hip_recipe(entry: str, defines, launch: Callable, contract: FusedContract) -> _Recipe:
    """A recipe on libptofuser_hip.so; ``entry`` names the exec symbol whose setup / teardown
    pair the recipe holds (the stage kernels export NULL-returning ones)."""
    stem = {"pf_scan_exec": "pf_scan", "pf_gated_qk_exec": "pf_gated_qk",
            "pf_qkv_flash_exec": "pf_qkv_flash"}.get(entry, "")
    return _Recipe(src_dir=_build.LIB_DIR, src_file=_build.LIB_NAME, defines=defines,
                   setup_sym=f"{stem}_setup" if stem else "",
                   teardown_sym=f"{stem}_teardown" if stem else "",
                   bind=_bound, launch=_adapt(launch), contract=contract)


def default_fused_registry() -> FusedKernelRegistry:
    reg = FusedKernelRegistry()
    reg.register("chunk_h_scan", _hip_recipe(
        "pf_scan_exec", _shape_key("B", "H", "nc", "perdim_decay"), _scan_launch,
        FusedContract(
            in_slots=["w", "u", "k", "decay"], in_dtypes=[_BF, _BF, _BF, _F32],
            out_names=["h_out", "final"], out_dtype=_BF,
            notes="resident-state chunk recurrence; w/u/k [B,nc,C,H,D]; decay [B,H,nc] scalar "
                  "or [B,H,nc,D] per key channel (perdim_decay=True); C in {16,32,64,128}, "
                  "D in {64,128}; fp32 operands run fp32 end to end")))
    reg.register("kkt_gated", _hip_recipe(
        "pf_gated_qk_exec", _shape_key("nc", "H"), _kkt_launch,
        FusedContract(
            in_slots=["k", "g_sum", "beta"], in_dtypes=[_BF, _F32, _F32],
            out_names=["L"], out_dtype=_BF,
            notes="gated strict-lower k·kᵀ on the token layout k [1,T,H,D] -> L [T,H,C]")))
    reg.register("gated_qk", _hip_recipe(
        "pf_gated_qk_exec", _shape_key("nc", "H", "causal"), _gated_qk_launch,
        FusedContract(
            in_slots=["a", "b", "g_sum", "beta"], in_dtypes=[_BF, _BF, _F32, _F32],
            out_names=["L"], out_dtype=_BF,
            notes="gated a·bᵀ on the token layout a,b [1,T,H,D]; chunk_o score = "
                  "(q, k, beta=1, causal)")))
    for key, launch, slots, note in (
            ("kkt_gated_native", _kkt_native_launch, ["k", "g_native", "beta_native"],
             "native kkt (k·kᵀ, real beta, strict lower); k [M,C,D], g/beta [M,C]"),
            ("gated_qk_native", _gated_qk_native_launch,
             ["a", "b", "g_native", "beta_native"],
             "native a·bᵀ + gate/mask epilogue; chunk_o Aqk = (q, k, beta=1, causal)")):
        for suffix in ("", "_v2"):
            reg.register(key + suffix, _hip_recipe(
                "pf_gated_qk_exec", _shape_key("nc", "H", "C", "D", "causal"), launch,
                FusedContract(
                    in_slots=list(slots), in_dtypes=[_BF] * (len(slots) - 2) + [_F32, _F32],
                    out_names=["L"], out_dtype=_BF,
                    notes=note + ("; same kernel as the plain key (the score never leaves the "
                                  "chip in either)" if suffix else ""))))
    for suffix in ("", "_v2"):
        reg.register("qk_prologue" + suffix, _hip_recipe(
            "pf_gated_qk_exec", _shape_key("nc", "H", "C", "D"), _prologue_launch,
            FusedContract(
                in_slots=["q", "k", "P", "invP"], in_dtypes=[_BF, _BF, _F32, _F32],
                out_names=["L"], out_dtype=_BF,
                notes="per-channel prologue tril((q⊙P)·(k⊙invP)ᵀ); q/k/P/invP [M,C,D], "
                      "L [M,C,C]")))
    qkv = FusedContract(
        in_slots=["q", "k", "v", "g_native", "beta_native"],
        in_dtypes=[_BF, _BF, _BF, _F32, _F32], out_names=["o"], out_dtype=_F32,
        notes="chunk_o flash: o = tril((q·kᵀ)·exp(min(g_i-g_j,0)))·v in one launch; "
              "q/k/v [M,C,D], o [M,C,D] fp32")
    qkvp = FusedContract(
        in_slots=["q", "k", "v", "coef_ag", "coef_bg"],
        in_dtypes=[_BF, _BF, _BF, _F32, _F32], out_names=["o"], out_dtype=_F32,
        notes="per-channel chunk_o flash: o = tril((q⊙coef_ag)·(k⊙coef_bg)ᵀ)·v in one launch")
    for suffix in ("", "_v2"):
        reg.register("qkv_flash_native" + suffix, _hip_recipe(
            "pf_qkv_flash_exec", _shape_key("nc", "H", "C", "D", "DV"), _qkv_launch, qkv))
        reg.register("qkvp_flash_native" + suffix, _hip_recipe(
            "pf_qkv_flash_exec", _shape_key("nc", "H", "C", "D", "DV"), _qkvp_launch, qkvp))
    reg.register("gdn_forward", _hip_recipe(
        "pf_gdn_exec", _shape_key("B", "H", "nc", "C", "D"), _gdn_forward_launch,
        FusedContract(
            in_slots=["q", "k", "v", "g_native", "beta_native"],
            in_dtypes=[_BF, _BF, _BF, _F32, _F32], out_names=["o"], out_dtype=_F32,
            notes="whole GDN forward: q/k/v [M,C,D] (bf16, or fp32 end to end), cumulative "
                  "gate g_native and beta [M,C] fp32 -> o [B,H,nc,C,D] fp32; C = 64 or 128, "
                  "D = 128")))
    reg.register("kda_forward", _hip_recipe(
        "pf_kda_exec", _shape_key("B", "H", "nc", "C", "D"), _kda_forward_launch,
        FusedContract(
            in_slots=["q", "k", "v", "g_native", "beta_native"],
            in_dtypes=[_BF, _BF, _BF, _F32, _F32], out_names=["o"], out_dtype=_F32,
            notes="whole KDA forward: q/k/v [M,C,D] (bf16, or fp32 end to end), per-channel "
                  "cumulative gate g_native [M,C,D] and beta [M,C] fp32 -> o [B,H,nc,C,D] fp32; "
                  "C = 64 or 128, D = 128")))
    return reg


_DEFAULT: Optional[FusedKernelRegistry] = None


def shared_fused_registry() -> FusedKernelRegistry:
    """Process-wide registry, shared by every executor (and across graph capture/replay)."""
    global _DEFAULT
    if _DEFAULT is None:
        _DEFAULT = default_fused_registry()
    return _DEFAULT
