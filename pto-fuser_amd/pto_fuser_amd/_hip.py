"""ctypes binding of libptofuser_hip.so — the C-ABI boundary (include/pto_fuser_hip.h).

The reference binds its kernel ``.so`` files the same way (src/pto_fuser/fused.py:50-55:
raw ``data_ptr()`` values and the borrowed current stream); here the stream is
``torch.cuda.current_stream().cuda_stream`` on ROCm.  Every exec returns a status code that
is turned into :class:`HipKernelError`; there is no fallback path — if the library cannot be
loaded, the call raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

from . import _build

PF_DTYPE_F32 = 0
PF_DTYPE_BF16 = 1
PF_OK = 0
PF_ERR_ARG = -1
PF_ERR_WORKSPACE = -2
PF_ERR_ALLOC = -3
PF_ERR_SCRATCH = -4

c_void_p, c_int, c_float, c_size_t = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes); the complete exported surface of include/pto_fuser_hip.h
SIGNATURES = {
    "pf_status_string": (ctypes.c_char_p, [c_int]),
    "pf_abi_version": (c_int, []),
    "pf_source_hash": (ctypes.c_char_p, []),
    "pf_gdn_workspace_bytes": (c_size_t, [c_int] * 7),
    "pf_gdn_setup": (c_void_p, [c_int] * 7),
    "pf_gdn_create": (c_void_p, []),
    "pf_gdn_reserve": (c_int, [c_void_p] + [c_int] * 7),
    "pf_gdn_exec": (c_int, [c_void_p] * 8 + [c_int] * 7 + [c_float, c_void_p, c_void_p]),
    "pf_gdn_teardown": (None, [c_void_p]),
    "pf_gdn_exec_static": (c_int, [c_void_p] * 8 + [c_int] * 7 + [c_float, c_void_p]),
    "pf_gdn_chunk_local_exec": (c_int, [c_void_p] * 4 + [c_int] * 7 + [c_float, c_void_p, c_void_p]),
    "pf_gdn_scan_output_exec": (c_int, [c_void_p] * 7 + [c_int] * 7 + [c_void_p, c_void_p]),
    "pf_kkt_inv_exec": (c_int, [c_void_p] * 5 + [c_int] * 5 + [c_void_p]),
    "pf_tri_inv_exec": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "pf_gated_qk_exec": (c_int, [c_void_p] * 8 + [c_int] * 7 + [c_void_p]),
    "pf_qkv_flash_exec": (c_int, [c_void_p] * 8 + [c_int] * 4 + [c_void_p]),
    "pf_scan_exec": (c_int, [c_void_p] * 7 + [c_int] * 8 + [c_void_p]),
    "pf_kda_workspace_bytes": (c_size_t, [c_int] * 7),
    "pf_kda_setup": (c_void_p, [c_int] * 7),
    "pf_kda_create": (c_void_p, []),
    "pf_kda_reserve": (c_int, [c_void_p] + [c_int] * 7),
    "pf_kda_exec": (c_int, [c_void_p] * 8 + [c_int] * 7 + [c_float, c_void_p, c_void_p]),
    "pf_kda_teardown": (None, [c_void_p]),
    "pf_gated_qk_setup": (c_void_p, []),
    "pf_gated_qk_teardown": (None, [c_void_p]),
    "pf_qkv_flash_setup": (c_void_p, []),
    "pf_qkv_flash_teardown": (None, [c_void_p]),
    "pf_scan_setup": (c_void_p, []),
    "pf_scan_teardown": (None, [c_void_p]),
}


class HipKernelError(RuntimeError):
    """A libptofuser_hip call returned a non-zero status."""

    def __init__(self, fn: str, status: int, text: str) -> None:
        super().__init__(f"{fn} failed with status {status}: {text}")
        self.fn, self.status = fn, status


_LIB: Optional[ctypes.CDLL] = None


def lib_path() -> str:
    return os.environ.get("PF_HIP_LIB", _build.LIB_PATH)


class StaleLibraryError(RuntimeError):
    """The library on disk was built from sources other than the tree's current ones."""


def load(build_if_missing: bool = True) -> ctypes.CDLL:
    """Load (once) the HIP library and bind every signature.  Builds it first only when no
    library file exists yet.  The in-tree library must carry the current tree's source hash
    (``_build.source_hash()``): one built from other sources raises :class:`StaleLibraryError`
    instead of running old kernels.  ``PF_HIP_LIB`` names another library file and skips the
    check (for libraries built elsewhere on purpose)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = lib_path()
    explicit = "PF_HIP_LIB" in os.environ
    if not os.path.exists(path):
        if not build_if_missing or explicit:
            raise FileNotFoundError(f"libptofuser_hip.so not found at {path}")
        _build.ensure_built()
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)          # AttributeError here = ABI drift, loudly
        fn.restype = res
        fn.argtypes = args
    if not explicit:
        built, tree = lib.pf_source_hash().decode(), _build.source_hash()
        if built != tree:
            raise StaleLibraryError(
                f"{path} was built from other sources (library {built}, tree {tree}): "
                f"rebuild it with __graft_entry__.build() before running")
    _LIB = lib
    return lib


def status_text(status: int) -> str:
    return load().pf_status_string(status).decode()


def check(fn: str, status: int) -> None:
    if status != PF_OK:
        raise HipKernelError(fn, status, status_text(status))


def ptr(t) -> Optional[int]:
    """Raw device pointer of a tensor (None stays None -> NULL)."""
    return None if t is None else t.data_ptr()


def current_stream_handle(device=None) -> int:
    import torch
    return torch.cuda.current_stream(device).cuda_stream
