"""The C-ABI boundary, without a GPU: the built library loads, exports every entry point that
include/*.h declares, the ctypes bindings agree with the header's parameter lists, and the
host-side contract checks (status codes, workspace sizing) behave as documented.  Nothing here
launches a kernel."""
import glob
import os
import re

import pytest

from pto_fuser_amd import _build, _hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    """name -> parameter count, for every function prototype in include/*.h."""
    out = {}
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", " ", open(h).read(), flags=re.S)
        text = re.sub(r"//[^\n]*", " ", text)
        for m in re.finditer(r"\b(pf_\w+)\s*\(([^;{)]*)\)\s*;", text):
            params = [p for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
            out[m.group(1)] = len(params)
    return out


@pytest.fixture(scope="module")
def lib():
    _build.ensure_built()
    return _hip.load()


def test_header_declares_entry_points():
    fns = _header_functions()
    for name in ("pf_gdn_exec", "pf_gdn_setup", "pf_gdn_teardown", "pf_tri_inv_exec",
                 "pf_kkt_inv_exec", "pf_gdn_chunk_local_exec", "pf_gdn_scan_output_exec"):
        assert name in fns, name


def test_library_exports_every_declared_symbol(lib):
    fns = _header_functions()
    missing = [n for n in fns if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_bindings_match_header_arity(lib):
    fns = _header_functions()
    assert set(_hip.SIGNATURES) == set(fns), (set(_hip.SIGNATURES) ^ set(fns))
    for name, (_, argtypes) in _hip.SIGNATURES.items():
        assert len(argtypes) == fns[name], f"{name}: binding has {len(argtypes)} args, header {fns[name]}"


def test_status_strings_and_version(lib):
    assert lib.pf_abi_version() >= 1
    assert _hip.status_text(_hip.PF_OK) == "ok"
    assert "argument" in _hip.status_text(_hip.PF_ERR_ARG)
    assert "workspace" in _hip.status_text(_hip.PF_ERR_WORKSPACE)


def test_workspace_sizing_contract(lib):
    # bf16: T (bf16) + G (fp32), each 256-byte aligned, + a 256-byte slot for the scale (the
    # bf16 scan forms P itself); fp32: T + P (fp32) + G + the slot
    M = 4 * 16 * 64
    al = lambda n: (n + 255) // 256 * 256
    want = al(M * 64 * 64 * 2) + al(M * 64 * 4) + 256
    assert lib.pf_gdn_workspace_bytes(4, 16, 4096, 64, 128, 128, _hip.PF_DTYPE_BF16) == want
    want32 = 2 * al(M * 64 * 64 * 4) + al(M * 64 * 4) + 256
    assert lib.pf_gdn_workspace_bytes(4, 16, 4096, 64, 128, 128, _hip.PF_DTYPE_F32) == want32
    # unsupported shapes / dtypes report size 0 and setup refuses them
    assert lib.pf_gdn_workspace_bytes(1, 1, 100, 64, 128, 128, 1) == 0      # T % C != 0
    assert lib.pf_gdn_workspace_bytes(1, 1, 128, 32, 128, 128, 1) == 0      # C != 64
    assert lib.pf_gdn_workspace_bytes(1, 1, 128, 64, 64, 128, 1) == 0       # DK != 128
    assert lib.pf_gdn_workspace_bytes(1, 1, 128, 64, 128, 128, 7) == 0      # bad dtype
    # the longest chain: 2^22 tokens (32-bit per-chain addressing); one chunk more is refused
    assert lib.pf_gdn_workspace_bytes(1, 1, 1 << 22, 64, 128, 128, 1) > 0
    assert lib.pf_gdn_workspace_bytes(1, 1, (1 << 22) + 64, 64, 128, 128, 1) == 0
    assert lib.pf_gdn_exec(None, None, None, None, None, None, None, None, 1, 1, (1 << 22) + 64, 64,
                           128, 128, 1, 0.1, None, None) == _hip.PF_ERR_ARG
    assert not lib.pf_gdn_setup(1, 1, 100, 64, 128, 128, 1)


@pytest.mark.parametrize("B,H,T,C", [(1, 1, 64, 64), (4, 16, 4096, 64), (1, 32, 32768, 128),
                                     (3, 5, 192, 64)])
def test_fp32_workspace_holds_bf16(lib, B, H, T, C):
    """A handle reserved for the fp32 layout of a shape serves the bf16 call of that shape
    without growing (the integration stub reserves it so)."""
    for fn in (lib.pf_gdn_workspace_bytes, lib.pf_kda_workspace_bytes):
        f32 = fn(B, H, T, C, 128, 128, _hip.PF_DTYPE_F32)
        b16 = fn(B, H, T, C, 128, 128, _hip.PF_DTYPE_BF16)
        assert 0 < b16 <= f32


def test_kda_workspace_and_rejects(lib):
    # W, QE, k e^-G (bf16 [M,C,128] each) + T diag(beta) (bf16 [M,C,C]) + DEC (fp32 [M,128]),
    # 256-B aligned
    M = 2 * 32 * 128
    want = 3 * ((M * 64 * 128 * 2 + 255) // 256 * 256) + (M * 64 * 64 * 2 + 255) // 256 * 256 \
        + (M * 128 * 4 + 255) // 256 * 256
    assert lib.pf_kda_workspace_bytes(2, 32, 8192, 64, 128, 128, _hip.PF_DTYPE_BF16) == want
    # fp32 operands: W, U, QE, KR, P and DEC in fp32
    M1 = 128
    want32 = 4 * ((M1 * 64 * 128 * 4 + 255) // 256 * 256) + (M1 * 64 * 64 * 4 + 255) // 256 * 256 \
        + (M1 * 128 * 4 + 255) // 256 * 256
    assert lib.pf_kda_workspace_bytes(1, 1, 8192, 64, 128, 128, _hip.PF_DTYPE_F32) == want32
    assert lib.pf_kda_workspace_bytes(1, 1, 64, 64, 128, 128, _hip.PF_DTYPE_F32) > 0     # one chunk
    assert lib.pf_kda_workspace_bytes(1, 1, 64, 64, 128, 128, _hip.PF_DTYPE_BF16) > 0    # bf16 too
    assert lib.pf_kda_workspace_bytes(1, 1, 96, 64, 128, 128, _hip.PF_DTYPE_BF16) == 0   # T % C
    assert not lib.pf_kda_setup(1, 1, 100, 64, 128, 128, 1)
    assert lib.pf_kda_workspace_bytes(1, 1, 1 << 22, 64, 128, 128, 1) > 0
    assert lib.pf_kda_workspace_bytes(1, 1, (1 << 22) + 64, 64, 128, 128, 1) == 0
    assert lib.pf_kda_exec(None, None, None, None, None, None, None, None, 1, 1, 128, 64, 128, 128,
                           1, 0.1, None, None) == _hip.PF_ERR_WORKSPACE
    assert lib.pf_kda_exec(None, None, None, None, None, None, None, None, 1, 1, 128, 64, 128, 128,
                           0, 0.1, None, None) == _hip.PF_ERR_WORKSPACE                  # fp32 shape ok
    assert lib.pf_kda_exec(None, None, None, None, None, None, None, None, 1, 1, 128, 64, 128, 128,
                           7, 0.1, None, None) == _hip.PF_ERR_ARG                        # no such dtype
    assert lib.pf_kda_exec(None, None, None, None, None, None, None, None, 1, 1, 64, 64, 128, 128,
                           1, 0.1, None, None) == _hip.PF_ERR_WORKSPACE                  # bf16, one chunk
    assert lib.pf_kda_exec(None, None, None, None, None, None, None, None, 1, 1, 64, 64, 128, 64,
                           1, 0.1, None, None) == _hip.PF_ERR_ARG                        # dv 64


def test_exec_rejects_contract_violations_before_launch(lib):
    """Bad shapes, null pointers and missing workspaces return negative codes; nothing is
    enqueued (the calls are safe without a device)."""
    st = lib.pf_gdn_exec(None, None, None, None, None, None, None, None,
                         1, 1, 128, 64, 128, 128, 1, 0.1, None, None)
    assert st == _hip.PF_ERR_WORKSPACE
    st = lib.pf_gdn_exec(None, None, None, None, None, None, None, None,
                         1, 1, 100, 64, 128, 128, 1, 0.1, None, None)
    assert st == _hip.PF_ERR_ARG
    assert lib.pf_tri_inv_exec(None, None, 4, 64, None) == _hip.PF_ERR_ARG
    assert lib.pf_tri_inv_exec(1, 1, 4, 96, None) == _hip.PF_ERR_ARG       # unsupported C
    assert lib.pf_kkt_inv_exec(None, None, None, None, None, 4, 64, 128, 1, 0, None) == _hip.PF_ERR_ARG
    assert lib.pf_gdn_chunk_local_exec(None, None, None, None, 1, 1, 128, 64, 128, 128, 1,
                                       0.1, None, None) == _hip.PF_ERR_WORKSPACE
    assert lib.pf_gdn_scan_output_exec(None, None, None, None, None, None, None, 1, 1, 128, 64,
                                       128, 128, 1, None, None) == _hip.PF_ERR_WORKSPACE
    # stage kernels: null operands, unsupported (C, D, dtype) and bad output dtypes
    assert lib.pf_gated_qk_exec(None, None, None, None, None, None, None, None, 1, 1, 64, 128,
                                1, 1, 0, None) == _hip.PF_ERR_ARG
    assert lib.pf_gated_qk_exec(1, 1, None, None, None, None, None, 1, 1, 1, 16, 128,
                                1, 1, 0, None) == _hip.PF_ERR_ARG      # bf16 needs C >= 32
    assert lib.pf_gated_qk_exec(1, 1, None, None, None, None, None, 1, 1, 1, 64, 96,
                                0, 1, 0, None) == _hip.PF_ERR_ARG      # D = 96
    assert lib.pf_gated_qk_exec(1, 1, None, None, None, None, None, 1, 1, 1, 64, 128,
                                0, 1, 5, None) == _hip.PF_ERR_ARG      # out dtype
    assert lib.pf_qkv_flash_exec(1, 1, None, None, None, None, None, 1, 4, 64, 128, 1,
                                 None) == _hip.PF_ERR_ARG              # v missing
    assert lib.pf_qkv_flash_exec(1, 1, 1, None, None, None, None, 1, 4, 256, 128, 0,
                                 None) == _hip.PF_ERR_ARG              # C = 256
    assert lib.pf_scan_exec(1, 1, 1, None, None, 1, None, 1, 1, 2, 64, 128, 1, 0, 0,
                            None) == _hip.PF_ERR_ARG                   # decay missing
    assert lib.pf_scan_exec(1, 1, 1, 1, None, 1, None, 0, 1, 2, 64, 128, 1, 0, 0,
                            None) == _hip.PF_ERR_ARG                   # B = 0


def test_static_forward_rejects_on_host(lib):
    """The allocation-free forward refuses an input beyond its static scratch (8192 bf16 chunks)
    and unsupported shapes before touching the device (safe without one)."""
    st = lib.pf_gdn_exec_static(1, 1, 1, 1, 1, None, 1, None, 8, 16, 4096, 64, 128, 128,
                                _hip.PF_DTYPE_BF16, 0.1, None)
    assert st == _hip.PF_ERR_SCRATCH and "static scratch" in _hip.status_text(st)
    st = lib.pf_gdn_exec_static(1, 1, 1, 1, 1, None, 1, None, 1, 1, 100, 64, 128, 128,
                                _hip.PF_DTYPE_BF16, 0.1, None)
    assert st == _hip.PF_ERR_ARG                                         # T % C != 0
    st = lib.pf_gdn_exec_static(None, 1, 1, 1, 1, None, 1, None, 1, 1, 128, 64, 128, 128,
                                _hip.PF_DTYPE_BF16, 0.1, None)
    assert st == _hip.PF_ERR_ARG                                         # q missing


def test_ops_validate_on_host():
    torch = pytest.importorskip("torch")
    from pto_fuser_amd import gdn_chunk_forward, kkt_inverse, tri_inv
    q = torch.zeros(1, 1, 64, 128)
    with pytest.raises(ValueError, match="HIP device"):
        gdn_chunk_forward(q, q, q, torch.zeros(1, 1, 64))
    with pytest.raises(ValueError, match="multiple of the chunk"):
        gdn_chunk_forward(torch.zeros(1, 1, 65, 128), q, q, torch.zeros(1, 1, 65))
    with pytest.raises(ValueError, match="unsupported shape"):
        gdn_chunk_forward(torch.zeros(1, 1, 64, 64), q, q, torch.zeros(1, 1, 64))
    with pytest.raises(ValueError):
        tri_inv(torch.zeros(2, 64, 32))
    with pytest.raises(ValueError):
        kkt_inverse(torch.zeros(64, 128), None, torch.zeros(64), chunk_size=32)
    from pto_fuser_amd import kda_chunk_forward
    qb = torch.zeros(1, 1, 128, 128, dtype=torch.bfloat16)
    gk = torch.zeros(1, 1, 128, 128)
    with pytest.raises(ValueError, match="HIP device"):
        kda_chunk_forward(qb, qb, qb, torch.zeros(1, 1, 128), gk)
    with pytest.raises(ValueError, match="bfloat16 or float32"):
        kda_chunk_forward(qb.half(), qb.half(), qb.half(), torch.zeros(1, 1, 128), gk)
    with pytest.raises(ValueError, match="multiple of the chunk size"):
        kda_chunk_forward(qb[:, :, :96], qb[:, :, :96], qb[:, :, :96], torch.zeros(1, 1, 96), gk[:, :, :96])
